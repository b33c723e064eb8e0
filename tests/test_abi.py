"""The C-ABI library (CPU-side checks, no device calls): it loads, and it exports every function include/*.h declares."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = set()
    for fn in os.listdir(os.path.join(ROOT, "include")):
        if fn.endswith(".h"):
            src = open(os.path.join(ROOT, "include", fn)).read()
            src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
            for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b((?:rq|gw|ctx)_\w+)\s*\(", src, flags=re.M):
                names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    import gwenedeg_amd as gw
    lib = ctypes.CDLL(gw.LIB_PATH)
    names = declared_functions()
    assert len(names) > 40
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_python_binding_covers_the_passes():
    import gwenedeg_amd as gw
    for n in ("rq_model_load", "rq_seq_new", "rq_ctx_new", "rq_decode", "rq_prefill", "rq_forward_batch", "gw_q8_matmul"):
        assert n in gw.EXPORTED


def _offsets(header_dir, tmp):
    """sizes and field offsets of RqModelOpts / RqModelInfo / RqSegment / RqSeqMem / RqModelMem as gcc lays them out
    from a header"""
    import subprocess
    src = os.path.join(tmp, "off.c")
    hdr = "gwenedeg_gpu.h" if os.path.exists(os.path.join(header_dir, "gwenedeg_gpu.h")) else "runq.h"
    fields = {"RqModelOpts": ["ctx_len", "no_tokenizer", "mem", "kv_bits", "repack"],
              "RqModelInfo": ["vocab_size", "warning", "chat", "rope_theta", "linear_layers", "fingerprint"],
              "RqSegment": ["seq", "tokens", "n", "logits", "hidden", "h_in"],
              "RqSeqMem": ["kv", "state", "checkpoints", "total"],
              "RqModelMem": ["weights", "runtime", "seq", "total", "budget", "budget_src", "read"],
              "RqRepackInfo": ["available", "n", "t", "weights", "extra"],
              "RqMtpOpts": ["vocab", "mem"],
              "RqSeqFile": ["len", "kv_type", "linear", "n_ck", "ck", "bytes"]}
    lines = [f'#include "{hdr}"', "#include <stdio.h>", "#include <stddef.h>", "int main(void) {"]
    for t, fs in fields.items():
        lines.append(f'printf("{t} %zu\\n", sizeof({t}));')
        lines += [f'printf("{t}.{f} %zu\\n", offsetof({t}, {f}));' for f in fs]
    lines.append("return 0; }")
    open(src, "w").write("\n".join(lines))
    exe = os.path.join(tmp, "off")
    subprocess.run(["gcc", "-I", header_dir, src, "-o", exe], check=True)
    out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout
    return dict(line.rsplit(" ", 1) for line in out.strip().splitlines())


def test_struct_layouts_match_the_header(tmp_path):
    """the Python mirror has the C header's layout (field order and widths of runq.h:63-81, :132-146, :364-374)"""
    import gwenedeg_amd as gw
    c = _offsets(os.path.join(ROOT, "include"), str(tmp_path))
    for name, st in (("RqModelOpts", gw.RqModelOpts), ("RqModelInfo", gw.RqModelInfo), ("RqSegment", gw.RqSegment)):
        assert int(c[name]) == ctypes.sizeof(st), name
        for key, v in c.items():
            if key.startswith(name + "."):
                assert int(v) == getattr(st, key.split(".")[1]).offset, key


def test_header_layouts_match_runq_h(tmp_path):
    """include/gwenedeg_gpu.h against the reference's own runq.h (where the reference tree exists: this container)"""
    import pytest
    ref = "/root/reference/src"
    if not os.path.exists(os.path.join(ref, "runq.h")):
        pytest.skip("reference tree not present")
    a = _offsets(os.path.join(ROOT, "include"), str(tmp_path))
    b = _offsets(ref, str(tmp_path))
    assert a == b


def test_cpu_only_paths_fail_cleanly():
    """no device here: loading a model reports an error code and text, never crashes"""
    import gwenedeg_amd as gw
    try:
        import torch
        if torch.cuda.is_available():
            return
    except ImportError:
        pass
    try:
        gw.Model("/nonexistent.gguf")
    except gw.RqError as e:
        assert e.code == gw.RQ_ERR_LOAD
    else:
        raise AssertionError("expected an error")


def test_one_hip_runtime_per_process():
    """importing the package before torch still leaves one HIP runtime in the process (two copies of libamdhip64, the
    system's and torch's, cannot both see the device)"""
    import subprocess
    import sys
    code = ("import sys; sys.path.insert(0, %r)\n"
            "import gwenedeg_amd\n"
            "import torch\n"
            "libs = {l.split()[-1] for l in open('/proc/self/maps') if 'libamdhip64' in l}\n"
            "print(len(libs), sorted(libs))\n") % ROOT
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr[-2000:]
    n = int(out.stdout.split()[0])
    assert n == 1, out.stdout


# What each of the reference's host modules still needs once libgwenedeg_amd.so replaces its model.o, gguf.o, forward.o
# and seqfile.o (gguf.o is kept for the tokenizer): nothing. model.c's chat templates (rq_chat_name, rq_chat_check,
# chat_gen_suffix) and its load error exit (load_fail) are the library's too (gw_host.c); everything else on the
# reference's runq.h / internal.h surface those modules call resolves to the library.
HOST_NEEDS = {
    "sampler": set(), "threads": set(), "spec": set(), "constrain": set(), "http": set(), "json": set(),
    "chat": set(), "tokenizer": set(), "engine": set(), "cli": set(), "serve": set(), "tools": set(),
}


def test_tokenizer_entry_points_are_weak():
    """the library reaches the host's tokenizer.o / gguf.o only through weak references (a program without them, e.g.
    the Python binding, loads the library and gets models without a tokenizer), and it exports the model.c host
    helpers those objects call"""
    import subprocess
    lib = os.path.join(ROOT, "gwenedeg_amd", "lib", "libgwenedeg_amd.so")
    out = subprocess.run(["nm", "-D", lib], capture_output=True, text=True, check=True).stdout
    kind = {ln.split()[-1]: ln.split()[-2] for ln in out.splitlines() if ln.strip()}
    for f in ("gguf_parse", "gguf_chat_variant", "gguf_sampling", "build_tokenizer_gguf", "free_tokenizer"):
        assert kind.get(f) == "w", (f, kind.get(f))
    for f in ("load_fail", "chat_gen_suffix", "rq_chat_name", "rq_chat_check"):
        assert kind.get(f) == "T", (f, kind.get(f))


def test_reference_host_modules_link():
    """the reference's host modules (compiled from its sources by oracle/Makefile into oracle/_ref) against the
    library's exports: the unresolved symbols of the reference's own namespace are exactly HOST_NEEDS"""
    import subprocess
    ref = os.path.join(ROOT, "oracle", "_ref")
    objs = {m: os.path.join(ref, m + ".o") for m in list(HOST_NEEDS) + ["gguf"]}
    if not all(os.path.exists(p) for p in objs.values()):
        pytest.skip("the reference's host objects are not built (oracle/Makefile needs the reference tree)")
    def syms(args, path):
        out = subprocess.run(["nm", *args, path], capture_output=True, text=True, check=True).stdout
        return {ln.split()[-1] for ln in out.splitlines() if ln.strip()}
    provided = syms(["-D", "--defined-only"], os.path.join(ROOT, "gwenedeg_amd", "lib", "libgwenedeg_amd.so"))
    for p in objs.values():
        provided |= syms(["--defined-only"], p)
    ours = ("rq_", "gguf", "load_", "chat_", "fw_", "seq_", "ctx_", "embed_", "forward_", "mtp_", "kq_", "q8p_")
    for mod, need in HOST_NEEDS.items():
        und = {s for s in syms(["-u"], objs[mod]) if s.startswith(ours)} - provided
        assert und == need, f"{mod}.o: unresolved {sorted(und)}, documented {sorted(need)}"


# The RqModel / RqSeq fields the reference's host modules read directly (sampler.c:321-331, spec.c:32-54 / :219 /
# :271-429, chat.c:38-357, tokenizer.c:794-827: the Tokenizer the host's tokenizer.o builds in place): their offsets and sizes in the reference's internal.h as gcc lays it out
# on x86-64, which the library's structs keep (the reference's field names; the library's own fields follow)
REF_FIELDS = {
    "RqModel": {"config": (0, 48), "config.dim": (8, 4), "config.vocab_size": (28, 4), "config.seq_len": (32, 4),
                "config.shared_classifier": (40, 4), "config.group_size": (44, 4), "fp": (1752, 8),
                "tok": (280, 1368), "tok.vocab_size": (304, 4), "tok.bos_token_id": (312, 4),
                "tok.eos_token_id": (316, 4), "tok.n_added": (1384, 4), "tok.marks35": (1644, 4),
                "has_weights": (1760, 4), "has_tok": (1764, 4), "is_gguf": (1768, 4), "warning": (1776, 256),
                "hy.on": (2080, 4),
                "chat": (2684, 4), "samp_temp": (2768, 4), "samp_topp": (2772, 4), "samp_topk": (2776, 4),
                "samp_set": (2780, 4), "user_tmpl": (2784, 2048), "sys_tmpl": (4832, 2048),
                "tmpl_missing": (6880, 2176), "mtp_of": (9056, 8)},
    "RqSeq": {"m": (0, 8), "cap": (8, 4), "kv_len": (12, 4), "att_nb": (16, 4), "kvt": (20, 4), "len": (80, 4),
              "hwm": (84, 4), "tokens": (96, 8), "nck": (120, 4), "rng": (1808, 8), "hvalid": (1816, 4),
              "hpos": (1820, 4), "hprev": (1824, 8)},
}
REF_SIZES = {"RqModel": 9208, "RqSeq": 1832}
# the library's names for the fields it keeps under its own name (the reference's nested Hybrid.on, the fingerprint)
OURS = {"hy.on": "hy_on", "fp": "ref_fp"}


def _field_offsets(tmp, include_dirs, header, names):
    import subprocess
    lines = [f'#include "{header}"', "#include <stdio.h>", "#include <stddef.h>", "int main(void) {"]
    for t, fs in REF_FIELDS.items():
        for f in fs:
            g = names.get(f, f)
            lines.append(f'printf("{t}.{f} %zu %zu\\n", offsetof(struct {t}, {g}), sizeof(((struct {t} *)0)->{g}));')
    lines.append("return 0; }")
    src = os.path.join(tmp, "fo.c")
    open(src, "w").write("\n".join(lines))
    exe = os.path.join(tmp, "fo")
    cmd = ["gcc", "-D__HIP_PLATFORM_AMD__", *sum((["-I", d] for d in include_dirs), []), src, "-o", exe]
    subprocess.run(cmd, check=True, capture_output=True)
    out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout
    return {k: (int(a), int(b)) for k, a, b in (ln.split() for ln in out.strip().splitlines())}


def test_internal_layouts_keep_the_reference_offsets(tmp_path):
    """the library's RqModel / RqSeq keep, at the reference's offsets and widths, every field the reference's host
    modules read (so its sampler.o, spec.o and chat.o run unmodified against the library): against the committed
    table, and against the reference's own internal.h compiled here where the reference tree exists"""
    inc = [os.path.join(ROOT, "gwenedeg_amd", "csrc"), os.path.join(ROOT, "include"), "/opt/rocm/include"]
    if not os.path.exists("/opt/rocm/include/hip/hip_runtime_api.h"):
        pytest.skip("ROCm headers not present")
    ours = _field_offsets(str(tmp_path), inc, "gw_internal.h", OURS)
    table = {f"{t}.{f}": v for t, fs in REF_FIELDS.items() for f, v in fs.items()}
    assert ours == table
    ref = "/root/reference/src"
    if os.path.exists(os.path.join(ref, "internal.h")):
        theirs = _field_offsets(str(tmp_path), [ref], "internal.h", {})
        assert theirs == table
