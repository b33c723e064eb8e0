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
# and seqfile.o (and gguf.o is kept for the tokenizer): the functions outside the hot path that stay with the host
# (model.c's chat templates and load error helper). Everything else on the reference's
# runq.h / internal.h surface those modules call resolves to the library.
HOST_NEEDS = {
    "sampler": set(), "threads": set(), "spec": set(), "constrain": set(), "http": set(), "json": set(),
    "chat": {"chat_gen_suffix"},
    "tokenizer": {"load_fail"},
    "engine": set(),
    "cli": {"rq_chat_check", "rq_chat_name"},
    "serve": {"rq_chat_check", "rq_chat_name"},
    "tools": {"rq_chat_name"},
}


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
