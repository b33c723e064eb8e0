"""The reference's own host modules against the library (tests/host_modules.c): its sampler.o, threads.o, spec.o,
chat.o, tokenizer.o and gguf.o, compiled unmodified from its sources (oracle/_ref), read this library's RqModel / RqSeq
fields at their offsets and drive its passes. The same host program linked with the reference's whole CPU library must
print the same: sampled tokens and RNG states (sampler.c:307-368), rq_generate's tokens and logits hashes
(chat.c:385-415), the speculative loop with prompt lookup (spec.c:404-600: multi-row verify passes, rollbacks) giving
rq_generate's output, and, on a model file with a tokenizer, the tokenizer and chat templates rq_model_load builds
(model.c:1010-1016): token ids, token bytes, rendered conversations and a chat reply generated and detokenized."""
import json
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_DIR = os.path.join(ROOT, "gwenedeg_amd", "lib")
REF = os.path.join(ROOT, "oracle", "_ref")
SRC = os.path.join(ROOT, "tests", "host_modules.c")
HOST = ["sampler", "threads", "spec", "chat", "tokenizer", "gguf"]                         # kept on the host
REFLIB = ["model", "gguf", "forward", "tokenizer", "sampler", "chat", "threads", "spec", "seqfile"]  # the reference's


def _objs(names):
    p = [os.path.join(REF, n + ".o") for n in names]
    if not all(os.path.exists(x) for x in p):
        pytest.skip("the reference's objects are not built (oracle/Makefile needs the reference tree)")
    return p


def _build(tmp, which):
    exe = os.path.join(tmp, f"host_modules_{which}")
    if which == "ours":
        cmd = ["gcc", "-O2", "-I", os.path.join(ROOT, "include"), SRC, *_objs(HOST), "-L", LIB_DIR,
               "-lgwenedeg_amd", f"-Wl,-rpath,{LIB_DIR}", "-fopenmp", "-lm", "-lpthread", "-o", exe]
    else:
        cmd = ["gcc", "-O2", "-I", os.path.join(ROOT, "include"), SRC, *_objs(REFLIB), "-fopenmp", "-lm", "-lpthread",
               "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    return exe


def test_host_api_declarations_match_runq_h(tmp_path):
    """the host-module API types host_modules.c declares have runq.h's layouts (runq.h:376-653), and the program links
    against the library with the reference's host objects"""
    exe = _build(str(tmp_path), "ours")
    ours = subprocess.run([exe, "--layouts"], capture_output=True, text=True, check=True).stdout
    ref = "/root/reference/src/runq.h"
    if not os.path.exists(ref):
        pytest.skip("reference tree not present")
    src = open(SRC).read()
    body = src[src.index("static void layouts(void) {"):src.index("int main(")]
    prog = os.path.join(str(tmp_path), "lay.c")
    open(prog, "w").write('#include "runq.h"\n#include <stdio.h>\n#include <stddef.h>\n' + body +
                          "int main(void) { layouts(); return 0; }\n")
    lay = os.path.join(str(tmp_path), "lay")
    subprocess.run(["gcc", "-I", os.path.dirname(ref), prog, "-o", lay], check=True)
    theirs = subprocess.run([lay], capture_output=True, text=True, check=True).stdout
    assert ours == theirs


@pytest.mark.gpu
@pytest.mark.parametrize("tok", [False, True])
def test_reference_host_modules_run_unmodified(tmp_path, tok):
    """the same host program, linked with the library plus the reference's host objects and with the reference's whole
    CPU library, on a Qwen3-0.6B-shaped model (2 layers, full vocabulary): identical output, and the speculative loop's
    lookup rounds actually verified guesses. tok: the file carries a tokenizer block and both load it (no_tokenizer 0):
    the library builds it through the host's tokenizer.o, and the text side prints the same"""
    import torch
    assert torch.cuda.is_available()
    from gwenedeg_amd import synth
    import gwenedeg_amd as gw
    d = dict(synth.SHAPES["qwen3_0_6b"])
    d["n_layers"] = 2
    d["tokenizer"] = int(tok)
    path = synth.write_gguf(str(tmp_path / "m.gguf"), d, seed=21)
    m = gw.Model(path, ctx_len=512)
    if gw.exact_mode() & 3 != 3:
        pytest.skip("this host does not provide the reference's float operations (AVX-512)")
    del m
    base = np.random.default_rng(21).integers(0, d["vocab"], 16).astype(np.int32)
    ids = np.concatenate([base, base, base])  # (a repeated prompt: the lookup finds matches)
    ids_path = str(tmp_path / "ids.bin")
    ids.tofile(ids_path)
    outs = {}
    for which in ("ours", "ref"):
        exe = _build(str(tmp_path), which)
        env = dict(os.environ, OMP_NUM_THREADS=str(min(16, len(os.sched_getaffinity(0)))))
        r = subprocess.run([exe, path, ids_path] + (["--tok"] if tok else []), capture_output=True, text=True,
                           timeout=600, env=env)
        assert r.returncode == 0, f"{which}: {r.stderr[-3000:]}"
        outs[which] = json.loads(r.stdout.strip().splitlines()[-1])
    a, b = outs["ours"], outs["ref"]
    assert a["sample"] == b["sample"]
    assert a["sample_batch"] == b["sample_batch"] and a["batch_rng"] == b["batch_rng"]
    assert len({t for smp in a["sample"][1:] for t in smp["tokens"]}) > 4  # (the draws differ)
    for ga, gb in zip(a["generate"], b["generate"]):
        assert ga == gb
        assert ga["spec"]["same_tokens"] == 1 and ga["spec"]["logits"] == ga["logits"]
    drafted = sum(g["spec"]["lookup_drafted"] for g in a["generate"])
    accepted = sum(g["spec"]["lookup_accepted"] for g in a["generate"])
    assert accepted > 0 and drafted > accepted  # (guesses accepted, and refused ones rolled back)
    if not tok:
        assert a["spec_check"] == b["spec_check"] == -4  # RQ_ERR_STATE: a draft model needs its tokenizer
        assert "tok" not in a
        return
    assert a["spec_check"] == b["spec_check"] == 0
    assert a["tok"] == b["tok"]
    t = a["tok"]
    assert t["bos"] >= 0 and t["eos"] >= 0 and t["chat"] == "qwen3" and t["check"] == [0, 0]
    assert all(x["rc"] == 0 and x["round_trip"] == 1 for x in t["tokenize"])
    assert all(x["rc"] == 0 and len(x["ids"]) > 20 for x in t["render"])
    assert t["reply"]["rc"] == 0 and t["reply"]["n_gen"] >= 1


def test_tokenizer_only_matches_reference(tmp_path):
    """RqModelOpts.tokenizer_only (model.c:893-922), on the CPU: the library builds the tokenizer through the host's
    tokenizer.o / gguf.o without touching a device, and the host program prints what it prints linked with the
    reference's whole library: bos / eos, the chat variant, token ids and bytes, rendered conversations; a context or a
    sequence of such a model is refused (RQ_ERR_STATE). A file without a tokenizer block fails with the reference's
    message"""
    from gwenedeg_amd import synth
    d = dict(synth.SHAPES["tiny_gqa4"])
    outs = {}
    for name, tok in (("tok", 1), ("plain", 0)):
        d["tokenizer"] = tok
        path = synth.write_gguf(str(tmp_path / f"{name}.gguf"), d, seed=5)
        for which in ("ours", "ref"):
            exe = _build(str(tmp_path), which)
            r = subprocess.run([exe, path, "--tokenizer-only"], capture_output=True, text=True, timeout=300)
            assert r.returncode == 0, f"{which}: {r.stderr[-3000:]}"
            outs[(name, which)] = json.loads(r.stdout.strip().splitlines()[-1])
    a, b = outs[("tok", "ours")], outs[("tok", "ref")]
    assert a == b
    assert a["ctx"] == [0, -4] and a["seq"] == [0, -4]
    assert all(x["rc"] == 0 and x["round_trip"] == 1 for x in a["tok"]["tokenize"])
    assert outs[("plain", "ours")] == outs[("plain", "ref")]
    assert "tokenizer.ggml.model must be gpt2" in outs[("plain", "ours")]["load"]
