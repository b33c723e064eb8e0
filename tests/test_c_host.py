"""The library from a C host (tests/c_driver.c: the public header, rq_* calls only, no Python or torch in the process):
it links on the CPU, and on the GPU its prefill + greedy decode logits equal the oracle's bit for bit."""
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_DIR = os.path.join(ROOT, "gwenedeg_amd", "lib")


def _build(tmp):
    exe = os.path.join(tmp, "c_driver")
    cmd = ["gcc", "-O2", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "include"),
           os.path.join(ROOT, "tests", "c_driver.c"), "-L", LIB_DIR, "-lgwenedeg_amd", f"-Wl,-rpath,{LIB_DIR}", "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


def test_c_host_links(tmp_path):
    exe = _build(str(tmp_path))
    assert os.access(exe, os.X_OK)


@pytest.mark.gpu
@pytest.mark.parametrize("shape", ["tiny", "tiny_kq"])
def test_c_host_matches_oracle(tmp_path, synth_models, shape):
    from oracle import oracle as orc
    exe = _build(str(tmp_path))
    path = synth_models(shape)
    ids = np.random.default_rng(5).integers(0, 512, 24).astype(np.int32)
    ids_path, out_path = str(tmp_path / "ids.bin"), str(tmp_path / "lg.bin")
    ids.tofile(ids_path)
    steps = 8
    r = subprocess.run([exe, path, ids_path, str(steps), out_path], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    om = orc.Model(path, cap=256)
    lg = np.fromfile(out_path, np.float32).reshape(steps + 1, om.vocab)
    s = om.seq()
    for t in ids[:-1]:
        s.forward(int(t), logits=False)
    ref = s.forward(int(ids[-1]))
    toks = []
    for i in range(steps + 1):
        assert np.array_equal(lg[i].view(np.uint32), ref.view(np.uint32)), f"row {i}: max diff {np.abs(lg[i] - ref).max()}"
        tok = int(np.argmax(ref))
        toks.append(tok)
        if i < steps:
            ref = s.forward(tok)
    assert r.stdout.split()[1:2 + steps] == [str(t) for t in toks]
