"""Lazy device KV memory through the rq_* C ABI: a sequence reserves the address range of its capacity and maps device
memory in chunks per layer and half (K / V) as positions are first written; rq_seq_release unmaps the chunks past
max(keep, len) and lowers the high-water mark that rq_seq_resident reports (runq.h:270-277, forward.c:455-510). The
checks follow the reference's own (api_test.c:908-1002, "giving memory back"): resident == rq_seq_kv_bytes of the
high-water mark, the device memory given back matches what was unmapped, and the rows after a release equal a fresh
sequence's on the same prefix bit for bit. The fresh sequences are allocated whole (gw_seq_lazy(0)), so every
comparison is also lazy against whole. The model: 36 layers of the Qwen3-8B attention shape (8 KV heads of 128), so a
sequence at the 40,960-position capacity would hold 5.4 GiB of cache, with a small width (dim 512) so the weights
and the passes stay small."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

NONE, LAST, ALL = 0, 1, 2
L, NKV, HD, CAP = 36, 8, 128, 40960
BLOCK = 256 * NKV * HD * 2  # (one 256-position block of one layer's K or V, f16)


@pytest.fixture(scope="module")
def gw():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    import gwenedeg_amd
    return gwenedeg_amd


@pytest.fixture(scope="module")
def deep(gw, tmp_path_factory):
    from gwenedeg_amd import synth
    path = str(tmp_path_factory.mktemp("deep") / "deep36.gguf")
    synth.write_gguf(path, dict(dim=512, hidden=1024, n_layers=L, n_heads=32, n_kv_heads=NKV, head_dim=HD, vocab=2048,
                                ctx_len=CAP, tied=1, type_default=synth.Q8_0), seed=5)
    m = gw.Model(path)
    yield m
    m.close()


def _ids(vocab, n, seed):
    return np.random.default_rng(seed).integers(0, vocab, n).astype(np.int32)


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _whole(gw, m, cap):
    """a sequence allocated whole (the reference for the lazy ones)"""
    prev = gw.lib.gw_seq_lazy(0)
    try:
        return m.seq(cap)
    finally:
        gw.lib.gw_seq_lazy(prev)


def _chunk(gw, m):
    """the mapping chunk: the device bytes of a one-position sequence / (2 halves x L layers)"""
    s = m.seq(CAP)
    s.fill_synthetic(1, seed=1)
    b = s.device_bytes()
    s.close()
    assert b % (2 * L) == 0
    ch = b // (2 * L)
    assert ch >= BLOCK and ch % (2 << 20) == 0, ch
    return ch


def _mapped(n, ch):
    """device bytes of a lazy sequence whose highest written position is n - 1"""
    nb = (n + 255) // 256
    return 2 * L * ((nb * BLOCK + ch - 1) // ch) * ch


def _free():
    import torch
    return torch.cuda.mem_get_info()[0]


def test_release_gives_memory_back_and_continues_bitwise(gw, deep):
    """api_test.c:908-1002: a sequence prefilled to N positions, cut to keep = 768, 300, 0 and released: resident ==
    kv_bytes(keep), the device bytes drop to keep's chunks (and the device's free memory rises by what went), and the
    next rows (4 in a prefill, then a decode step) == a fresh sequence's on the same prefix, bit for bit"""
    m = deep
    assert gw.lib.gw_seq_lazy(-1) == 1
    c = m.ctx(max_batch=512)
    ch = _chunk(gw, m)
    N, R = 4608, 5  # (18 blocks: 9 MiB per layer and half)
    u = _ids(m.vocab, N + R, 3)
    s = m.seq(CAP)
    assert s.capacity == CAP and s.device_bytes() == 0
    r = s.resident()
    assert r.kv == s.kv_bytes(0) == CAP * 4 and r.total == r.kv and r.state == 0 and r.checkpoints == 0
    assert s.kv_bytes(1) == s.kv_bytes(256) < s.kv_bytes(257) and s.kv_bytes(CAP + 9) == s.kv_bytes(CAP)
    assert gw.lib.rq_seq_release(s._h, -1) == gw.RQ_ERR_ARG and gw.lib.rq_seq_release(s._h, 0) == 0
    f = _whole(gw, m, N + R + 16)
    assert f.device_bytes() == 2 * L * ((N + R + 16 + 255) // 256) * BLOCK
    for P in (768, 300, 0):
        f.reset()
        if P:
            c.prefill(f, u[:P], mode=NONE)
        ref = c.prefill(f, u[P:P + R - 1], mode=ALL)
        ref_last = c.decode(f, int(u[P + R - 1]))
        s.reset()
        c.prefill(s, u[:N], mode=NONE)
        assert s.device_bytes() == _mapped(N, ch)
        if P:
            s.truncate(P)
        else:
            s.reset()
        r0 = s.resident()
        assert r0.kv == s.kv_bytes(N)
        f0 = _free()
        s.release(P)
        f1 = _free()
        r1 = s.resident()
        assert r1.kv == s.kv_bytes(P) and r1.total == r1.kv and len(s) == P
        assert s.device_bytes() == (_mapped(P, ch) if P else 0)
        want = _mapped(N, ch) - s.device_bytes()
        assert want - (16 << 20) <= f1 - f0 <= want + (64 << 20), (P, f1 - f0, want)
        out = c.prefill(s, u[P:P + R - 1], mode=ALL)
        last = c.decode(s, int(u[P + R - 1]))
        assert np.array_equal(_bits(out), _bits(ref)) and np.array_equal(_bits(last), _bits(ref_last)), f"keep {P}"
    # keep below the length: nothing past the length goes (len R, one block)
    r0 = s.resident()
    s.release(0)
    r1 = s.resident()
    assert len(s) == R and r1.kv == r0.kv == s.kv_bytes(R) and s.device_bytes() == _mapped(R, ch)
    s.close()
    f.close()
    c.close()


def test_many_long_sequences_hold_what_they_use(gw, deep):
    """64 sequences of the 40,960-position capacity (whole, their caches would exceed the device's memory): creating
    them maps nothing; filled to 300 .. 4,143 positions each holds its chunks; one batched pass of a row per sequence
    equals whole-allocated sequences alone; half are then cut to 256 positions and released, and the next pass again
    equals the whole-allocated ones (continuing, or cut the same way); freeing them gives the memory back"""
    import ctypes
    import torch
    m = deep
    nseq = 64
    c = m.ctx(max_batch=nseq)
    ch = _chunk(gw, m)
    sm = gw.RqSeqMem()
    assert gw.lib.rq_seq_mem(ctypes.c_void_p(m._h), CAP, gw.RQ_KV_F16, ctypes.byref(sm)) == 0
    total = torch.cuda.mem_get_info()[1]
    assert nseq * sm.kv > total, "the case must not fit when allocated whole"
    f0 = _free()
    seqs = [m.seq(CAP) for _ in range(nseq)]
    f1 = _free()
    assert f0 - f1 < (64 << 20) and all(s.device_bytes() == 0 for s in seqs)
    lens = [300 + 61 * i for i in range(nseq)]
    for i, s in enumerate(seqs):
        s.fill_synthetic(lens[i], seed=100 + i)
        assert s.device_bytes() == _mapped(lens[i], ch)
        assert s.resident().kv == s.kv_bytes(lens[i])
    held = sum(s.device_bytes() for s in seqs)
    f2 = _free()
    assert abs((f1 - f2) - held) <= (64 << 20), (f1 - f2, held)
    tok = _ids(m.vocab, 2 * nseq, 7)
    out1, _ = c.forward_batch([gw.Segment(s, [int(tok[i])], ALL) for i, s in enumerate(seqs)])
    f2 = _free()  # (after the context's own buffers of a 64-row pass)
    cut = [i for i in range(nseq) if i % 2 == 0]
    for i in cut:
        seqs[i].truncate(256)
        seqs[i].release(256)
        assert seqs[i].device_bytes() == _mapped(256, ch) and seqs[i].resident().kv == seqs[i].kv_bytes(256)
    f3 = _free()
    gone = sum(_mapped(lens[i] + 1, ch) - _mapped(256, ch) for i in cut)
    assert abs((f3 - f2) - gone) <= (64 << 20), (f3 - f2, gone)
    out2, _ = c.forward_batch([gw.Segment(s, [int(tok[nseq + i])], ALL) for i, s in enumerate(seqs)])
    for i in (0, 1, 21, 42, 63):
        f = _whole(gw, m, lens[i] + 8)
        f.fill_synthetic(lens[i], seed=100 + i)
        a = c.decode(f, int(tok[i]))
        assert np.array_equal(_bits(a), _bits(out1[i])), f"sequence {i}, first pass"
        if i in cut:
            f.truncate(256)
        b = c.decode(f, int(tok[nseq + i]))
        assert np.array_equal(_bits(b), _bits(out2[i])), f"sequence {i}, after the release"
        f.close()
    for s in seqs:
        s.close()
    c.close()
    f4 = _free()
    assert f4 >= f1 - (16 << 20), (f4, f1)  # (the sequences' memory back, the context's too)


def test_greedy_decode_across_chunk_boundaries(gw, deep):
    """gw_decode_greedy maps the chunks its steps reach before it enqueues them: 24 steps from position 1,012 (past the
    first 2 MiB chunk of every layer at 1,024) and from 4,090 give the tokens and the next logits of a whole-allocated
    sequence"""
    m = deep
    c = m.ctx(max_batch=1)
    ch = _chunk(gw, m)
    for n0 in (1012, 4090):
        s, f = m.seq(CAP), _whole(gw, m, n0 + 64)
        s.fill_synthetic(n0, seed=11)
        f.fill_synthetic(n0, seed=11)
        assert s.device_bytes() == _mapped(n0, ch)
        a, b = c.decode_greedy(s, 17, 24), c.decode_greedy(f, 17, 24)
        assert np.array_equal(a, b), n0
        assert s.device_bytes() == _mapped(n0 + 24, ch) > _mapped(n0, ch)
        x, y = c.decode(s, int(a[-1])), c.decode(f, int(b[-1]))
        assert np.array_equal(_bits(x), _bits(y)), n0
        s.close()
        f.close()
    c.close()
