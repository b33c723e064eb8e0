"""gw_ctx_topk_noalloc (the top-k entry point that allocates nothing: its candidates and device outputs live in a static
per-device array) through the C ABI, against gw_ctx_topk on the same logits rows: two calls in a row on the full
Qwen3 vocabulary, the second with fewer rows and a smaller k, each equal to gw_ctx_topk's result; more rows than the
array holds are refused before any launch."""
import ctypes
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_topk_noalloc_equals_topk(tmp_path):
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    import gwenedeg_amd as gw
    from gwenedeg_amd import synth
    d = dict(synth.SHAPES["tiny"])
    d["vocab"] = 151936
    path = synth.write_gguf(os.path.join(str(tmp_path), "na.gguf"), d, seed=5)
    m = gw.Model(path, ctx_len=256)
    c = m.ctx(max_batch=32)
    seqs = [m.seq(256) for _ in range(16)]
    rng = np.random.default_rng(5)
    segs = [gw.Segment(sq, [int(t) for t in rng.integers(0, m.vocab, 1 + i % 3)], gw.RQ_LOGITS_LAST) for i, sq in enumerate(seqs)]
    c.forward_batch(segs)

    def noalloc(n, k):
        v, ix = np.zeros((n, k), np.float32), np.zeros((n, k), np.int32)
        r = gw.lib.gw_ctx_topk_noalloc(c._h, n, k, v.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                       ix.ctypes.data_as(ctypes.POINTER(ctypes.c_int)))
        return r, v, ix

    for n, k in ((16, 64), (3, 7)):  # (the second call smaller: fewer rows, smaller k, the same array)
        r, v, ix = noalloc(n, k)
        assert r == gw.RQ_OK, gw.lib.rq_ctx_error(c._h)
        rv, ri = c.topk(n, k)
        assert np.array_equal(ix, ri), (n, k)
        assert np.array_equal(v.view(np.uint32), rv.view(np.uint32)), (n, k)
    c2 = m.ctx(max_batch=32)
    c2.forward_batch([gw.Segment(sq, [1], gw.RQ_LOGITS_LAST) for sq in (m.seq(256) for _ in range(17))])
    v, ix = np.zeros((17, 4), np.float32), np.zeros((17, 4), np.int32)
    r = gw.lib.gw_ctx_topk_noalloc(c2._h, 17, 4, v.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                   ix.ctypes.data_as(ctypes.POINTER(ctypes.c_int)))
    assert r == gw.RQ_ERR_ARG and b"at most 16" in gw.lib.rq_ctx_error(c2._h)
