"""Whole-model parity on the GPU through the rq_* C ABI: the device forward passes against the oracle's forward pass
(or_forward_token) on seeded synthetic models, bit for bit (the logits; the KV cache through the logits of every later position), plus the reference's own invariants
(batched == sequential, chunking, sequence copy / truncate, long context past one attention block)."""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gw():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    import gwenedeg_amd
    return gwenedeg_amd


def _ids(vocab, n, seed):
    return np.random.default_rng(seed).integers(0, vocab, n).astype(np.int32)


def _bits_equal(a, b):
    return np.array_equal(np.ascontiguousarray(a, np.float32).view(np.uint32), np.ascontiguousarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("shape", ["tiny", "tiny_gqa4", "tiny_kq", "tiny_q5k", "tiny_q3k", "tiny_hd64", "tiny_hd32"])
def test_prefill_decode_bitexact_vs_oracle(gw, synth_models, shape):
    from oracle import oracle as orc
    path = synth_models(shape)
    m = gw.Model(path, ctx_len=1024)
    om = orc.Model(path, cap=1024)
    ids = _ids(m.vocab, 40, 3)
    c = m.ctx(max_batch=16)
    s = m.seq(1024)
    lg_all = c.prefill(s, ids, mode=gw.RQ_LOGITS_ALL)  # chunks of 16 rows
    os_ = om.seq()
    for i, t in enumerate(ids):
        ref = os_.forward(int(t))
        assert _bits_equal(lg_all[i], ref), f"row {i}: max diff {np.abs(lg_all[i] - ref).max()}"
    tok = int(np.argmax(lg_all[-1]))
    for step in range(6):
        lg = c.decode(s, tok)
        ref = os_.forward(tok)
        assert _bits_equal(lg, ref), f"decode step {step}: max diff {np.abs(lg - ref).max()}"
        tok = int(np.argmax(ref))


@pytest.mark.parametrize("kern,tile", [(1, 64), (1, 32), (2, 0), (3, 0), (4, 0), (5, 0), (6, 0), (7, 0), (8, 0)])
def test_prefill_gemm_kernels_bitexact_vs_oracle(gw, synth_models, kern, tile):
    """a 100-row prefill pass through each Q8_0 GEMM (gw_q8_gemm_kernel 1 with 64- or 32-row tiles: k_gemm_q8f; 2, 3:
    k_gemm_q8l of 128 / 64 columns; 4 .. 8: k_gemm_q8t's tiles and stages; 100 rows: 2 row tiles), every row's logits
    against the oracle bit for bit, then decode steps on the cache it wrote"""
    from oracle import oracle as orc
    path = synth_models("tiny")
    m = gw.Model(path, ctx_len=1024)
    om = orc.Model(path, cap=1024)
    ids = _ids(m.vocab, 100, 21)
    c = m.ctx(max_batch=128)
    s = m.seq(1024)
    pk, pt = gw.lib.gw_q8_gemm_kernel(kern), gw.lib.gw_matmul_tile_rows(tile)
    try:
        lg_all = c.prefill(s, ids, mode=gw.RQ_LOGITS_ALL)
    finally:
        gw.lib.gw_q8_gemm_kernel(pk)
        gw.lib.gw_matmul_tile_rows(pt)
    os_ = om.seq()
    for i, t in enumerate(ids):
        ref = os_.forward(int(t))
        assert _bits_equal(lg_all[i], ref), f"row {i}: max diff {np.abs(lg_all[i] - ref).max()}"
    tok = int(np.argmax(lg_all[-1]))
    for step in range(3):
        lg = c.decode(s, tok)
        ref = os_.forward(tok)
        assert _bits_equal(lg, ref), f"decode step {step}"
        tok = int(np.argmax(ref))


@pytest.mark.parametrize("n_prompt", [600, 1100])
def test_long_context_multi_block(gw, synth_models, n_prompt):
    """positions past 256: the attention split into blocks and combined (att_combine), prefill and decode; 600 takes
    the decode combine inside the wo matmul (<= 4 blocks), 1100 the separate combine kernel (5 blocks)"""
    from oracle import oracle as orc
    path = synth_models("tiny")
    m = gw.Model(path, ctx_len=2048)
    om = orc.Model(path, cap=2048)
    ids = _ids(m.vocab, n_prompt, 11)
    c = m.ctx(max_batch=128)
    s = m.seq(2048)
    lg = c.prefill(s, ids, mode=gw.RQ_LOGITS_LAST)
    os_ = om.seq()
    for t in ids[:-1]:
        os_.forward(int(t), logits=False)
    ref = os_.forward(int(ids[-1]))
    assert _bits_equal(lg, ref), f"max diff {np.abs(lg - ref).max()}"
    for tok in (5, 77, 900):
        assert _bits_equal(c.decode(s, tok), os_.forward(tok))


def test_batched_equals_sequential(gw, synth_models):
    """rq_forward_batch over several sequences gives each one the bits it gets alone (runq.h:22-24)"""
    path = synth_models("tiny_gqa4")
    m = gw.Model(path, ctx_len=1024)
    c1, cb = m.ctx(max_batch=1), m.ctx(max_batch=64)
    prompts = [_ids(m.vocab, n, 20 + n) for n in (5, 17, 33)]
    alone = []
    for p in prompts:
        s = m.seq(512)
        rows = [c1.decode(s, int(t)) for t in p]
        alone.append(np.stack(rows))
    seqs = [m.seq(512) for _ in prompts]
    lg, _ = cb.forward_batch([gw.Segment(s, p, gw.RQ_LOGITS_ALL) for s, p in zip(seqs, prompts)])
    o = 0
    for p, a in zip(prompts, alone):
        assert _bits_equal(lg[o:o + len(p)], a)
        o += len(p)
    # then one decode row per sequence, batched, against each alone
    toks = [11, 22, 33]
    lg, _ = cb.forward_batch([gw.Segment(s, [t], gw.RQ_LOGITS_LAST) for s, t in zip(seqs, toks)])
    for i, (p, t) in enumerate(zip(prompts, toks)):
        s = m.seq(512)
        for x in p:
            c1.decode(s, int(x), logits=False)
        assert _bits_equal(lg[i], c1.decode(s, t))


def test_seq_copy_truncate(gw, synth_models):
    path = synth_models("tiny")
    m = gw.Model(path, ctx_len=1024)
    c = m.ctx(max_batch=64)
    ids = _ids(m.vocab, 300, 4)
    a = m.seq(1024)
    c.prefill(a, ids, mode=gw.RQ_LOGITS_NONE)
    b = m.seq(1024)
    b.copy_from(a, 270)
    assert len(b) == 270 and np.array_equal(b.tokens(), ids[:270])
    a.truncate(270)
    la, lb = c.decode(a, 42), c.decode(b, 42)
    assert _bits_equal(la, lb)


def test_errors_validate_before_work(gw, synth_models):
    path = synth_models("tiny")
    m = gw.Model(path, ctx_len=64)
    c = m.ctx(max_batch=8)
    s = m.seq(16)
    with pytest.raises(gw.RqError) as e:
        c.decode(s, m.vocab)
    assert e.value.code == gw.RQ_ERR_ARG and len(s) == 0
    c.prefill(s, _ids(m.vocab, 16, 1), mode=gw.RQ_LOGITS_NONE)
    with pytest.raises(gw.RqError) as e:
        c.decode(s, 1)
    assert e.value.code == gw.RQ_ERR_CONTEXT and len(s) == 16
    c1 = m.ctx(max_batch=1)
    with pytest.raises(gw.RqError) as e:
        c1.forward_batch([gw.Segment(m.seq(16), [1], gw.RQ_LOGITS_LAST)])
    assert e.value.code == gw.RQ_ERR_STATE


def test_device_argmax(gw, synth_models):
    path = synth_models("tiny")
    m = gw.Model(path, ctx_len=256)
    c = m.ctx(max_batch=8)
    s = m.seq(256)
    lg = c.prefill(s, _ids(m.vocab, 9, 2))
    assert int(c.argmax(1)[0]) == int(np.argmax(lg))


@pytest.mark.parametrize("shape,n_prompt,steps", [("tiny", 9, 40), ("tiny_hd64", 250, 20), ("tiny_gqa4", 1000, 40),
                                                  ("tiny_kq", 5, 6)])
def test_decode_greedy_equals_step_by_step(gw, synth_models, shape, n_prompt, steps):
    """gw_decode_greedy (tokens fed on the device, one wait) against gw_decode_argmax step by step and the host argmax
    of rq_decode's logits: the same tokens, the same cache (the logits of a later step agree bit for bit); across
    key-block boundaries (250 + 20 passes position 256, 1000 + 40 passes 1024: the combine past GW_GV_NBMAX blocks);
    a K-quant model takes the step-by-step path"""
    path = synth_models(shape)
    m = gw.Model(path, ctx_len=2048)
    c = m.ctx(max_batch=64, max_ctx=2048)
    ids = _ids(m.vocab, n_prompt, 4)
    s1, s2 = m.seq(2048), m.seq(2048)
    lg = c.prefill(s1, ids)
    c.prefill(s2, ids)
    t0 = int(np.argmax(lg))
    got = c.decode_greedy(s1, t0, steps)
    ref, tok = [], t0
    for _ in range(steps):
        lg = c.decode(s2, tok)
        tok = int(np.argmax(lg))
        ref.append(tok)
    assert [int(t) for t in got] == ref
    assert len(s1) == len(s2) == n_prompt + steps
    assert np.array_equal(s1.tokens(), s2.tokens())
    a = c.decode(s1, 7)
    b = c.decode(s2, 7)
    assert _bits_equal(a, b)


@pytest.mark.parametrize("kvt", [3, 9, 0, 1, 5, 7])
def test_decode_greedy_kv_types(gw, synth_models, kvt):
    """gw_decode_greedy on sequences whose cache is not f16 (q8, q4k4, f32, bf16, bf16-dot, q8-dot): the tokens and the
    cache of gw_decode_argmax step by step (the fused one-row sequence serves the f16 / bf16 caches; the others run the
    per-step passes), across a key-block boundary"""
    path = synth_models("tiny_gqa4")
    m = gw.Model(path, ctx_len=1024)
    c = m.ctx(max_batch=64, max_ctx=1024)
    ids = _ids(m.vocab, 250, 5)
    s1, s2 = m.seq(1024, kv_type=kvt), m.seq(1024, kv_type=kvt)
    lg = c.prefill(s1, ids)
    c.prefill(s2, ids)
    t0 = int(np.argmax(lg))
    got = c.decode_greedy(s1, t0, 12)
    ref, tok = [], t0
    for _ in range(12):
        lg = c.decode(s2, tok)
        tok = int(np.argmax(lg))
        ref.append(tok)
    assert [int(t) for t in got] == ref
    assert _bits_equal(c.decode(s1, 7), c.decode(s2, 7))


def test_memory_and_pass_times(gw, synth_models):
    """rq_model_mem / rq_seq_mem / rq_seq_resident (runq.h:150-171, :274) count the device bytes the library holds,
    and rq_pass_times (runq.h:196-199) times a decode step and a 4-row pass on its own context"""
    import ctypes
    class SeqMem(ctypes.Structure):
        _fields_ = [("kv", ctypes.c_size_t), ("state", ctypes.c_size_t), ("checkpoints", ctypes.c_int), ("total", ctypes.c_size_t)]
    class ModelMem(ctypes.Structure):
        _fields_ = [("weights", ctypes.c_size_t), ("runtime", ctypes.c_size_t), ("seq", SeqMem), ("total", ctypes.c_size_t),
                    ("budget", ctypes.c_double), ("budget_src", ctypes.c_int), ("read", ctypes.c_size_t)]
    lib = gw.lib
    path = synth_models("tiny_gqa4")
    m = gw.Model(path, ctx_len=1024)
    mm = ModelMem()
    assert lib.rq_model_mem(ctypes.c_void_p(m._h), ctypes.byref(mm)) == 0
    assert mm.weights > 0 and mm.read == mm.weights and mm.budget == 0
    assert mm.total == mm.weights + mm.runtime + mm.seq.total
    sm = SeqMem()
    assert lib.rq_seq_mem(ctypes.c_void_p(m._h), 300, 2, ctypes.byref(sm)) == 0
    s = m.seq(300)
    lib.rq_seq_kv_bytes.restype = ctypes.c_size_t
    assert sm.kv == lib.rq_seq_kv_bytes(ctypes.c_void_p(s._h), 300) and sm.total == sm.kv and sm.state == 0
    res = SeqMem()
    lib.rq_seq_resident(ctypes.c_void_p(s._h), ctypes.byref(res))
    assert res.kv == lib.rq_seq_kv_bytes(ctypes.c_void_p(s._h), 0) == 300 * 4  # (lazy: no position written yet)
    s.fill_synthetic(20)
    lib.rq_seq_resident(ctypes.c_void_p(s._h), ctypes.byref(res))
    assert res.kv == lib.rq_seq_kv_bytes(ctypes.c_void_p(s._h), 256) and res.total == res.kv
    f16_kv = sm.kv - 300 * 4
    assert lib.rq_seq_mem(ctypes.c_void_p(m._h), 300, 0, ctypes.byref(sm)) == 0  # (f32: twice the f16 tiles)
    assert sm.kv - 300 * 4 == 2 * f16_kv
    assert lib.rq_seq_mem(ctypes.c_void_p(m._h), 300, 4, ctypes.byref(sm)) == gw.RQ_ERR_ARG  # (4: not a type)
    t1, t4 = ctypes.c_double(), ctypes.c_double()
    assert lib.rq_pass_times(ctypes.c_void_p(m._h), 2, ctypes.byref(t1), ctypes.byref(t4)) == 0
    assert 0 < t1.value < 1 and 0 < t4.value < 1


@pytest.mark.parametrize("shape", ["tiny", "tiny_gqa4"])
def test_decode_same_bits_without_warm_next(gw, synth_models, shape):
    """gw_gemv_warm_next (each decode GEMV warming the next matmul's first tiles) changes no bit: the same prefill and
    decode steps with it off and on give the same logits"""
    path = synth_models(shape)
    m = gw.Model(path, ctx_len=1024)
    c = m.ctx(max_batch=16)
    ids = _ids(m.vocab, 300, 9)
    out = {}
    prev = gw.lib.gw_gemv_warm_next(-1)
    try:
        for on in (0, 1):
            gw.lib.gw_gemv_warm_next(on)
            s = m.seq(1024)
            rows = [c.prefill(s, ids)]
            tok = int(np.argmax(rows[-1]))
            for _ in range(5):
                rows.append(c.decode(s, tok))
                tok = int(np.argmax(rows[-1]))
            out[on] = rows
    finally:
        gw.lib.gw_gemv_warm_next(prev)
    assert all(_bits_equal(a, b) for a, b in zip(out[0], out[1]))


def test_config5_mixed_pass_equals_each_sequence_alone(gw, tmp_path):
    """config 5's pass shape at the 8B model's widths (2 layers): decoding sequences at contexts up to 3000 (past the
    combine-in-GEMV limit), a fresh prompt chunk and a chunk that continues a shared 1,024-token prefix copied from the
    cache (rq_seq_copy), all in one rq_forward_batch, twice: every logits row equal bit for bit to the row the same
    sequence gives when it runs alone (runq.h:22-24)"""
    import os
    from gwenedeg_amd import synth
    d = dict(synth.SHAPES["qwen3_8b"], n_layers=2, vocab=4096)
    path = os.path.join(str(tmp_path), "c5.gguf")
    synth.write_gguf(path, d, seed=3)
    m = gw.Model(path, ctx_len=4096)
    c = m.ctx(max_batch=512, max_ctx=4096)
    rng = np.random.default_rng(8)
    ctxs = [256, 700, 1100, 1800, 2500, 3000]
    dec = [m.seq(4096) for _ in ctxs]
    for i, (sq, n) in enumerate(zip(dec, ctxs)):
        sq.fill_synthetic(n, seed=40 + i)
    shared = m.seq(4096)
    shared.fill_synthetic(1024, seed=77)
    fresh, cont = m.seq(4096), m.seq(4096)
    cont.copy_from(shared, 1024)
    seqs = dec + [fresh, cont]
    twins = [m.seq(4096) for _ in seqs]
    for tw, sq in zip(twins, seqs):
        if len(sq):
            tw.copy_from(sq, len(sq))
    toks = [int(t) for t in rng.integers(0, m.vocab, len(dec))]
    for rnd in range(2):
        ca = [int(t) for t in rng.integers(0, m.vocab, 200)]
        cb = [int(t) for t in rng.integers(0, m.vocab, 150)]
        segs = [gw.Segment(sq, [t], gw.RQ_LOGITS_LAST) for sq, t in zip(dec, toks)]
        segs += [gw.Segment(fresh, ca, gw.RQ_LOGITS_ALL), gw.Segment(cont, cb, gw.RQ_LOGITS_ALL)]
        lg, _ = c.forward_batch(segs)
        alone = [c.decode(tw, t) for tw, t in zip(twins[:len(dec)], toks)]
        alone += list(c.prefill(twins[-2], ca, mode=gw.RQ_LOGITS_ALL)) + list(c.prefill(twins[-1], cb, mode=gw.RQ_LOGITS_ALL))
        assert lg.shape[0] == len(alone) == len(dec) + 350
        for r, (a, b) in enumerate(zip(lg, alone)):
            assert _bits_equal(a, b), f"round {rnd} row {r}: max diff {np.abs(a - b).max()}"
        toks = [int(np.argmax(lg[i])) for i in range(len(dec))]


@pytest.mark.parametrize("shape,n_prompt", [("tiny", 300), ("tiny_gqa4", 40), ("tiny_hd64", 600)])
def test_bf16_kv_bitexact_vs_oracle(gw, synth_models, shape, n_prompt):
    """a bf16 KV cache (RQ_KV_BF16: the reference's bf16 tile layouts, round to nearest even, the same fp32 attention on
    the exactly converted values): the prefill's rows and decode steps bit for bit against the oracle's bf16 cache,
    across key blocks; the cache bytes themselves equal the oracle's"""
    from oracle import oracle as orc
    path = synth_models(shape)
    m = gw.Model(path, ctx_len=1024)
    om = orc.Model(path, cap=1024)
    ids = _ids(m.vocab, n_prompt, 12)
    c = m.ctx(max_batch=128)
    s = m.seq(1024, kv_type=gw.RQ_KV_BF16)
    lg_all = c.prefill(s, ids, mode=gw.RQ_LOGITS_ALL)
    os_ = om.seq(bf16=True)
    for i, t in enumerate(ids):
        ref = os_.forward(int(t))
        assert _bits_equal(lg_all[i], ref), f"row {i}: max diff {np.abs(lg_all[i] - ref).max()}"
    tok = int(np.argmax(lg_all[-1]))
    for step in range(5):
        lg = c.decode(s, tok)
        ref = os_.forward(tok)
        assert _bits_equal(lg, ref), f"decode step {step}: max diff {np.abs(lg - ref).max()}"
        tok = int(np.argmax(ref))


def test_bf16_and_f16_sequences_in_one_pass(gw, synth_models):
    """one rq_forward_batch over f16 and bf16 sequences (the attention items of each cache type in a launch of their
    own) gives every row the bits it gets alone; copies keep the type (rq_seq_copy refuses mixing)"""
    path = synth_models("tiny_gqa4")
    m = gw.Model(path, ctx_len=1024)
    c = m.ctx(max_batch=128)
    rng = np.random.default_rng(21)
    kinds = [gw.RQ_KV_F16, gw.RQ_KV_BF16, gw.RQ_KV_BF16, gw.RQ_KV_F16]
    seqs = [m.seq(1024, kv_type=k) for k in kinds]
    for sq, n in zip(seqs, (30, 270, 5, 300)):
        c.prefill(sq, _ids(m.vocab, n, n))
    twins = [m.seq(1024, kv_type=k) for k in kinds]
    for tw, sq in zip(twins, seqs):
        tw.copy_from(sq, len(sq))
    with pytest.raises(gw.RqError):
        twins[0].copy_from(seqs[1], 5)
    chunks = [[int(t) for t in rng.integers(0, m.vocab, k)] for k in (1, 7, 1, 20)]
    lg, _ = c.forward_batch([gw.Segment(sq, ch, gw.RQ_LOGITS_ALL) for sq, ch in zip(seqs, chunks)])
    alone = []
    for tw, ch in zip(twins, chunks):
        alone += list(c.prefill(tw, ch, mode=gw.RQ_LOGITS_ALL))
    assert lg.shape[0] == len(alone)
    for r, (a, b) in enumerate(zip(lg, alone)):
        assert _bits_equal(a, b), f"row {r}"



@pytest.mark.parametrize("shape", ["tiny_gqa4", "tiny_hd64"])
def test_every_kv_type_in_one_pass(gw, synth_models, shape):
    """one rq_forward_batch over sequences of every KV cache type (runq.h:214: f32, bf16, f16, q8, q4, q4k4 and the five
    dot-product types; each type's attention items in the launch of its kernel) at lengths on both sides of a
    256-position key block, decode rows and prompt rows: every row gets the bits it gets alone, and a type's rows do
    not depend on the other types beside them"""
    path = synth_models(shape)
    m = gw.Model(path, ctx_len=1024)
    c = m.ctx(max_batch=256)
    rng = np.random.default_rng(33)
    kinds = [gw.RQ_KV_F32, gw.RQ_KV_BF16, gw.RQ_KV_F16, gw.RQ_KV_Q8, gw.RQ_KV_Q4, gw.RQ_KV_Q4K4, gw.RQ_KV_BF16_DOT,
             gw.RQ_KV_F16_DOT, gw.RQ_KV_Q8_DOT, gw.RQ_KV_Q4_DOT, gw.RQ_KV_Q4K4_DOT]
    lens = [int(x) for x in rng.integers(3, 520, len(kinds))]
    seqs = [m.seq(1024, kv_type=k) for k in kinds]
    for sq, n in zip(seqs, lens):
        c.prefill(sq, _ids(m.vocab, n, n))
    twins = [m.seq(1024, kv_type=k) for k in kinds]
    for tw, sq in zip(twins, seqs):
        tw.copy_from(sq, len(sq))
    chunks = [[int(t) for t in rng.integers(0, m.vocab, 1 if i % 2 else 9)] for i in range(len(kinds))]
    lg, _ = c.forward_batch([gw.Segment(sq, ch, gw.RQ_LOGITS_ALL) for sq, ch in zip(seqs, chunks)])
    alone = []
    for tw, ch in zip(twins, chunks):
        alone += list(c.prefill(tw, ch, mode=gw.RQ_LOGITS_ALL))
    assert lg.shape[0] == len(alone)
    row = 0
    for k, ch in zip(kinds, chunks):
        for _ in ch:
            assert _bits_equal(lg[row], alone[row]), f"kv type {k}, row {row}"
            row += 1


@pytest.mark.parametrize("k", [1, 7, 40, 64])
def test_device_topk(gw, synth_models, k):
    """gw_ctx_topk: the k best logits of each row on the device and their ids, in sample_topk's order (larger first,
    the lower id first on ties: numpy's lexsort of the host logits), for the rows of a batched pass"""
    path = synth_models("tiny_gqa4")
    m = gw.Model(path, ctx_len=512)
    c = m.ctx(max_batch=64)
    seqs = [m.seq(512) for _ in range(5)]
    segs = [gw.Segment(sq, [int(t) for t in _ids(m.vocab, n, n)], gw.RQ_LOGITS_LAST) for sq, n in zip(seqs, (1, 3, 9, 30, 2))]
    lg, _ = c.forward_batch(segs)
    vals, idx = c.topk(5, k)
    order = np.lexsort((np.arange(m.vocab)[None, :].repeat(5, 0), -lg), axis=1)[:, :k]
    assert np.array_equal(idx, order)
    assert _bits_equal(vals, np.take_along_axis(lg, order, 1))
    for n in (1, 3, 5, 2, 1):  # calls of fewer rows in a row on the same buffers
        v, i = c.topk(n, k)
        assert np.array_equal(i, order[:n]) and _bits_equal(v, np.take_along_axis(lg[:n], order[:n], 1)), n
    # decode contexts without batch buffers (max_batch 0 and 1, runq.h:329): their decode leaves one row
    for mb in (0, 1):
        c1 = m.ctx(max_batch=mb, max_ctx=512)
        s1 = m.seq(512)
        c1.prefill(s1, _ids(m.vocab, 6, 40 + mb), mode=gw.RQ_LOGITS_NONE)
        row = c1.decode(s1, 5)
        v1, i1 = c1.topk(1, k)
        o1 = np.lexsort((np.arange(m.vocab), -row))[:k]
        assert np.array_equal(i1[0], o1), f"max_batch {mb}"
        assert _bits_equal(v1[0], row[o1])


def test_device_topk_full_vocab(gw, workdir):
    """gw_ctx_topk over a 151,936-id row (the Qwen3 vocabulary: 64 chunks of 2,374 logits, the last one short) against
    numpy's order of the host logits, k = 1 and 64; k above 64 is refused before any launch"""
    from gwenedeg_amd import synth
    d = dict(synth.SHAPES["tiny"])
    d["vocab"] = 151936
    path = synth.write_gguf(os.path.join(workdir, "tiny_v151936.gguf"), d, seed=3)
    m = gw.Model(path, ctx_len=256)
    c = m.ctx(max_batch=32)
    seqs = [m.seq(256) for _ in range(3)]
    segs = [gw.Segment(sq, [int(t) for t in _ids(m.vocab, n, n)], gw.RQ_LOGITS_LAST) for sq, n in zip(seqs, (1, 5, 17))]
    lg, _ = c.forward_batch(segs)
    ref = np.lexsort((np.arange(m.vocab)[None, :].repeat(3, 0), -lg), axis=1)
    for k in (1, 64):
        vals, idx = c.topk(3, k)
        assert np.array_equal(idx, ref[:, :k]), k
        assert _bits_equal(vals, np.take_along_axis(lg, ref[:, :k], 1))
    with pytest.raises(Exception):
        c.topk(3, 65)
