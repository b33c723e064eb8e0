"""The device forward path against the reference's own CPU path, compiled from its sources (oracle/_ref, carried with
the repository), on the GPU box's host: the BASELINE configurations at sizes that finish in seconds, with the
north star's three levels of correctness, here met exactly:
  per-block int32 dot sums bit-exact;  logits equal bit for bit (the tolerance's limit);  greedy tokens identical.
The device reproduces the reference's host-specific float operations from tables measured on this host
(gwenedeg_amd/csrc/gw_exact.c); where the host cannot provide them (no AVX-512) the tests are skipped."""
import ctypes
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


@pytest.fixture(scope="module")
def orc():
    from oracle import oracle
    if not oracle.have_ref():
        pytest.skip("oracle/_ref (the reference's CPU path) is not built")
    return oracle


def _exact(gw):
    return gw.exact_mode() & 3 == 3


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _synth(tmp, shape, seed=1, **over):
    from gwenedeg_amd import synth
    d = dict(synth.SHAPES[shape])
    d.update(over)
    path = os.path.join(tmp, f"{shape}.gguf")
    synth.write_gguf(path, d, seed=seed)
    return path, d


def _threads():
    return min(16, len(os.sched_getaffinity(0)))


def test_config1_greedy_128_steps_bit_identical(gw, orc, tmp_path):
    """config 1: the Qwen3-0.6B-shaped Q8_0 model, a 512-token prefill of random ids, 128 greedy steps: every logits
    row (prefill's last + 128 decode steps) equal bit for bit to the reference's, the same 128 tokens"""
    path, d = _synth(str(tmp_path), "qwen3_0_6b")
    m = gw.Model(path, ctx_len=1024)
    if not _exact(gw):
        pytest.skip("this host does not provide the reference's float operations (AVX-512)")
    ids = np.random.default_rng(1).integers(0, m.vocab, 512).astype(np.int32)
    _, rlg, rtok, _ = orc.run_ref_driver(path, ids, str(tmp_path / "ref"), steps=128, threads=_threads(), cap=1024)
    c = m.ctx(max_batch=512, max_ctx=1024)
    s = m.seq(1024)
    lg = c.prefill(s, ids, mode=gw.RQ_LOGITS_LAST)
    toks = []
    for step in range(129):
        assert np.array_equal(_bits(lg), _bits(rlg[step])), f"row {step}: max diff {np.abs(lg - rlg[step]).max()}"
        tok = int(np.argmax(lg))
        toks.append(tok)
        if step < 128:
            assert tok == int(rtok[step]), f"step {step}"
            lg = c.decode(s, tok)
    assert len(toks) == 129


@pytest.mark.parametrize("M", [1, 8, 64, 512])
def test_config2_isolated_q8_op(gw, orc, tmp_path, M):
    """config 2: W = 12288 x 4096 Q8_0 (codes uniform in [-127, 127], fp16 scales |N(0, 1e-3)|), X = N(0, 1) rows
    quantized per 32 (gw_quantize), M = 1 (GEMV), 8, 64, 512 (MFMA GEMM): the output against the reference's
    q8p_gemv_rows / q8p_gemm_item bit for bit, and the per-block int32 sums against integer brute force"""
    import torch
    N, K = 12288, 4096
    rng = np.random.default_rng(100 + M)
    wq = rng.integers(-127, 128, (N, K), dtype=np.int8)
    ws16 = np.abs(rng.normal(0, 1e-3, (N, K // 32))).astype(np.float16)
    x = rng.normal(0, 1, (M, K)).astype(np.float32)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    W, WS, X = dev(wq), dev(ws16.view(np.int16)), dev(x)
    xq = torch.zeros((M, K), dtype=torch.int8, device="cuda")
    xs = torch.zeros((M, K // 32), dtype=torch.float32, device="cuda")
    out = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    assert gw.lib.gw_quantize(X.data_ptr(), M, K, xq.data_ptr(), xs.data_ptr(), None) == 0
    assert gw.lib.gw_q8_matmul(out.data_ptr(), W.data_ptr(), WS.data_ptr(), N, K, xq.data_ptr(), xs.data_ptr(), M, None) == 0
    nb = 64  # block sums of the first 64 weight rows
    isum = torch.zeros((M, nb, K // 32), dtype=torch.int32, device="cuda")
    assert gw.lib.gw_q8_block_sums(isum.data_ptr(), W.data_ptr(), nb, K, xq.data_ptr(), M, None) == 0
    torch.cuda.synchronize()
    xq_h, xs_h = xq.cpu().numpy(), xs.cpu().numpy()
    ref, _ = orc.run_ref_q8op(str(tmp_path), wq, ws16.astype(np.float32), xq_h, xs_h, threads=_threads())
    got = out.cpu().numpy()
    assert np.array_equal(_bits(got), _bits(ref)), f"max diff {np.abs(got - ref).max()}"
    brute = np.einsum("ngk,mgk->mng", wq[:nb].reshape(nb, K // 32, 32).astype(np.int64),
                      xq_h.reshape(M, K // 32, 32).astype(np.int64))
    assert np.array_equal(isum.cpu().numpy().astype(np.int64), brute)


def test_config3_q4km_batched_decode(gw, orc, tmp_path):
    """config 3 (reduced depth): a Qwen3-4B-shaped Q4_K_M model (Q4_K q / k / o / gate / up and the embedding, Q6_K v /
    down / output), 2 layers; 6 sequences prefilled with a 300-token prompt, then 8 batched greedy decode passes of one
    row per sequence (rq_forward_batch): every logits row bit for bit against the reference's batched decode"""
    path, d = _synth(str(tmp_path), "qwen3_4b_q4km", n_layers=2)
    m = gw.Model(path, ctx_len=1024)
    if not _exact(gw):
        pytest.skip("this host does not provide the reference's float operations (AVX-512)")
    ns, steps = 6, 8
    ids = np.random.default_rng(3).integers(0, m.vocab, 300).astype(np.int32)
    _, rlg, rtok, _ = orc.run_ref_driver(path, ids, str(tmp_path / "ref"), steps=steps, threads=_threads(), cap=1024,
                                         batch_decode=ns)
    c = m.ctx(max_batch=512, max_ctx=1024)
    seqs = [m.seq(1024) for _ in range(ns)]
    toks = []
    for i, sq in enumerate(seqs):
        lg = c.prefill(sq, ids, mode=gw.RQ_LOGITS_LAST)
        assert np.array_equal(_bits(lg), _bits(rlg[i])), f"prefill of sequence {i}"
        toks.append(int(np.argmax(lg)))
    for st in range(steps):
        assert toks == [int(t) for t in rtok[st * ns:(st + 1) * ns]], f"tokens fed at step {st}"
        lg, _ = c.forward_batch([gw.Segment(sq, [t], gw.RQ_LOGITS_LAST) for sq, t in zip(seqs, toks)])
        ref = rlg[ns + st * ns: ns + (st + 1) * ns]
        assert np.array_equal(_bits(lg[:ns]), _bits(ref)), f"step {st}: max diff {np.abs(lg[:ns] - ref).max()}"
        toks = [int(np.argmax(r)) for r in lg[:ns]]


def test_config4_long_context_8b_shape(gw, orc, tmp_path):
    """config 4 (reduced): a Qwen3-8B-shaped Q8_0 model, 2 layers, a 2600-token prompt (11 key blocks: the attention
    combine past the decode matmul's fused limit) then 16 greedy decode steps: bit for bit against the reference"""
    path, d = _synth(str(tmp_path), "qwen3_8b", n_layers=2)
    m = gw.Model(path, ctx_len=4096)
    if not _exact(gw):
        pytest.skip("this host does not provide the reference's float operations (AVX-512)")
    ids = np.random.default_rng(4).integers(0, m.vocab, 2600).astype(np.int32)
    _, rlg, rtok, _ = orc.run_ref_driver(path, ids, str(tmp_path / "ref"), steps=16, threads=_threads(), cap=4096)
    c = m.ctx(max_batch=512, max_ctx=4096)
    s = m.seq(4096)
    lg = c.prefill(s, ids, mode=gw.RQ_LOGITS_LAST)
    for step in range(17):
        assert np.array_equal(_bits(lg), _bits(rlg[step])), f"row {step}: max diff {np.abs(lg - rlg[step]).max()}"
        if step < 16:
            tok = int(np.argmax(lg))
            assert tok == int(rtok[step])
            lg = c.decode(s, tok)


@pytest.mark.parametrize("shape,layers", [("qwen3_0_6b", 3), ("qwen3_4b_q4km", 2)])
def test_hidden_rows_bit_identical(gw, orc, tmp_path, shape, layers):
    """the rows' final hidden states (after output_norm: runq.h:347-350, :369) against the reference's
    rq_decode_hidden token by token, bit for bit with the logits: rq_decode_hidden one row at a time, and fw_rows
    (internal.h:339, the spec loop's prefill) in chunks of 8 rows and as one 40-row pass"""
    path, d = _synth(str(tmp_path), shape, n_layers=layers)
    m = gw.Model(path, ctx_len=256)
    if not _exact(gw):
        pytest.skip("this host does not provide the reference's float operations (AVX-512)")
    ids = np.random.default_rng(7).integers(0, m.vocab, 40).astype(np.int32)
    _, rlg, rhid, _ = orc.run_ref_driver(path, ids, str(tmp_path / "ref"), threads=_threads(), cap=256, hidden=True)
    assert rhid.shape == (40, m.dim)
    c1 = m.ctx(max_batch=1, max_ctx=256)
    s1 = m.seq(256)
    for j, t in enumerate(ids):
        lg, hid = c1.decode_hidden(s1, int(t))
        assert np.array_equal(_bits(hid), _bits(rhid[j])), f"rq_decode_hidden row {j}"
        assert np.array_equal(_bits(lg), _bits(rlg[j])), f"rq_decode_hidden logits row {j}"
    for nb in (8, 64):
        c = m.ctx(max_batch=nb, max_ctx=256)
        s = m.seq(256)
        lg, hid = c.prefill_hidden(s, ids, mode=gw.RQ_LOGITS_ALL)
        assert np.array_equal(_bits(hid), _bits(rhid)), f"fw_rows (max_batch {nb}): hidden rows"
        assert np.array_equal(_bits(lg), _bits(rlg)), f"fw_rows (max_batch {nb}): logits rows"


def test_hidden_rows_after_batched_passes_on_one_context(gw, orc, tmp_path):
    """hidden rows from one-row passes that follow multi-row passes on the same context (the speculative loop's
    pattern, spec.c:336-350): a 20-token prefill in passes of 8 rows, then rq_decode_hidden, then fw_rows of 41 tokens
    with max_batch 8 (its last chunk one row), on an all-Q8_0 model (the one-row passes take the fused decode
    sequence, which keeps no pending residual): every hidden row and logits row bit for bit against the reference's
    rq_decode_hidden token by token"""
    path, d = _synth(str(tmp_path), "qwen3_0_6b", n_layers=3)
    m = gw.Model(path, ctx_len=256)
    if not _exact(gw):
        pytest.skip("this host does not provide the reference's float operations (AVX-512)")
    ids = np.random.default_rng(12).integers(0, m.vocab, 62).astype(np.int32)
    _, rlg, rhid, _ = orc.run_ref_driver(path, ids, str(tmp_path / "ref"), threads=_threads(), cap=256, hidden=True)
    c = m.ctx(max_batch=8, max_ctx=256)
    s = m.seq(256)
    lg, hid = c.prefill_hidden(s, ids[:20], mode=gw.RQ_LOGITS_ALL)
    assert np.array_equal(_bits(hid), _bits(rhid[:20])) and np.array_equal(_bits(lg), _bits(rlg[:20]))
    lg, hid = c.decode_hidden(s, int(ids[20]))
    assert np.array_equal(_bits(hid), _bits(rhid[20])), "rq_decode_hidden after a batched prefill: hidden row"
    assert np.array_equal(_bits(lg), _bits(rlg[20])), "rq_decode_hidden after a batched prefill: logits"
    lg, hid = c.prefill_hidden(s, ids[21:62], mode=gw.RQ_LOGITS_ALL)
    assert np.array_equal(_bits(hid), _bits(rhid[21:62])), "fw_rows n 41, max_batch 8: hidden rows"
    assert np.array_equal(_bits(lg), _bits(rlg[21:62])), "fw_rows n 41, max_batch 8: logits rows"


# RQ_KV_F16, RQ_KV_BF16, RQ_KV_Q8, RQ_KV_Q4, RQ_KV_Q4K4, the dot-product types RQ_KV_BF16_DOT, F16_DOT, Q8_DOT, Q4_DOT,
# Q4K4_DOT, and RQ_KV_F32
@pytest.mark.parametrize("kvt", [2, 1, 3, 8, 9, 5, 6, 7, 12, 13, 0])
def test_seqfile_with_reference(gw, orc, tmp_path, kvt):
    """the KV disk tier (runq.h:283-314) against the reference's seqfile.c: the same model fingerprint; the reference's
    saved sequence (300-token prompt + 4 greedy steps) read by rq_seq_file_info and loaded by rq_seq_load continues bit
    for bit as the device's own sequence of the same tokens; the device's saved file matches the reference's header
    and tokens (all but the RNG word and the hash over it) and its whole K / V blocks byte for byte, and loads back;
    with each cache type the device keeps (a file loads only into a sequence of its cache type; the quantized caches'
    blocks hold the rotated, quantized rows, and the bf16-dot V its position pairs, so their bytes pin the store)"""
    import ctypes
    path, d = _synth(str(tmp_path), "qwen3_0_6b", n_layers=2)
    m = gw.Model(path, ctx_len=1024)
    if not _exact(gw):
        pytest.skip("this host does not provide the reference's float operations (AVX-512)")
    ids = np.random.default_rng(11).integers(0, m.vocab, 300).astype(np.int32)
    info, rlg, rtok, kvp = orc.run_ref_driver(path, ids, str(tmp_path / "ref"), steps=4, threads=_threads(), cap=1024, kv=True,
                                              kv_type=kvt)
    assert int(info["fingerprint"], 16) == m.info.fingerprint
    lib = gw.lib

    class SeqFile(ctypes.Structure):
        _fields_ = [("len", ctypes.c_int), ("kv_type", ctypes.c_int), ("linear", ctypes.c_int), ("n_ck", ctypes.c_int),
                    ("ck", ctypes.c_int * 32), ("bytes", ctypes.c_longlong)]
    fi, tk = SeqFile(), ctypes.POINTER(ctypes.c_int)()
    assert lib.rq_seq_file_info(ctypes.c_void_p(m._h), kvp.encode(), ctypes.byref(fi), ctypes.byref(tk)) == 0
    L = fi.len
    assert L == 304 and fi.kv_type == kvt and fi.bytes == os.path.getsize(kvp)
    saved = np.ctypeslib.as_array(tk, shape=(L,)).copy()
    assert np.array_equal(saved[:300], ids) and np.array_equal(saved[300:], rtok[:4])
    # the device's own sequence of the same tokens, and the reference's file loaded, each continued by one token
    c = m.ctx(max_batch=512, max_ctx=1024)
    own = m.seq(1024, kv_type=kvt)
    c.prefill(own, saved, mode=gw.RQ_LOGITS_NONE)
    loaded = m.seq(1024, kv_type=kvt)
    assert lib.rq_seq_load(ctypes.c_void_p(loaded._h), kvp.encode(), L) == 0
    assert lib.rq_seq_len(ctypes.c_void_p(loaded._h)) == L
    a, b = c.decode(own, 7), c.decode(loaded, 7)
    assert np.array_equal(_bits(a), _bits(b))
    # the device's file of the same sequence (before the extra token: a fresh copy of it)
    mine = m.seq(1024, kv_type=kvt)
    assert lib.rq_seq_load(ctypes.c_void_p(mine._h), kvp.encode(), L) == 0
    p2 = str(tmp_path / "mine.seq")
    assert lib.rq_seq_save(ctypes.c_void_p(mine._h), p2.encode()) == 0
    lib.rq_seq_save_bytes.restype = ctypes.c_longlong
    assert lib.rq_seq_save_bytes(ctypes.c_void_p(mine._h)) == os.path.getsize(p2) == os.path.getsize(kvp)
    r, o = np.fromfile(kvp, np.uint8), np.fromfile(p2, np.uint8)
    hdr = np.ones(264, bool)
    hdr[248:264] = False  # (the RNG word and the hash)
    assert np.array_equal(r[:264][hdr], o[:264][hdr])
    assert np.array_equal(r[4096:4096 + 4 * L], o[4096:4096 + 4 * L])
    hd = m.info.head_dim
    tile = {0: (64, 64), 2: (32, 32), 1: (32, 32), 3: (17, 17), 8: (17, 9), 9: (9, 9)}[kvt & ~4 if kvt in (5, 6, 7, 12, 13) else kvt]
    # (K, V tile bytes per dim: a dot-product type's are its base type's)
    off_kv = int(np.frombuffer(r[224:232].tobytes(), np.uint64)[0])
    bk, bv = (16 * m.info.n_kv_heads * hd * t for t in tile)
    nblk = (L + 255) // 256
    for l in range(2):
        for kv in range(2):  # (the first block of each section is whole: positions 0..255 < L)
            s0, blk = off_kv + nblk * (l * (bk + bv) + kv * bk), (bv if kv else bk)
            assert np.array_equal(r[s0:s0 + blk], o[s0:s0 + blk]), f"layer {l} kv {kv}"
    again = m.seq(1024, kv_type=kvt)
    assert lib.rq_seq_load(ctypes.c_void_p(again._h), p2.encode(), 200) == 0
    assert lib.rq_seq_len(ctypes.c_void_p(again._h)) == 200
    c2 = m.seq(1024, kv_type=kvt)
    c.prefill(c2, saved[:200], mode=gw.RQ_LOGITS_NONE)
    assert np.array_equal(_bits(c.decode(again, 9)), _bits(c.decode(c2, 9)))
    # errors: another length past the file, a corrupt header
    assert lib.rq_seq_load(ctypes.c_void_p(m.seq(1024, kv_type=kvt)._h), p2.encode(), L + 1) == -1  # RQ_ERR_ARG
    bad = o.copy()
    bad[100] ^= 1
    p3 = str(tmp_path / "bad.seq")
    bad.tofile(p3)
    assert lib.rq_seq_load(ctypes.c_void_p(m.seq(1024, kv_type=kvt)._h), p3.encode(), 10) == -7  # RQ_ERR_MISMATCH
    other = gw.RQ_KV_BF16 if kvt == gw.RQ_KV_F16 else gw.RQ_KV_F16
    assert lib.rq_seq_load(ctypes.c_void_p(m.seq(1024, kv_type=other)._h), p2.encode(), 10) == -7


# RQ_KV_Q8, RQ_KV_Q4, RQ_KV_Q4K4; the dot-product types RQ_KV_BF16_DOT, F16_DOT, Q8_DOT, Q4_DOT, Q4K4_DOT; RQ_KV_F32
@pytest.mark.parametrize("shape,kvt", [("qwen3_0_6b", k) for k in (3, 8, 9, 5, 6, 7, 12, 13, 0)] +
                         [("tiny_hd64", k) for k in (9, 12, 5, 0)] + [("tiny_kv16", k) for k in (2, 3, 9, 0, 5, 7)])
def test_quantized_kv_greedy_bit_identical(gw, orc, tmp_path, shape, kvt):
    """the rotated 8-bit / 4-bit KV caches (forward.c:1609-1790), the bf16 dot-product attention types
    (forward.c:1452-1606: bf16 q, K, V and weights, vdpbf16ps's pairs, FTZ / DAZ) and the f32 cache (forward.c:1945-1950:
    fp32 tiles, the fp32 attention) on a Qwen3-0.6B-shaped model (2 layers; and head_dim-64 models of 8 and of 16
    query heads on one kv head, the latter's rows past the 8-vector attention items): a 300-token prefill (two key blocks,
    16-vector row blocks) and 24 greedy steps, every logits row equal bit for bit to the reference's own cache of that
    type, the same tokens; then a pass of that sequence's next token beside a fresh sequence's prompt (both of the
    type) equal to each run alone"""
    # (tiny_hd64 with a vocabulary of 1024 rows: a Q8_0 matrix of rows not a multiple of 16 turns the reference's packed
    # SIMD kernels off for the whole model (model.c:383-400), and its generic single-row dot_q8 (forward.c:906) does
    # not round as its GEMM does under its -Ofast build)
    path, d = _synth(str(tmp_path), shape, seed=4, **({"n_layers": 2} if shape == "qwen3_0_6b" else {"vocab": 1024}))
    m = gw.Model(path, ctx_len=512)
    if not _exact(gw):
        pytest.skip("this host does not provide the reference's float operations (AVX-512)")
    ids = np.random.default_rng(9).integers(0, m.vocab, 300).astype(np.int32)
    _, rlg, rtok, _ = orc.run_ref_driver(path, ids, str(tmp_path / "ref"), steps=24, threads=_threads(), cap=512, kv_type=kvt)
    c = m.ctx(max_batch=512, max_ctx=512)
    s = m.seq(512, kv_type=kvt)
    lg = c.prefill(s, ids, mode=gw.RQ_LOGITS_LAST)
    for step in range(25):
        assert np.array_equal(_bits(lg), _bits(rlg[step])), f"row {step}: max diff {np.abs(lg - rlg[step]).max()}"
        tok = int(np.argmax(lg))
        if step < 24:
            assert tok == int(rtok[step]), f"step {step}"
            lg = c.decode(s, tok)
    # batch invariance: the next token of s beside a fresh prompt, against each alone
    s2, s3 = m.seq(512, kv_type=kvt), m.seq(512, kv_type=kvt)
    assert gw.lib.rq_seq_copy(ctypes.c_void_p(s2._h), ctypes.c_void_p(s._h), len(s)) == 0
    p2 = ids[:40]
    both, _ = c.forward_batch([gw.Segment(s, [tok], gw.RQ_LOGITS_LAST), gw.Segment(s3, p2, gw.RQ_LOGITS_LAST)])
    alone_a = c.decode(s2, tok)
    s4 = m.seq(512, kv_type=kvt)
    alone_b = c.prefill(s4, p2, mode=gw.RQ_LOGITS_LAST)
    assert np.array_equal(_bits(both[0]), _bits(alone_a)) and np.array_equal(_bits(both[1]), _bits(alone_b))


@pytest.mark.parametrize("shape", ["tiny_q5k", "tiny_q3k", "tiny_iq4xs", "tiny_q2k", "tiny_iq2_xxs", "tiny_iq2_xs",
                                   "tiny_iq2_s", "tiny_iq3_xxs", "tiny_iq3_s", "tiny_iq1_s", "tiny_iq1_m"])
def test_q5k_q3k_models_greedy_bit_identical(gw, orc, tmp_path, shape):
    """Q5_K_M-, Q3_K_M-, IQ4_XS- and Q2_K-style models (Q5_K / Q3_K / IQ4_XS / Q2_K matrices beside Q4_K / Q5_K / Q6_K
    ones, the K-quant or IQ4_XS embedding) and one model per codebook i-quant (every matrix and the embedding of that
    type, Q6_K output): a 64-token prefill and 24 greedy steps, every logits row equal bit for bit to the reference's,
    the same tokens. The i-quant models' matrices hold at most 1.25 times the file's bytes on the device"""
    import ctypes
    path, d = _synth(str(tmp_path), shape, seed=7)
    m = gw.Model(path, ctx_len=512)
    if "iq" in shape:
        class SeqMem(ctypes.Structure):
            _fields_ = [("kv", ctypes.c_size_t), ("state", ctypes.c_size_t), ("checkpoints", ctypes.c_int),
                        ("total", ctypes.c_size_t)]
        class ModelMem(ctypes.Structure):
            _fields_ = [("weights", ctypes.c_size_t), ("runtime", ctypes.c_size_t), ("seq", SeqMem),
                        ("total", ctypes.c_size_t), ("budget", ctypes.c_double), ("budget_src", ctypes.c_int),
                        ("read", ctypes.c_size_t)]
        mm = ModelMem()
        assert gw.lib.rq_model_mem(ctypes.c_void_p(m._h), ctypes.byref(mm)) == 0
        L, dim, hd = d["n_layers"], d["dim"], d["head_dim"]
        norms = (2 * L * dim + 2 * L * hd + dim) * 4
        rope = 512 * hd * 4
        assert mm.weights - norms - rope <= 1.25 * (os.path.getsize(path) - norms), (mm.weights, os.path.getsize(path))
    if not _exact(gw):
        pytest.skip("this host does not provide the reference's float operations (AVX-512)")
    ids = np.random.default_rng(5).integers(0, m.vocab, 64).astype(np.int32)
    _, rlg, rtok, _ = orc.run_ref_driver(path, ids, str(tmp_path / "ref"), steps=24, threads=_threads(), cap=512)
    c = m.ctx(max_batch=64, max_ctx=512)
    s = m.seq(512)
    lg = c.prefill(s, ids, mode=gw.RQ_LOGITS_LAST)
    for step in range(25):
        assert np.array_equal(_bits(lg), _bits(rlg[step])), f"row {step}: max diff {np.abs(lg - rlg[step]).max()}"
        tok = int(np.argmax(lg))
        if step < 24:
            assert tok == int(rtok[step]), f"step {step}"
            lg = c.decode(s, tok)


@pytest.mark.parametrize("shape,repack", [("tiny_iq3_xxs", 1), ("tiny_iq3_s", 1), ("tiny_iq3_xxs", 4), ("tiny_iq3_s", 2),
                                          ("tiny_iq3_s", 4)])
def test_iq3_repack_same_bits(gw, orc, tmp_path, shape, repack):
    """RqModelOpts.repack (runq.h:76-82): an IQ3 model loaded with its matrices repacked as 4-bit codes (RQ_REPACK_ALL
    or the type's bit; another type's bit repacks nothing) gives the same logits as loaded without, bit for bit, over a
    64-token prefill and 24 greedy steps; rq_repack_info (model.c:1402-1438) reports the type, whether it is
    repacked, and the repack's extra bytes, which the weights grow by"""
    import ctypes

    class RT(ctypes.Structure):
        _fields_ = [("type", ctypes.c_char_p), ("bit", ctypes.c_int), ("repacked", ctypes.c_int), ("mats", ctypes.c_int),
                    ("share", ctypes.c_double), ("bytes", ctypes.c_size_t), ("extra", ctypes.c_size_t)]

    class RI(ctypes.Structure):
        _fields_ = [("available", ctypes.c_int), ("n", ctypes.c_int), ("t", RT * 4), ("weights", ctypes.c_size_t),
                    ("extra", ctypes.c_size_t)]
    path, d = _synth(str(tmp_path), shape, seed=3)
    base = 18 if "xxs" in shape else 21
    hits = repack & 1 or (repack & 4 and base == 18) or (repack & 2 and base == 21)
    ids = np.random.default_rng(8).integers(0, d["vocab"], 64).astype(np.int32)
    runs, infos = [], []
    for rp in (0, repack):
        m = gw.Model(path, ctx_len=512, repack=rp)
        ri = RI()
        assert gw.lib.rq_repack_info(ctypes.c_void_p(m._h), ctypes.byref(ri)) == 0
        infos.append(ri)
        c = m.ctx(max_batch=64, max_ctx=512)
        s = m.seq(512)
        rows = [c.prefill(s, ids, mode=gw.RQ_LOGITS_LAST)]
        for _ in range(24):
            rows.append(c.decode(s, int(np.argmax(rows[-1]))))
        runs.append(rows)
        s.close()
        c.close()
        m.close()
    assert all(np.array_equal(_bits(a), _bits(b)) for a, b in zip(runs[0], runs[1]))
    a, b = infos
    assert a.available == 1 and a.n == 1 and a.t[0].type.decode() == ("IQ3_XXS" if base == 18 else "IQ3_S")
    assert a.t[0].bit == (4 if base == 18 else 2) and a.t[0].repacked == 0 and a.t[0].mats == 2 * 7
    nblk = sum(r * c_ for r, c_ in [(1024, 512), (256, 512), (256, 512), (512, 1024), (1024, 512), (1024, 512),
                                    (512, 1024)]) * 2 // 256
    assert a.t[0].extra == nblk * (144 - (100 if base == 18 else 112)) and a.extra == a.t[0].extra
    assert b.t[0].repacked == int(bool(hits)) and b.extra == (0 if hits else a.extra)
    assert b.weights == a.weights + (a.t[0].extra if hits else 0)


def test_bf16_kv_greedy_bit_identical(gw, orc, tmp_path):
    """a bf16 KV cache (RQ_KV_BF16) on a Qwen3-0.6B-shaped model (2 layers): a 300-token prefill (two key blocks) and
    24 greedy steps, every logits row equal bit for bit to the reference's own bf16 cache, the same tokens"""
    path, d = _synth(str(tmp_path), "qwen3_0_6b", seed=4, n_layers=2)
    m = gw.Model(path, ctx_len=512)
    if not _exact(gw):
        pytest.skip("this host does not provide the reference's float operations (AVX-512)")
    ids = np.random.default_rng(9).integers(0, m.vocab, 300).astype(np.int32)
    _, rlg, rtok, _ = orc.run_ref_driver(path, ids, str(tmp_path / "ref"), steps=24, threads=_threads(), cap=512,
                                         kv_type=gw.RQ_KV_BF16)
    c = m.ctx(max_batch=512, max_ctx=512)
    s = m.seq(512, kv_type=gw.RQ_KV_BF16)
    lg = c.prefill(s, ids, mode=gw.RQ_LOGITS_LAST)
    for step in range(25):
        assert np.array_equal(_bits(lg), _bits(rlg[step])), f"row {step}: max diff {np.abs(lg - rlg[step]).max()}"
        tok = int(np.argmax(lg))
        if step < 24:
            assert tok == int(rtok[step]), f"step {step}"
            lg = c.decode(s, tok)
