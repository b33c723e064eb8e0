"""Kernel-level parity on the GPU through the C ABI (gw_quantize, gw_q8_matmul, gw_q8_block_sums, gw_kq_matmul):
bit-exact against the oracle on the same seeded inputs (integer sums exact; fp32 outputs the same bits, since both
compute the reference's fold operation for operation)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    import gwenedeg_amd as gw
    return torch, gw


def _rand_q8(rng, N, K):
    wq = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    ws16 = np.abs(rng.normal(0, 1e-3, size=(N, K // 32))).astype(np.float16)
    return wq, ws16


def _to_dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("M,K", [(1, 1024), (3, 4096), (4, 2560), (5, 3072), (8, 12288), (17, 1024)])
def test_quantize_bitexact(dev, M, K):
    torch, gw = dev
    from oracle import oracle as orc
    rng = np.random.default_rng(M * 1000 + K)
    x = rng.normal(0, 1, size=(M, K)).astype(np.float32)
    x[0, :32] = 0.0            # an all-zero group: s = 0, q = 0
    x[0, 32:64] = 1e-30        # tiny values
    if M > 1:
        x[1, 64:96] = -3.5     # a constant group: every q = -127
    q_ref, s_ref = orc.quantize(x)
    xd = _to_dev(torch, x)
    q = torch.zeros((M, K), dtype=torch.int8, device="cuda")
    s = torch.zeros((M, K // 32), dtype=torch.float32, device="cuda")
    assert gw.lib.gw_quantize(xd.data_ptr(), M, K, q.data_ptr(), s.data_ptr(), None) == 0
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy(), q_ref)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))


@pytest.mark.parametrize("M,N,K,tile", [(1, 256, 1024, 0), (1, 1024, 4096, 0), (2, 512, 12288, 0), (4, 64, 2560, 0),
                                        (7, 128, 4096, 0), (16, 48, 1024, 0), (64, 32, 1024, 0), (40, 208, 768, 32),
                                        (100, 208, 768, 64), (40, 208, 800, 32), (100, 208, 864, 64), (512, 384, 4096, 0)])
def test_q8_matmul_bitexact(dev, M, N, K, tile):
    """the Q8_0 operator against the oracle bit for bit (above 32 rows the MFMA GEMM, its row tile forced where given;
    K % 128 == 0: k_gemm_q8f, else k_gemm_q8 with a partial last stage)"""
    torch, gw = dev
    from oracle import oracle as orc
    rng = np.random.default_rng(N + 7 * K + M)
    wq, ws16 = _rand_q8(rng, N, K)
    x = rng.normal(0, 1, size=(M, K)).astype(np.float32)
    xq, xs = orc.quantize(x)
    ref = orc.q8_matmul(wq, ws16.astype(np.float32), xq, xs)
    out = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    W, WS, XQ, XS = (_to_dev(torch, a) for a in (wq, ws16.view(np.int16), xq, xs))
    prev = gw.lib.gw_matmul_tile_rows(tile)
    try:
        assert gw.lib.gw_q8_matmul(out.data_ptr(), W.data_ptr(), WS.data_ptr(), N, K, XQ.data_ptr(), XS.data_ptr(), M, None) == 0
        torch.cuda.synchronize()
    finally:
        gw.lib.gw_matmul_tile_rows(prev)
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"max diff {np.abs(got - ref).max()}"


@pytest.mark.parametrize("kern", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("M,N,K", [(9, 128, 128), (33, 208, 768), (64, 1008, 1024), (100, 384, 4096), (130, 256, 12288),
                                   (512, 1024, 4096), (512, 512, 12288)])
def test_q8_gemm_kernels_bitexact(dev, M, N, K, kern):
    """the Q8_0 MFMA GEMM (K % 128 == 0) with each kernel forced (gw_q8_gemm_kernel: 1 k_gemm_q8f, 2 / 3 k_gemm_q8l of 128 / 64 columns, 4 / 5 k_gemm_q8t of 64 x 64 tiles with 256- /
    128-byte stages, 6 / 7 of 32 x 32 / 32 x 16 tiles, 8 of 32 x 32 tiles with 512-byte stages where K % 512 == 0, else 6) against
    the oracle bit for bit: partial row tiles (9, 33, 100, 130 rows), partial column tiles (208, 1,008), one stage (K =
    128) and two (256 would be one pair of stages; 768 an odd count), the 8B widths at 512 rows"""
    torch, gw = dev
    from oracle import oracle as orc
    rng = np.random.default_rng(N + 5 * K + M)
    wq, ws16 = _rand_q8(rng, N, K)
    xq, xs = orc.quantize(rng.normal(0, 1, size=(M, K)).astype(np.float32))
    ref = orc.q8_matmul(wq, ws16.astype(np.float32), xq, xs)
    out = torch.full((M, N), 7.0, dtype=torch.float32, device="cuda")
    W, WS, XQ, XS = (_to_dev(torch, a) for a in (wq, ws16.view(np.int16), xq, xs))
    prev, pb = gw.lib.gw_q8_gemm_kernel(kern), gw.lib.gw_q8_batch_kernel(2)
    try:
        assert gw.lib.gw_q8_matmul(out.data_ptr(), W.data_ptr(), WS.data_ptr(), N, K, XQ.data_ptr(), XS.data_ptr(), M, None) == 0
        torch.cuda.synchronize()
    finally:
        gw.lib.gw_q8_gemm_kernel(prev)
        gw.lib.gw_q8_batch_kernel(pb)
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"max diff {np.abs(got - ref).max()}"


_FEW_ROWS = {}


@pytest.mark.parametrize("off", [0, 1, 2])
@pytest.mark.parametrize("M", [2, 5, 8, 9, 16, 17, 24, 32, 33, 48, 64])
@pytest.mark.parametrize("N,K", [(12288, 4096), (4096, 12288), (1008, 1056)])
def test_q8_matmul_few_rows_bitexact(dev, M, N, K, off):
    """the Q8_0 operator at 2 .. 64 activation rows against the oracle bit for bit, with each kernel choice
    (gw_q8_batch_kernel: chosen per launch, the batched GEMV in passes of 8 rows, the MFMA GEMM): the 8B widths, and a
    matrix of 1,008 rows (a partial column tile) by 33 groups (a partial stage: k_gemm_q8)"""
    torch, gw = dev
    from oracle import oracle as orc
    key = (M, N, K)
    if key not in _FEW_ROWS:  # (the inputs and the oracle's result, shared by both kernels' cases)
        rng = np.random.default_rng(N + 3 * K + M)
        wq, ws16 = _rand_q8(rng, N, K)
        xq, xs = orc.quantize(rng.normal(0, 1, size=(M, K)).astype(np.float32))
        _FEW_ROWS.clear()
        _FEW_ROWS[key] = (wq, ws16, xq, xs, orc.q8_matmul(wq, ws16.astype(np.float32), xq, xs))
    wq, ws16, xq, xs, ref = _FEW_ROWS[key]
    out = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    W, WS, XQ, XS = (_to_dev(torch, a) for a in (wq, ws16.view(np.int16), xq, xs))
    prev = gw.lib.gw_q8_batch_kernel(off)
    try:
        assert gw.lib.gw_q8_matmul(out.data_ptr(), W.data_ptr(), WS.data_ptr(), N, K, XQ.data_ptr(), XS.data_ptr(), M, None) == 0
        torch.cuda.synchronize()
    finally:
        gw.lib.gw_q8_batch_kernel(prev)
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"max diff {np.abs(got - ref).max()}"


def test_q8_pack_and_block_sums(dev):
    torch, gw = dev
    from oracle import oracle as orc
    rng = np.random.default_rng(5)
    N, K, M = 96, 2048, 3
    wq, ws16 = _rand_q8(rng, N, K)
    blocks = np.zeros((N, K // 32, 34), np.uint8)
    blocks[:, :, 0:2] = ws16.view(np.uint8).reshape(N, K // 32, 2)
    blocks[:, :, 2:] = wq.view(np.uint8).reshape(N, K // 32, 32)
    B = _to_dev(torch, blocks.reshape(-1))
    codes = torch.zeros((N, K), dtype=torch.int8, device="cuda")
    scales = torch.zeros((N, K // 32), dtype=torch.int16, device="cuda")
    assert gw.lib.gw_q8_pack(B.data_ptr(), N, K, codes.data_ptr(), scales.data_ptr(), None) == 0
    torch.cuda.synchronize()
    assert np.array_equal(codes.cpu().numpy(), wq)
    assert np.array_equal(scales.cpu().numpy().view(np.uint16), ws16.view(np.uint16))
    xq = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    xq[0, :32] = 127
    wq2 = wq.copy()
    wq2[0, :32] = 127  # the largest group sum: 32 * 127 * 127 = 516,128
    codes2 = _to_dev(torch, wq2)
    isum = torch.zeros((M, N, K // 32), dtype=torch.int32, device="cuda")
    XQ = _to_dev(torch, xq)
    assert gw.lib.gw_q8_block_sums(isum.data_ptr(), codes2.data_ptr(), N, K, XQ.data_ptr(), M, None) == 0
    torch.cuda.synchronize()
    ref = orc.q8_block_sums(wq2, xq)
    got = isum.cpu().numpy()
    assert got[0, 0, 0] == 516128
    assert np.array_equal(got, ref)
    # brute force in int64 for one row
    assert np.array_equal(got[1, 7], (wq2[7].astype(np.int64).reshape(-1, 32) * xq[1].astype(np.int64).reshape(-1, 32)).sum(1))


@pytest.mark.parametrize("typ", [10, 11, 12, 13, 14, 23, 16, 17, 22, 18, 21, 19, 29])
@pytest.mark.parametrize("M,tile", [(1, 0), (3, 0), (6, 0), (9, 0), (20, 0), (32, 0), (40, 0), (40, 32), (40, 64),
                                    (100, 64)])
def test_kq_matmul_bitexact(dev, typ, M, tile):
    """the K-quant and i-quant operator (Q2_K, Q3_K, Q4_K, Q5_K, Q6_K; IQ4_XS and the codebook types IQ2_XXS, IQ2_XS,
    IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M decoded in the kernels) against the oracle bit for bit: up to 8 rows the batched
    GEMV, 9 .. 32 the 32-row GEMM (k_gemm_kq32; the other types: the batched GEMV in passes of 8), above it the MFMA
    GEMM with 32- and 64-row tiles (forced) or, this narrow, the GEMV again (N not a multiple of the column tiles)"""
    torch, gw = dev
    from oracle import oracle as orc
    from gwenedeg_amd import synth
    rng = np.random.default_rng(typ * 10 + M)
    N, K = (64, 1024) if M <= 8 else (200, 768)
    sl = synth.synth_library()
    rb = sl.gw_synth_row_bytes(typ, K)
    blocks = np.zeros((N, rb), np.uint8)
    w = rng.normal(0, 0.02, size=(N, K)).astype(np.float32)
    for r in range(N):
        sl.gw_synth_encode_row(typ, blocks[r].ctypes.data, w[r].ctypes.data, K)
    x = rng.normal(0, 1, size=(M, K)).astype(np.float32)
    xq, xs = orc.quantize(x)
    ref = orc.kq_matmul(typ, blocks, xq, xs, N, K)
    out = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    Bd, XQ, XS = (_to_dev(torch, a) for a in (blocks.reshape(-1), xq, xs))
    prev = gw.lib.gw_matmul_tile_rows(tile)
    try:
        assert gw.lib.gw_kq_matmul(out.data_ptr(), typ, Bd.data_ptr(), N, K, XQ.data_ptr(), XS.data_ptr(), M, None) == 0
        torch.cuda.synchronize()
    finally:
        gw.lib.gw_matmul_tile_rows(prev)
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"max diff {np.abs(got - ref).max()}"


@pytest.mark.parametrize("typ", [12, 14])
@pytest.mark.parametrize("K", [2560, 9728])
@pytest.mark.parametrize("M", [9, 20, 32])
@pytest.mark.parametrize("kq16,nqr,sb", [(1, 0, 0), (0, 0, 0), (0, 1, 2), (0, 2, 2), (0, 4, 1), (0, 2, 1)])
def test_kq32_at_the_4b_widths(dev, typ, K, M, kq16, nqr, sb):
    """the 9..32-row K-quant GEMMs (k_gemm_kq16 and k_gemm_kq32: Q4_K, Q6_K) at the Qwen3-4B widths (K = 2560: q / k / v / gate / up,
    K = 9728: down), 1,024 weight rows (1,008: a partial last tile), each split of a tile's activation rows over blocks
    (nqr quads of 8 per block, 0: chosen by the launch) and step width (sb super-blocks per step, 0: chosen): its load
    pipeline in steady state (10 and 38 super-blocks per row against its look-ahead of five), bit for bit against the
    oracle"""
    torch, gw = dev
    from oracle import oracle as orc
    from gwenedeg_amd import synth
    rng = np.random.default_rng(typ * 100 + M + K)
    N = 1008 if nqr == 2 or kq16 else 1024
    sl = synth.synth_library()
    rb = sl.gw_synth_row_bytes(typ, K)
    blocks = np.zeros((N, rb), np.uint8)
    w = rng.normal(0, 0.02, size=(N, K)).astype(np.float32)
    for r in range(N):
        sl.gw_synth_encode_row(typ, blocks[r].ctypes.data, w[r].ctypes.data, K)
    x = rng.normal(0, 1, size=(M, K)).astype(np.float32)
    xq, xs = orc.quantize(x)
    ref = orc.kq_matmul(typ, blocks, xq, xs, N, K)
    out = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    Bd, XQ, XS = (_to_dev(torch, a) for a in (blocks.reshape(-1), xq, xs))
    prev, prev_sb, prev_k = gw.lib.gw_kq32_quads(nqr), gw.lib.gw_kq32_step(sb), gw.lib.gw_kq_small_kernel(kq16)
    try:
        assert gw.lib.gw_kq_matmul(out.data_ptr(), typ, Bd.data_ptr(), N, K, XQ.data_ptr(), XS.data_ptr(), M, None) == 0
        torch.cuda.synchronize()
    finally:
        gw.lib.gw_kq32_quads(prev)
        gw.lib.gw_kq32_step(prev_sb)
        gw.lib.gw_kq_small_kernel(prev_k)
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"max diff {np.abs(got - ref).max()}"


def _topk_rows_case(name, rng):
    """(logits rows x n, k) of a top-k case"""
    if name == "normal_151936":
        return rng.normal(0, 3, size=(3, 151936)).astype(np.float32), 40
    if name == "ties":  # values on a grid of 0.5: long runs of equal values, the k-th inside a tie
        return (np.round(rng.normal(0, 2, size=(4, 20000)) * 2) / 2).astype(np.float32), 64
    if name == "all_equal":  # every key's value digits equal: the index decides, 8 digits
        return np.full((2, 5000), 1.25, np.float32), 33
    if name == "signed_zeros_inf":  # -0 and +0 tie (the lower index first), -inf after every number
        x = np.zeros((2, 3000), np.float32)
        x[:, ::2] = -0.0
        x[0, 100:200] = -np.inf
        x[1, :1500] = -np.inf
        x[1, 2000] = 1.0
        return x, 50
    if name == "short":  # n below 64 x k: chunks of one or two values, empty chunks at the end
        return rng.normal(0, 1, size=(5, 70)).astype(np.float32), 64
    if name == "nan_tail":  # fewer numbers than k: NaN after -inf, the lower index first
        x = rng.normal(0, 1, size=(2, 70)).astype(np.float32)
        x[:, 3::7] = np.nan
        x[1, 0] = -np.inf
        return x, 64
    if name == "max_n":
        return rng.normal(0, 1, size=(1, 262144)).astype(np.float32), 64
    raise KeyError(name)


@pytest.mark.parametrize("name", ["normal_151936", "ties", "all_equal", "signed_zeros_inf", "short", "nan_tail", "max_n"])
def test_topk_rows_order(dev, name):
    """gw_topk_rows (the selection of gw_ctx_topk) against numpy's lexsort on the same rows: the k largest values,
    ties to the lower index, larger first (sampler.c:186-217); the values' bits as in the row (-0 kept)"""
    torch, gw = dev
    rng = np.random.default_rng(len(name))
    x, k = _topk_rows_case(name, rng)
    rows, n = x.shape
    ld = n + 3  # (a row pitch above n)
    xp = np.zeros((rows, ld), np.float32)
    xp[:, :n] = x
    X = _to_dev(torch, xp)
    vals = torch.zeros((rows, k), dtype=torch.float32, device="cuda")
    idx = torch.zeros((rows, k), dtype=torch.int32, device="cuda")
    scr = torch.empty(rows * 32768, dtype=torch.uint8, device="cuda")
    assert gw.lib.gw_topk_rows(X.data_ptr(), n, ld, rows, k, vals.data_ptr(), idx.data_ptr(), scr.data_ptr(), None) == 0
    torch.cuda.synchronize()
    order = np.lexsort((np.arange(n)[None, :].repeat(rows, 0), -x), axis=1)[:, :k]
    assert np.array_equal(idx.cpu().numpy(), order)
    assert np.array_equal(vals.cpu().numpy().view(np.uint32), np.take_along_axis(x, order, 1).view(np.uint32))


def test_topk_rows_refuses(dev):
    """k above 64, k >= n, n above 262144 or ld below n: RQ_ERR_ARG before any launch"""
    torch, gw = dev
    X = torch.zeros(300000, dtype=torch.float32, device="cuda")
    v = torch.zeros(64, dtype=torch.float32, device="cuda")
    i = torch.zeros(64, dtype=torch.int32, device="cuda")
    s = torch.empty(32768, dtype=torch.uint8, device="cuda")
    for n, ld, k in ((1000, 1000, 65), (10, 10, 10), (262145, 262145, 8), (1000, 999, 8), (1000, 1000, 0)):
        assert gw.lib.gw_topk_rows(X.data_ptr(), n, ld, 1, k, v.data_ptr(), i.data_ptr(), s.data_ptr(), None) == -1, (n, ld, k)


@pytest.mark.parametrize("base", [18, 21])
@pytest.mark.parametrize("M,tile", [(1, 0), (5, 0), (20, 0), (40, 32), (100, 64)])
def test_iq3_repacked_matmul_bitexact(dev, base, M, tile):
    """the IQ3 repack (RqModelOpts.repack: IQ3_XXS / IQ3_S held as 4-bit codes, types 0x112 / 0x115) through the
    operator: the file's IQ3 blocks converted on the device, then every dispatch path (batched GEMV, MFMA GEMM with both
    tiles) against the oracle's IQ3 result, bit for bit"""
    torch, gw = dev
    from oracle import oracle as orc
    from gwenedeg_amd import synth
    rng = np.random.default_rng(base * 10 + M)
    N, K = (64, 1024) if M <= 8 else (200, 768)
    sl = synth.synth_library()
    rb = sl.gw_synth_row_bytes(base, K)
    blocks = np.zeros((N, rb), np.uint8)
    w = rng.normal(0, 0.02, size=(N, K)).astype(np.float32)
    for r in range(N):
        sl.gw_synth_encode_row(base, blocks[r].ctypes.data, w[r].ctypes.data, K)
    xq, xs = orc.quantize(rng.normal(0, 1, size=(M, K)).astype(np.float32))
    ref = orc.kq_matmul(base, blocks, xq, xs, N, K)
    out = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    Bd, XQ, XS = (_to_dev(torch, a) for a in (blocks.reshape(-1), xq, xs))
    prev = gw.lib.gw_matmul_tile_rows(tile)
    try:
        assert gw.lib.gw_kq_matmul(out.data_ptr(), 0x100 | base, Bd.data_ptr(), N, K, XQ.data_ptr(), XS.data_ptr(), M,
                                   None) == 0
        torch.cuda.synchronize()
    finally:
        gw.lib.gw_matmul_tile_rows(prev)
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"max diff {np.abs(got - ref).max()}"
