"""Pins the oracle (oracle/oracle.c, the C restatement the GPU is checked against) before it is trusted, on the CPU:

* against the reference itself, compiled from its own sources (oracle/_ref, built by oracle/Makefile where the reference
  tree exists and carried with the repository): the Q8_0 GEMV / GEMM and the K-quant dot on the same int8 inputs, and
  whole forward passes (every logit, bit for bit) on synthetic models;
* where the reference exposes no entry point, against what the mathematics fixes: brute-force integer block sums,
  every fp16 value, IEEE float16 rounding and the reference's saturation, the quantizer's closed form and its
  rounding of exact halves away from zero, float64 exp / attention / RoPE, an independent numpy decoder of the ggml Q3_K /
  Q4_K / Q5_K / Q6_K / Q2_K / IQ4_XS block formats (the published layout);
* the product's host-measured tables (gwenedeg_amd/csrc/gw_exact.c: the reference's rsqrtss / vrcp14ps / libmvec expf
  as the device reproduces them) against the reference's own operations on this host.
The reference's fixtures for this path (tests/golden/logits, dequant) need model files absent here; the golden vectors
written by tests/golden/make_golden.py from oracle/_ref are checked in test_golden_vectors.
"""
import ctypes
import os

import numpy as np
import pytest

from oracle import oracle as orc

HAVE_REF = orc.have_ref()
need_ref = pytest.mark.skipif(not HAVE_REF, reason="oracle/_ref not built (needs the reference's sources at build time)")


def _u32(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ------------------------------------------------------------------------------------------------ formats


def test_fp16_to_f32_every_value():
    """or_fp16_to_f32 (kquants.h:143-156) on all 65536 halves against numpy's exact widening (NaN payloads kept)"""
    L = orc.lib()
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    mine = np.array([L.or_fp16_to_f32(int(v)) for v in h], np.float32)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(_u32(mine)[~nan], _u32(ref)[~nan])
    assert np.isnan(mine[nan]).all()


def test_f32_f16_rounding_and_saturation():
    """or_f32_f16 (forward.c:1325-1344): IEEE round-to-nearest-even like numpy below 65520, the reference's saturation
    to 65504 from there (numpy gives inf), denormal halves, NaN stays NaN"""
    L = orc.lib()
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * s for s in (1e-7, 1e-4, 1.0, 300.0, 6e4)])
    x = np.concatenate([x, np.float32([0.0, -0.0, 65504.0, 65519.99, -65519.99, 5.96e-8, 2.98e-8, 2.99e-8])])
    mine = np.array([L.or_f32_f16(float(v)) for v in x], np.uint16)
    ok = np.abs(x) < 65520.0
    ref = np.zeros(x.size, np.uint16)
    ref[ok] = x[ok].astype(np.float16).view(np.uint16)
    assert np.array_equal(mine[ok], ref[ok])
    big = np.float32([65520.0, 1e6, 3e38, -7e4])
    sat = np.array([L.or_f32_f16(float(v)) for v in big], np.uint16)
    assert list(sat) == [0x7bff, 0x7bff, 0x7bff, 0xfbff]
    n = L.or_f32_f16(float("nan"))
    assert (n & 0x7c00) == 0x7c00 and (n & 0x3ff) != 0


# ----------------------------------------------------------------------------------------------- quantize


def test_quantize_closed_form():
    """or_quantize (forward.c:803-836): scale = max|x| * (1/127), q = trunc(x * (127/max) + copysign(0.49999997));
    the group's extreme maps to +-127, reconstruction within half a step, all-zero groups give q = 0 and scale 0"""
    rng = np.random.default_rng(1)
    x = rng.standard_normal((64, 256)).astype(np.float32) * rng.uniform(0.01, 10, (64, 1)).astype(np.float32)
    x[3, 32:64] = 0.0
    q, s = orc.quantize(x)
    g = x.reshape(64, 8, 32)
    wmax = np.abs(g).max(-1)
    assert np.array_equal(_u32(s), _u32(wmax * np.float32(1 / 127)))
    qa = np.abs(q.reshape(64, 8, 32).astype(np.int32))
    nz = wmax > 0
    assert (qa.max(-1)[nz] == 127).all() and (qa <= 127).all()
    assert (q.reshape(64, 8, 32)[~nz] == 0).all() and (s[~nz] == 0).all()
    err = np.abs(q.reshape(64, 8, 32) * s[..., None].astype(np.float64) - g)
    assert (err <= s[..., None] * 0.5 * (1 + 1e-6) + 1e-30).all()


def test_quantize_rounds_half_away_from_zero():
    """q = trunc(y + copysign(0.49999997, y)) in fp32 (forward.c:804-836, "rounded half away from zero"): exact halves go
    away from zero (0.5 -> 1, 2.5 -> 3: a round-half-even rint gives 0 and 2), values just below a half go down"""
    x = np.zeros(32, np.float32)
    x[0] = 127.0                      # inv = 127 / 127 = 1: y = x
    x[1:10] = [2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 126.5, 1.4999999, -2.4999998]
    q, s = orc.quantize(x[None])
    assert s[0, 0] == np.float32(127.0) * np.float32(1 / 127)
    assert list(q[0, :10]) == [127, 3, 4, -3, -4, 1, -1, 127, 1, -2]


# --------------------------------------------------------------------------------------------- Q8_0 matmul


def _q8_case(rng, M, N, K):
    wq = rng.integers(-127, 128, (N, K), dtype=np.int8)
    ws = np.abs(rng.standard_normal((N, K // 32)) * 1e-3).astype(np.float16).astype(np.float32)
    xq, xs = orc.quantize(rng.standard_normal((M, K)).astype(np.float32))
    return wq, ws, xq, xs


def test_q8_block_sums_brute_force():
    """or_q8_block_sums: the exact int32 sum per (row, column, group) against int64 numpy"""
    rng = np.random.default_rng(2)
    wq, _, xq, _ = _q8_case(rng, 3, 48, 256)
    mine = orc.q8_block_sums(wq, xq)
    ref = np.einsum("ngk,mgk->mng", wq.reshape(48, 8, 32).astype(np.int64), xq.reshape(3, 8, 32).astype(np.int64))
    assert np.array_equal(mine.astype(np.int64), ref)


def test_q8_fold_is_the_group_order():
    """or_q8_matmul = the fold val = val + (ws * xs) * (float) isum, groups in order (forward.c:906-916), rebuilt here
    from the brute-force sums with numpy float32 scalars one operation at a time; and close to float64"""
    rng = np.random.default_rng(3)
    wq, ws, xq, xs = _q8_case(rng, 2, 16, 512)
    out = orc.q8_matmul(wq, ws, xq, xs)
    isum = np.einsum("ngk,mgk->mng", wq.reshape(16, 16, 32).astype(np.int64), xq.reshape(2, 16, 32).astype(np.int64))
    for m in range(2):
        for n in range(16):
            v = np.float32(0)
            for g in range(16):
                v = np.float32(v + np.float32(np.float32(ws[n, g] * xs[m, g]) * np.float32(isum[m, n, g])))
            assert np.float32(out[m, n]).view(np.uint32) == v.view(np.uint32)
    w64 = wq.astype(np.float64) * np.repeat(ws.astype(np.float64), 32, 1)
    x64 = xq.astype(np.float64) * np.repeat(xs.astype(np.float64), 32, 1)
    assert np.allclose(out, x64 @ w64.T, rtol=1e-5, atol=1e-6)


@need_ref
@pytest.mark.parametrize("M", [1, 3, 8, 13])
def test_q8_matmul_vs_reference_kernels(tmp_path, M):
    """or_q8_matmul against the reference's own q8p_gemv_rows (M = 1) / q8p_gemm_item (M > 1), kernels_avx512.h,
    compiled from its sources: bit for bit"""
    rng = np.random.default_rng(10 + M)
    wq, ws, xq, xs = _q8_case(rng, M, 96, 1024)
    ref, _ = orc.run_ref_q8op(str(tmp_path), wq, ws, xq, xs)
    assert np.array_equal(_u32(orc.q8_matmul(wq, ws, xq, xs)), _u32(ref))


# ---------------------------------------------------------------------------------------------- K-quants


def _kq_blocks(typ, N, K, seed):
    from gwenedeg_amd import synth
    lib = synth.synth_library()
    rb = lib.gw_synth_row_bytes(typ, K)
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    out = np.zeros((N, rb), np.uint8)
    for n in range(N):
        lib.gw_synth_encode_row(typ, out[n].ctypes.data_as(ctypes.c_void_p), w[n].ctypes.data_as(ctypes.c_void_p), K)
    return out


def _np_dequant_q4k(b):
    """ggml's dequantize_row_q4_K on one 144-byte block, from the published layout (d, dmin, scales[12], qs[128])"""
    d, dmin = b[0:2].view(np.float16)[0].astype(np.float32), b[2:4].view(np.float16)[0].astype(np.float32)
    sc, qs = b[4:16], b[16:144]

    def scale_min(j):
        if j < 4:
            return int(sc[j]) & 63, int(sc[j + 4]) & 63
        return (int(sc[j + 4]) & 0xF) | ((int(sc[j - 4]) >> 6) << 4), (int(sc[j + 4]) >> 4) | ((int(sc[j]) >> 6) << 4)
    y = np.zeros(256, np.float32)
    for c in range(4):
        q = qs[32 * c:32 * c + 32]
        for half in range(2):
            s, m = scale_min(2 * c + half)
            d1, m1 = np.float32(d * np.float32(s)), np.float32(dmin * np.float32(m))
            nib = (q & 0xF) if half == 0 else (q >> 4)
            y[64 * c + 32 * half:64 * c + 32 * half + 32] = d1 * nib.astype(np.float32) - m1
    return y


def _np_dequant_q6k(b):
    """ggml's dequantize_row_q6_K on one 210-byte block (ql[128], qh[64], int8 scales[16], fp16 d)"""
    ql, qh, sc = b[0:128], b[128:192], b[192:208].view(np.int8)
    d = b[208:210].view(np.float16)[0].astype(np.float32)
    y = np.zeros(256, np.float32)
    for n in range(2):
        l_, h_, s_ = ql[64 * n:], qh[32 * n:], sc[8 * n:]
        for l in range(32):
            i = l // 16
            q = [(int(l_[l]) & 0xF) | (((int(h_[l]) >> 0) & 3) << 4), (int(l_[l + 32]) & 0xF) | (((int(h_[l]) >> 2) & 3) << 4),
                 (int(l_[l]) >> 4) | (((int(h_[l]) >> 4) & 3) << 4), (int(l_[l + 32]) >> 4) | (((int(h_[l]) >> 6) & 3) << 4)]
            for k in range(4):
                y[128 * n + 32 * k + l] = np.float32(d * np.float32(s_[i + 2 * k])) * np.float32(q[k] - 32)
    return y


def _np_dequant_q5k(b):
    """ggml's dequantize_row_q5_K on one 176-byte block (d, dmin, scales[12], qh[32], qs[128]): per 64 values c, the
    nibbles of qs[32 c ..] plus 16 where bit 2 c (low nibbles) / 2 c + 1 (high) of qh[l] is set"""
    d, dmin = b[0:2].view(np.float16)[0].astype(np.float32), b[2:4].view(np.float16)[0].astype(np.float32)
    sc, qh, qs = b[4:16], b[16:48], b[48:176]

    def scale_min(j):
        if j < 4:
            return int(sc[j]) & 63, int(sc[j + 4]) & 63
        return (int(sc[j + 4]) & 0xF) | ((int(sc[j - 4]) >> 6) << 4), (int(sc[j + 4]) >> 4) | ((int(sc[j]) >> 6) << 4)
    y = np.zeros(256, np.float32)
    for c in range(4):
        q = qs[32 * c:32 * c + 32].astype(np.int32)
        for half in range(2):
            s, m = scale_min(2 * c + half)
            d1, m1 = np.float32(d * np.float32(s)), np.float32(dmin * np.float32(m))
            nib = (q & 0xF) if half == 0 else (q >> 4)
            nib = nib + np.where(qh.astype(np.int32) & (1 << (2 * c + half)), 16, 0)
            y[64 * c + 32 * half:64 * c + 32 * half + 32] = d1 * nib.astype(np.float32) - m1
    return y


def _np_dequant_q3k(b):
    """ggml's dequantize_row_q3_K on one 110-byte block (hmask[32], qs[64], scales[12], fp16 d): the 16 6-bit scales
    unpacked as ggml's kmask shuffle on 32-bit words, then per 128 values and shift 2 j the 2-bit quants minus 4 where
    the hmask bit is clear"""
    hm, qs = b[0:32].astype(np.int32), b[32:96].astype(np.int32)
    d = b[108:110].view(np.float16)[0].astype(np.float32)
    aux = [int(v) for v in b[96:108].view(np.uint32)] + [0]
    k1, k2, tmp = 0x03030303, 0x0F0F0F0F, aux[2]
    aux[2] = ((aux[0] >> 4) & k2) | (((tmp >> 4) & k1) << 4)
    aux[3] = ((aux[1] >> 4) & k2) | (((tmp >> 6) & k1) << 4)
    aux[0] = (aux[0] & k2) | (((tmp >> 0) & k1) << 4)
    aux[1] = (aux[1] & k2) | (((tmp >> 2) & k1) << 4)
    scales = np.array(aux, np.uint32).view(np.int8).astype(np.int32)
    y = np.zeros(256, np.float32)
    i, m, o = 0, 1, 0
    for n in range(2):
        q = qs[32 * n:32 * n + 32]
        for j in range(4):
            for half in range(2):
                dl = np.float32(d * np.float32(scales[i] - 32))
                i += 1
                qq = ((q[16 * half:16 * half + 16] >> (2 * j)) & 3) - np.where(hm[16 * half:16 * half + 16] & m, 0, 4)
                y[o:o + 16] = dl * qq.astype(np.float32)
                o += 16
            m <<= 1
    return y


_KV_IQ4NL = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.float32)


def _np_dequant_iq4xs(b):
    """ggml's dequantize_row_iq4_xs on one 136-byte block (fp16 d, u16 scales_h, scales_l[4], qs[128]): group ib's
    6-bit ls from nibble ib % 2 of scales_l[ib / 2] and bits 2 ib .. 2 ib + 1 of scales_h, values d (ls - 32) times the
    code value of the low (first 16) and high (last 16) nibbles of qs[16 ib ..]"""
    d = b[0:2].view(np.float16)[0].astype(np.float32)
    sh = int(b[2:4].view(np.uint16)[0])
    y = np.zeros(256, np.float32)
    for ib in range(8):
        ls = ((int(b[4 + ib // 2]) >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4)
        dl = np.float32(d * np.float32(ls - 32))
        q = b[8 + 16 * ib:8 + 16 * ib + 16].astype(np.int32)
        y[32 * ib:32 * ib + 16] = dl * _KV_IQ4NL[q & 15]
        y[32 * ib + 16:32 * ib + 32] = dl * _KV_IQ4NL[q >> 4]
    return y


def _np_dequant_q2k(b):
    """ggml's dequantize_row_q2_K on one 84-byte block (scales[16], qs[64], fp16 d, fp16 dmin): per 128 values n and
    shift 2 j, the 32 values l take bits 2 j of qs[32 n + l]; sub-block of 16 (scale byte: sc low nibble, m high)"""
    sc, qs = b[0:16].astype(np.int32), b[16:80].astype(np.int32)
    d, dmin = b[80:82].view(np.float16)[0].astype(np.float32), b[82:84].view(np.float16)[0].astype(np.float32)
    y = np.zeros(256, np.float32)
    for n in range(2):
        for j in range(4):
            for l in range(32):
                i = 128 * n + 32 * j + l
                s_ = sc[i // 16]
                dl, ml = np.float32(d * np.float32(s_ & 15)), np.float32(dmin * np.float32(s_ >> 4))
                y[i] = dl * np.float32((qs[32 * n + l] >> (2 * j)) & 3) - ml
    return y


def _iq_grids():
    """the codebooks from their compact codes (gwenedeg_amd/csrc/gw_iq_tables.h, parsed as text), expanded here:
    entry -> array of its 8 (or 4) values"""
    import re
    src = open(os.path.join(os.path.dirname(__file__), "..", "gwenedeg_amd", "csrc", "gw_iq_tables.h")).read()
    tab = {m.group(1): [int(v, 16) for v in re.findall(r"0x[0-9a-f]+", m.group(2))]
           for m in re.finditer(r"static const uint16_t (\w+)\[\d+\] = \{(.*?)\};", src, re.S)}
    a2, a3x = [8, 25, 43], [4, 12, 20, 28, 36, 44, 52, 62]
    g = {}
    for n in ("iq2xxs", "iq2xs", "iq2s"):
        g[n] = np.array([[a2[(c >> 2 * j) & 3] for j in range(8)] for c in tab[f"gw_{n}_codes"]], np.int32)
    g["iq3xxs"] = np.array([[a3x[(c >> 3 * j) & 7] for j in range(4)] for c in tab["gw_iq3xxs_codes"]], np.int32)
    g["iq3s"] = np.array([[2 * ((c >> 3 * j) & 7) + 1 for j in range(4)] for c in tab["gw_iq3s_codes"]], np.int32)
    g["iq1s"] = np.array([[((c >> 2 * j) & 3) - 1 for j in range(8)] for c in tab["gw_iq1s_codes"]], np.int32)
    return g


_GRIDS = None


def _ksigns(s7):
    return s7 | ((bin(s7).count("1") & 1) << 7)


def _np_dequant_cb(typ, b):
    """ggml's dequantize_row_iq2_xxs / iq2_xs / iq2_s / iq3_xxs / iq3_s / iq1_s / iq1_m on one block, from the published
    layouts (fp16 d first, IQ1_M's d in the top nibbles of its 4 scale words): values d * scale * grid * sign, with the
    scale expressions of each type; IQ1: d (2 s + 1) (grid +- 1/8)"""
    global _GRIDS
    if _GRIDS is None:
        _GRIDS = _iq_grids()
    G = _GRIDS
    f32, u16 = np.float32, lambda o: int(b[o:o + 2].view(np.uint16)[0])
    u32 = lambda o: int(b[o:o + 4].view(np.uint32)[0])
    h2f = lambda h: np.array([h], np.uint16).view(np.float16)[0].astype(np.float32)
    y = np.zeros(256, np.float32)
    if typ == 29:
        sc = [u16(48 + 2 * i) for i in range(4)]
        d = h2f((sc[0] >> 12) | ((sc[1] >> 8) & 0xF0) | ((sc[2] >> 4) & 0xF00) | (sc[3] & 0xF000))
    else:
        d = h2f(u16(0))
    for ib in range(8):
        for l in range(4):
            o = 32 * ib + 8 * l
            if typ == 16:
                a0, a1 = u32(2 + 8 * ib), u32(6 + 8 * ib)
                db = f32(f32(d * f32(0.5 + (a1 >> 28))) * f32(0.25))
                gr, sg = G["iq2xxs"][(a0 >> 8 * l) & 255], _ksigns((a1 >> 7 * l) & 127)
            elif typ in (17, 22):
                sc = int(b[(66 if typ == 17 else 74) + ib])
                db = f32(f32(d * f32(0.5 + ((sc >> 4 * (l // 2)) & 15))) * f32(0.25))
                if typ == 17:
                    q = u16(2 + 2 * (4 * ib + l))
                    gr, sg = G["iq2xs"][q & 511], _ksigns(q >> 9)
                else:
                    gr = G["iq2s"][int(b[2 + 4 * ib + l]) | (((int(b[66 + ib]) >> 2 * l) & 3) << 8)]
                    sg = int(b[34 + 4 * ib + l])
            elif typ == 18:
                a = u32(66 + 4 * ib)
                db = f32(f32(d * f32(0.5 + (a >> 28))) * f32(0.5))
                gr = np.concatenate([G["iq3xxs"][int(b[2 + 8 * ib + 2 * l])], G["iq3xxs"][int(b[3 + 8 * ib + 2 * l])]])
                sg = _ksigns((a >> 7 * l) & 127)
            elif typ == 21:
                qh = int(b[66 + ib])
                db = f32(d * f32(1 + 2 * ((int(b[106 + ib // 2]) >> 4 * (ib % 2)) & 15)))
                gr = np.concatenate([G["iq3s"][int(b[2 + 8 * ib + 2 * l]) | (((qh >> 2 * l) & 1) << 8)],
                                     G["iq3s"][int(b[3 + 8 * ib + 2 * l]) | (((qh >> (2 * l + 1)) & 1) << 8)]])
                sg = int(b[74 + 4 * ib + l])
            else:
                if typ == 19:
                    qh = u16(34 + 2 * ib)
                    idx, s3, neg = int(b[2 + 4 * ib + l]) | (((qh >> 3 * l) & 7) << 8), (qh >> 12) & 7, qh & 0x8000
                else:
                    scw = u16(48 + 2 * (ib // 2))
                    q = (int(b[32 + 2 * ib + l // 2]) >> 4 * (l % 2)) & 15
                    idx, s3, neg = int(b[4 * ib + l]) | ((q & 7) << 8), (scw >> (6 * (ib % 2) + 3 * (l // 2))) & 7, q & 8
                dl = f32(d * f32(2 * s3 + 1))
                delta = f32(-0.125 if neg else 0.125)
                y[o:o + 8] = dl * (G["iq1s"][idx].astype(np.float32) + delta)
                continue
            sgn = np.array([-1.0 if (sg >> j) & 1 else 1.0 for j in range(8)], np.float32)
            y[o:o + 8] = (db * gr.astype(np.float32)) * sgn
    return y


_KQ_DEC = {11: (_np_dequant_q3k, 110), 12: (_np_dequant_q4k, 144), 13: (_np_dequant_q5k, 176), 14: (_np_dequant_q6k, 210),
           23: (_np_dequant_iq4xs, 136), 10: (_np_dequant_q2k, 84)}
_CB_BYTES = {16: 66, 17: 74, 22: 82, 18: 98, 21: 110, 19: 50, 29: 56}  # (the codebook i-quants, iquants.h:140-154)
for _t, _n in _CB_BYTES.items():
    _KQ_DEC[_t] = ((lambda t: (lambda blk: _np_dequant_cb(t, blk)))(_t), _n)
_ALL_KQ = [10, 11, 12, 13, 14, 23, 16, 17, 22, 18, 21, 19, 29]


@pytest.mark.parametrize("typ", _ALL_KQ)
def test_kq_dequant_vs_independent_decoder(typ):
    """or_kq_dequant_row (kquants.h:222-251; Q2_K / IQ4_XS iquants.h:224-231, :330-340) against a numpy decoder written
    from ggml's block layout: bit for bit"""
    blk = _kq_blocks(typ, 4, 512, 20 + typ)
    dec, bs = _KQ_DEC[typ]
    for n in range(4):
        mine = orc.kq_dequant_row(typ, blk[n], 512)
        ref = np.concatenate([dec(blk[n][i * bs:(i + 1) * bs]) for i in range(2)])
        assert np.array_equal(_u32(mine), _u32(ref)), f"row {n}"


@need_ref
@pytest.mark.parametrize("typ", sorted(_CB_BYTES) + [23, 10])
def test_iq_dequant_vs_reference(tmp_path, typ):
    """or_kq_dequant_row on the i-quants against the reference's iq_dequant_row (iquants.h:217, compiled from its
    sources: its own codebooks, iq_grids.h) on 1,024 random blocks (32,768 grid lookups: every entry of the largest
    codebook, IQ1's 2,048, drawn with probability 1 - 3e-7): bit for bit. Pins the codebooks"""
    nb = 1024
    blk = _kq_blocks(typ, 1, 256 * nb, 90 + typ)[0]
    mine = orc.kq_dequant_row(typ, blk, 256 * nb)
    ref = orc.run_ref_iq_dequant(str(tmp_path), typ, blk, nb)
    assert np.array_equal(_u32(mine), _u32(ref))


@need_ref
@pytest.mark.parametrize("typ", _ALL_KQ)
@pytest.mark.parametrize("M", [1, 5, 11])
def test_kq_matmul_vs_reference(tmp_path, typ, M):
    """or_kq_matmul (kquants.h:86-109's fold; Q2_K / IQ4_XS iquants.h:49-57's) against the reference's kernels compiled
    from its sources (K-quants: the generic kq_dot; Q2_K / IQ4_XS: iq_rows, the forward's AVX-512 dispatch, 1 row and
    blocks of 8):
    bit for bit; and close to the float64 product of the dequantized rows"""
    N, K = 32, 1024
    blk = _kq_blocks(typ, N, K, 30 + typ + M)
    xq, xs = orc.quantize(np.random.default_rng(M).standard_normal((M, K)).astype(np.float32))
    mine = orc.kq_matmul(typ, blk, xq, xs, N, K)
    ref = orc.run_ref_kq(str(tmp_path), typ, blk, xq, xs, N, K)
    assert np.array_equal(_u32(mine), _u32(ref))
    w = np.stack([orc.kq_dequant_row(typ, blk[n], K) for n in range(N)]).astype(np.float64)
    x = xq.astype(np.float64) * np.repeat(xs.astype(np.float64), 32, 1)
    assert np.allclose(mine, x @ w.T, rtol=1e-4, atol=1e-5)


# ----------------------------------------------------------------------------------- exp, rsqrt, RoPE, SwiGLU


def test_exp_att_accuracy_and_clamp():
    """or_exp_att (forward.c:1301-1321, Cephes): within 2 ulp of exp on [-86, 0]; arguments below -86 clamp to e^-86"""
    L = orc.lib()
    x = np.linspace(-86.0, 0.0, 20001, dtype=np.float32)
    mine = np.array([L.or_exp_att(float(v)) for v in x], np.float32)
    ref = np.exp(x.astype(np.float64)).astype(np.float32)
    assert np.abs(_u32(mine).astype(np.int64) - _u32(ref).astype(np.int64)).max() <= 2
    assert L.or_exp_att(-1000.0) == L.or_exp_att(-86.0) > 0


def test_rsqrt_ref_close_to_ieee():
    """or_rsqrt_ref (the reference's 1.0f / sqrtf: rsqrtss + one Newton step) within 3 ulp of the exact value (the
    estimate's error after one step: 1 / sqrtf itself is off by up to 3 ulp in the reference)"""
    L = orc.lib()
    t = np.exp(np.random.default_rng(4).uniform(-20, 20, 5000)).astype(np.float32)
    mine = np.array([L.or_rsqrt_ref(float(v)) for v in t], np.float32)
    ref = (1.0 / np.sqrt(t.astype(np.float64))).astype(np.float32)
    assert np.abs(_u32(mine).astype(np.int64) - _u32(ref).astype(np.int64)).max() <= 3


def test_rope_row_vs_float64():
    """or_rope_row (forward.c:1248-1264): cos / sin of pos * theta^(-j / (hd/2)) within float32 accuracy"""
    L = orc.lib()
    hd, pos = 128, 777
    cs = np.zeros(hd, np.float32)
    L.or_rope_row(cs.ctypes.data_as(ctypes.c_void_p), hd, pos, ctypes.c_float(np.float32(np.log(1e6))))
    j = np.arange(hd // 2)
    ang = pos * 1e6 ** (-j / (hd // 2))
    assert np.allclose(cs[:64], np.cos(ang), atol=5e-4) and np.allclose(cs[64:], np.sin(ang), atol=5e-4)


def test_product_swiglu_tables_reproduce_the_reference_ops():
    """the product's host-measured SwiGLU tables (gw_exact.c, what the device reads) against the reference's own
    operations on this host (libmvec expf, vrcp14ps + Newton, or_swiglu's host mode): bit for bit"""
    from gwenedeg_amd import LIB_PATH
    L = ctypes.CDLL(LIB_PATH)
    L.gw_swiglu_tab_host.restype = ctypes.c_float
    L.gw_swiglu_tab_host.argtypes = [ctypes.c_float, ctypes.c_float]
    O = orc.lib()
    rng = np.random.default_rng(6)
    for scale in (1e-6, 0.05, 1.0, 8.0, 60.0):
        h = (rng.standard_normal(4096) * scale).astype(np.float32)
        h2 = rng.standard_normal(4096).astype(np.float32)
        ref = h.copy()
        O.or_set_swiglu_host(-1)
        O.or_swiglu(ref.ctypes.data_as(ctypes.c_void_p), h2.ctypes.data_as(ctypes.c_void_p), h.size)
        mine = np.array([L.gw_swiglu_tab_host(float(a), float(b)) for a, b in zip(h, h2)], np.float32)
        assert np.array_equal(_u32(mine), _u32(ref)), f"scale {scale}"
    # the library compared the host's libmvec expf with its published method on every input of the SwiGLU's range
    # (5.1e8 floats) while measuring: on this image they agree everywhere, so the device carries no table of differences
    L.gw_exact_mode.restype = ctypes.c_int
    mode = L.gw_exact_mode()
    if mode & 2:
        assert mode & 4, "this host's libmvec expf differs from its published method somewhere (a table is used)"


# ---------------------------------------------------------------------------------------------- attention


def _att_case(rng, n, nkv=2, hd=128):
    kv_len = (n + 255) // 256 * 256
    kc = np.zeros(kv_len * nkv * hd, np.uint16)
    vc = np.zeros_like(kc)
    K = rng.standard_normal((n, nkv, hd)).astype(np.float16)
    V = rng.standard_normal((n, nkv, hd)).astype(np.float16)
    L = orc.lib()
    for t in range(n):
        for g in range(nkv):
            o = L.or_kv_tile(t, g, nkv, hd)
            kc[o + np.arange(hd) * 16 + t % 16] = K[t, g].view(np.uint16)
            vc[o + (t % 16) * hd + np.arange(hd)] = V[t, g].view(np.uint16)
    return kc, vc, K.astype(np.float64), V.astype(np.float64)


@pytest.mark.parametrize("n", [1, 17, 256, 600])
def test_attention_vs_float64(n):
    """or_attention over the tiled f16 cache (forward.c:1894-1899 layout; one block or several combined) against a
    float64 softmax attention"""
    rng = np.random.default_rng(n)
    hd, scale = 128, np.float32(1 / np.sqrt(128))
    kc, vc, K, V = _att_case(rng, n)
    q = rng.standard_normal(hd).astype(np.float32)
    out = np.zeros(hd, np.float32)
    P = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    orc.lib().or_attention(P(out), P(q), P(kc), P(vc), n, 1, 2, hd, ctypes.c_float(scale))
    s = K[:, 1] @ q.astype(np.float64) * float(scale)
    p = np.exp(s - s.max())
    ref = (p / p.sum()) @ V[:, 1]
    assert np.allclose(out, ref, rtol=2e-5, atol=2e-6)


def test_attention_combine_matches_single_pass():
    """several 256-blocks combined (att_combine) equal, to rounding, the same positions in a float64 single pass; and a
    single block is its own combination (block partial / l)"""
    rng = np.random.default_rng(9)
    n, hd = 700, 128
    kc, vc, K, V = _att_case(rng, n)
    q = rng.standard_normal(hd).astype(np.float32)
    P = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    L = orc.lib()
    scale = np.float32(1 / np.sqrt(128))
    out = np.zeros(hd, np.float32)
    L.or_attention(P(out), P(q), P(kc), P(vc), n, 0, 2, hd, ctypes.c_float(scale))
    o1 = np.zeros(hd + 2, np.float32)
    ml = np.zeros(2, np.float32)
    part = np.zeros(hd, np.float32)
    L.or_attention_block(P(part), P(ml), P(q), P(kc), P(vc), 200, 0, 0, 2, hd, ctypes.c_float(scale))
    direct = np.zeros(hd, np.float32)
    L.or_attention(P(direct), P(q), P(kc), P(vc), 200, 0, 2, hd, ctypes.c_float(scale))
    assert np.array_equal(_u32(direct), _u32(part * np.float32(np.float32(1) / ml[1])))
    s = K[:, 0] @ q.astype(np.float64) * float(scale)
    p = np.exp(s - s.max())
    assert np.allclose(out, (p / p.sum()) @ V[:, 0], rtol=2e-5, atol=2e-6)


# -------------------------------------------------------------------------------------- whole forward pass


@need_ref
@pytest.mark.parametrize("shape,over,n,kvt", [
    ("tiny", {}, 40, 2),
    ("tiny_kq", {}, 20, 2),
    ("tiny_iq4xs", {}, 20, 2),
    ("tiny_q2k", {}, 20, 2),
    ("tiny_iq2_xxs", {}, 20, 2),
    ("tiny_iq2_xs", {}, 20, 2),
    ("tiny_iq2_s", {}, 20, 2),
    ("tiny_iq3_xxs", {}, 20, 2),
    ("tiny_iq3_s", {}, 20, 2),
    ("tiny_iq1_s", {}, 20, 2),
    ("tiny_iq1_m", {}, 20, 2),
    ("qwen3_0_6b", dict(n_layers=3, vocab=4096, tied=0), 12, 2),
    ("tiny", {}, 40, 1),
    ("qwen3_0_6b", dict(n_layers=2, vocab=4096, tied=0), 270, 1),
    ("tiny", {}, 270, 3),
    ("tiny", {}, 270, 8),
    ("tiny", {}, 270, 9),
    ("tiny_hd64", {}, 40, 3),
    ("tiny", {}, 270, 5),
    ("tiny", {}, 270, 6),
    ("tiny", {}, 270, 7),
    ("tiny", {}, 270, 12),
    ("tiny", {}, 270, 13),
    ("tiny", {}, 270, 0),
    ("tiny_hd64", {}, 270, 12),
    ("tiny_hd64", {}, 270, 5),
    ("tiny_kv16", {}, 270, 2),
    ("tiny_kv16", {}, 270, 3),
    ("tiny_kv16", {}, 270, 7),
])
def test_forward_bit_exact_vs_reference(tmp_path, shape, over, n, kvt):
    """or_forward_token position by position against the reference compiled from its sources (rq_prefill with every
    row's logits, ref_driver), on seeded synthetic models: every logit bit for bit. On an AVX-512 host the oracle's
    SwiGLU runs the reference's own vector expf and rcp14; nothing else in the pass depends on the host. kvt: both with
    that KV cache type (runq.h:214: 0 f32, 2 f16, 1 bf16, 3 q8, 8 q4, 9 q4k4: the rotated, quantized caches of
    forward.c:1609-1790; + 4: their bf16 dot-product attention, kernels_avx512.h:1439-1475; 270 positions: two
    attention blocks)"""
    from gwenedeg_amd import synth
    d = dict(synth.SHAPES[shape])
    d.update(over)
    path = str(tmp_path / "m.gguf")
    synth.write_gguf(path, d, seed=1)
    ids = np.random.default_rng(7).integers(0, d["vocab"], n).astype(np.int32)
    _, lg, _, _ = orc.run_ref_driver(path, ids, str(tmp_path / "ref"), threads=4, cap=512, all_logits=True, kv_type=kvt)
    om = orc.Model(path, cap=512)
    s = om.seq(kv_type=kvt)
    for i, t in enumerate(ids):
        mine = s.forward(int(t))
        assert np.array_equal(_u32(mine), _u32(lg[i])), f"position {i}: max diff {np.abs(mine - lg[i]).max()}"


def test_golden_vectors():
    """the oracle against the reference's kernel outputs committed in tests/golden/ref_kernels.npz (written by
    tests/golden/make_golden.py from oracle/_ref): Q8_0 GEMV (M = 1) and GEMM item (M = 6), Q4_K and Q6_K dots, Q2_K
    and the i-quants' matmul and dequantization, bit for bit; holds without the reference's build"""
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_kernels.npz"))
    for M in (1, 6):
        got = orc.q8_matmul(z[f"q8_m{M}_wq"], z[f"q8_m{M}_ws"], z[f"q8_m{M}_xq"], z[f"q8_m{M}_xs"])
        assert np.array_equal(_u32(got), _u32(z[f"q8_m{M}_out"])), f"Q8_0 M={M}"
    for typ in (12, 14):
        blk = z[f"kq{typ}_blk"]
        got = orc.kq_matmul(typ, blk, z[f"kq{typ}_xq"], z[f"kq{typ}_xs"], blk.shape[0], 512)
        assert np.array_equal(_u32(got), _u32(z[f"kq{typ}_out"])), f"type {typ}"
    for typ in orc.IQ_TYPES:  # (Q2_K and the i-quants: the matmul and the dequantization of every block)
        blk = z[f"iq{typ}_blk"]
        got = orc.kq_matmul(typ, blk, z[f"iq{typ}_xq"], z[f"iq{typ}_xs"], blk.shape[0], 512)
        assert np.array_equal(_u32(got), _u32(z[f"iq{typ}_out"])), f"type {typ}"
        dq = orc.kq_dequant_row(typ, blk.reshape(-1), blk.shape[0] * 512)
        assert np.array_equal(_u32(dq), _u32(z[f"iq{typ}_dq"])), f"type {typ} dequant"


@need_ref
@pytest.mark.parametrize("V,k,T,topp", [(1000, 1, 0.8, 0.0), (5000, 7, 1.0, 0.9), (151936, 40, 0.7, 0.95),
                                        (151936, 64, 1.3, 0.0), (4096, 64, 0.5, 0.5)])
def test_sample_topk_vs_reference(tmp_path, V, k, T, topp):
    """gw_sample_topk (the library's host replay of sample_topk on a row's k candidates) against the reference's own
    sample_topk on the full row (oracle/_ref/ref_sample): the same token and RNG state, row after row; candidates in
    the reference's order (larger first, lower index on ties), ties planted"""
    import ctypes
    import gwenedeg_amd as gw
    rng = np.random.default_rng(V + k)
    rows = 12
    x = (rng.standard_normal((rows, V)) * 2).astype(np.float32)
    x[1, 10] = x[1, 20] = x[1, 30] = np.float32(x[1].max() + 1)  # a three-way tie at the top
    x[2, :] = np.float32(0.25)  # a row of equal values
    state = 0x2545F4914F6CDD1D
    ref_tok, ref_state = orc.run_ref_sample(str(tmp_path), x, k, T, topp, state)
    order = np.lexsort((np.arange(V)[None, :].repeat(rows, 0), -x), axis=1)[:, :k]
    st = ctypes.c_ulonglong(state)
    mine = []
    for r in range(rows):
        vals = np.ascontiguousarray(x[r, order[r]], np.float32)
        idx = np.ascontiguousarray(order[r], np.int32)
        t = gw.lib.gw_sample_topk(vals.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                  idx.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), k, T, topp, ctypes.byref(st))
        mine.append(int(t))
    assert mine == ref_tok
    assert st.value == ref_state


def test_sample_topk_argument_checks():
    """gw_sample_topk refuses what sample_topk's candidate array cannot hold (k above 64, below 1), a temperature that
    is not positive, and null pointers, without touching the RNG state; k = 1 returns the first candidate and still
    advances the RNG by one draw, as sample_topk does (sampler.c:186-256)"""
    import ctypes
    import gwenedeg_amd as gw
    v = np.linspace(3, 1, 65).astype(np.float32)
    i = np.arange(100, 165, dtype=np.int32)
    fp, ip = v.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), i.ctypes.data_as(ctypes.POINTER(ctypes.c_int))
    st = ctypes.c_ulonglong(12345)
    for k, T in ((65, 1.0), (0, 1.0), (8, 0.0), (8, -1.0), (8, float("nan"))):
        assert gw.lib.gw_sample_topk(fp, ip, k, T, 0.9, ctypes.byref(st)) == gw.RQ_ERR_ARG
        assert st.value == 12345
    assert gw.lib.gw_sample_topk(None, ip, 8, 1.0, 0.9, ctypes.byref(st)) == gw.RQ_ERR_ARG
    assert gw.lib.gw_sample_topk(fp, ip, 1, 1.0, 0.9, ctypes.byref(st)) == 100
    assert st.value != 12345
