/* The oracle: a plain-C restatement of the reference's (j3k0/gwenedeg) arithmetic for the forward hot path.
 *
 * TEST INFRASTRUCTURE ONLY. tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it as the checker;
 * the product never links, calls or falls back to it.
 *
 * Compiled with -O2 -fno-fast-math -ffp-contract=off (oracle/Makefile): every fp32 operation below is one IEEE
 * operation rounded to nearest, in the order written; fmaf() is written where the reference's definition has a
 * fused multiply-add (the attention's chains: forward.c:1295-1299 with FP_FAST_FMAF on the AVX-512 builds).
 *
 * How each part is pinned (tests/test_oracle.py; every check chosen so that a dropped term, a wrong sign or index or a
 * transposed operand fails it):
 *   fp16 widening: all 65536 halves against numpy; f32_f16: numpy's round-to-nearest-even below 65520, the
 *     reference's saturation above, subnormals, NaN;
 *   quantize: the closed form on random rows, hand-computed half-way cases (round half away from zero), all-zero groups;
 *   Q8_0 fold: per-block int32 sums by integer brute force; the group-order fold rebuilt in numpy float32; the whole
 *     matmul bit for bit against the reference's own compiled kernels (oracle/_ref/ref_q8op: q8p_gemv_rows,
 *     q8p_gemm_item) at M = 1, 3, 8, 13, and against the golden vectors of tests/golden/ref_kernels.npz;
 *   K-quant fold: bit for bit against the reference's kq_dot (ref_q8op kq); the dequantization against an
 *     independent numpy decoder of the Q3_K / Q4_K / Q5_K / Q6_K block formats;
 *   Q2_K and IQ4_XS folds: bit for bit against the reference's iq_rows (ref_q8op iq: its AVX-512 i-quant kernels at 1 row and in
 *     blocks of 8); the dequantization against an independent numpy decoder of the block format;
 *   exp_att: within 2 ulp of expf, the -86 clamp; attention: one block against a float64 softmax, several blocks
 *     against the one-block result (the combine's invariant);
 *   rsqrt (or_rsqrt_ref: the reference's -Ofast 1.0f / sqrtf = rsqrtss + one Newton step): within 3 ulp of IEEE and,
 *     through the whole forward, bit for bit; RoPE: against float64 cos / sin; SwiGLU on AVX-512 hosts (libmvec's
 *     vector expf + vrcp14ps + Newton, the -Ofast lowering of forward.c:1953-1958): against the product's
 *     host-measured tables and, through the whole forward, bit for bit;
 *   the whole forward (or_forward_token): logits bit for bit against the compiled reference (oracle/_ref/ref_driver)
 *     on synthetic Q8_0, Q4_K_M and IQ4_XS models, including a Qwen3-0.6B-shaped model with 3 layers, and with every
 *     KV cache type but f32 (the quantized caches and the bf16 dot-product attention over two key blocks).
 * On a host without AVX-512 the oracle's SwiGLU falls back to the portable form (1 / (1 + expf)); the reference built
 * for such a host lowers the loop to other instructions, so there the SwiGLU is pinned only to tolerance.
 */
#define _GNU_SOURCE
#include <float.h>
#include <immintrin.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"
#include "gw_iq_tables.h" /* (the i-quant codebooks, checked against the reference's own dequantization by the tests) */

#define GS 32
#define ATT_T 16
#define ATT_P 256
#define ATT_DC 32

/* ------------------------------------------------------------------------------------------ formats */

float or_fp16_to_f32(uint16_t h) {
    /* kquants.h:143-156: exact */
    uint32_t sign = (uint32_t)(h & 0x8000) << 16, e = h >> 10 & 0x1f, m = h & 0x3ff, bits;
    if (e == 0x1f) bits = sign | 0x7f800000u | m << 13;
    else if (e) bits = sign | (e + 112) << 23 | m << 13;
    else if (m) {
        float f = (float)m * 5.9604644775390625e-8f;
        memcpy(&bits, &f, 4);
        bits |= sign;
    } else bits = sign;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t or_f32_f16(float f) {
    /* forward.c:1325-1344: round to nearest even, saturating at 65504, subnormals exact, NaN quiet */
    uint32_t u;
    memcpy(&u, &f, 4);
    uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
    uint32_t h;
    if (a > 0x7f800000u) h = 0x7e00u | ((a >> 13) & 0x3ffu);
    else if (a >= 0x477ff000u) h = 0x7bffu;
    else if (a < 0x38800000u) {
        float fs;
        memcpy(&fs, &a, 4);
        h = (uint32_t)rintf(fs * 0x1p24f);
    } else {
        uint32_t n = a - 0x38000000u;
        h = (n + 0xfffu + ((n >> 13) & 1)) >> 13;
    }
    return (uint16_t)(sign | h);
}

/* ------------------------------------------------------------------------------------- quantization */

void or_quantize(int8_t *q, float *s, const float *x, int n) {
    /* forward.c:803-836: s = wmax * (1 / 127), inv = 127 / wmax, q = trunc(v + copysign(0.49999997, v)), v = x * inv;
     * an all-zero group: s = 0, q = 0 */
    for (int g = 0; g < n / GS; g++) {
        const float *xg = x + (size_t)g * GS;
        int8_t *qg = q + (size_t)g * GS;
        float wmax = 0;
        for (int i = 0; i < GS; i++) {
            float v = fabsf(xg[i]);
            if (v > wmax) wmax = v;
        }
        s[g] = wmax * (1.0f / 127.0f);
        if (!(wmax > 0)) {
            memset(qg, 0, GS);
            continue;
        }
        float inv = 127.0f / wmax;
        for (int i = 0; i < GS; i++) {
            float v = xg[i] * inv;
            qg[i] = (int8_t)(int32_t)(v + copysignf(0.49999997f, v));
        }
    }
}

/* ------------------------------------------------------------------------------------------- Q8_0 */

float or_dot_q8(const int8_t *wq, const float *ws, const int8_t *xq, const float *xs, int k) {
    /* forward.c:906-916 (the fold as kernels_avx512.h:157-162 states it): per group an exact int32 sum, then
     * val = val + (ws * xs) * (float) isum, each operation rounded, groups in order */
    float val = 0;
    for (int g = 0; g < k / GS; g++) {
        int32_t isum = 0;
        for (int i = 0; i < GS; i++)
            isum += (int32_t)wq[g * GS + i] * (int32_t)xq[g * GS + i];
        float sc = ws[g] * xs[g];
        float p = sc * (float)isum;
        val = val + p;
    }
    return val;
}

void or_q8_matmul(float *out, const int8_t *wq, const float *ws, const int8_t *xq, const float *xs, int M, int N, int K) {
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++)
            out[(size_t)m * N + n] = or_dot_q8(wq + (size_t)n * K, ws + (size_t)n * (K / GS), xq + (size_t)m * K,
                                               xs + (size_t)m * (K / GS), K);
}

void or_q8_block_sums(int32_t *isum, const int8_t *wq, const int8_t *xq, int M, int N, int K) {
    int G = K / GS;
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++)
            for (int g = 0; g < G; g++) {
                int32_t a = 0;
                for (int i = 0; i < GS; i++)
                    a += (int32_t)wq[(size_t)n * K + g * GS + i] * (int32_t)xq[(size_t)m * K + g * GS + i];
                isum[((size_t)m * N + n) * G + g] = a;
            }
}

void or_q8_from_blocks(int8_t *q, float *s, const uint8_t *blk, size_t nblk) {
    /* model.c:47-59 */
    for (size_t i = 0; i < nblk; i++, blk += 34) {
        uint16_t h;
        memcpy(&h, blk, 2);
        s[i] = or_fp16_to_f32(h);
        memcpy(q + 32 * i, blk + 2, 32);
    }
}

/* ---------------------------------------------------------------------------------------- K-quants */

enum { T_F32 = 0, T_Q8_0 = 8, T_Q2_K = 10, T_Q3_K = 11, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_IQ2_XXS = 16, T_IQ2_XS = 17,
       T_IQ3_XXS = 18, T_IQ1_S = 19, T_IQ3_S = 21, T_IQ2_S = 22, T_IQ4_XS = 23, T_IQ1_M = 29 };
/* the codebook i-quants (iquants.h:12-27) */
#define IS_CB(t) ((t) == T_IQ2_XXS || (t) == T_IQ2_XS || (t) == T_IQ2_S || (t) == T_IQ3_XXS || (t) == T_IQ3_S || \
                  (t) == T_IQ1_S || (t) == T_IQ1_M)
#define IS_KQ(t) (((t) >= T_Q2_K && (t) <= T_Q6_K) || (t) == T_IQ4_XS || IS_CB(t))

/* IQ4_XS's 16 code values (ggml's kvalues_iq4nl, iq_grids.h:1082; iquants.h:28-30) */
static const int8_t kv_iq4nl[16] = { -127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113 };

static uint16_t u16(const uint8_t *p) { uint16_t v; memcpy(&v, p, 2); return v; }

static void q4k_scale_min(const uint8_t *s, int j, int *sc, int *m) {
    /* kquants.h:169-178 (ggml's get_scale_min_k4) */
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 15) | (s[j - 4] >> 6) << 4;
        *m = (s[j + 4] >> 4) | (s[j] >> 6) << 4;
    }
}

static int q4k_q(const uint8_t *b, int i) { return (b[16 + 32 * (i / 64) + i % 32] >> (4 * (i / 32 % 2))) & 15; } /* :180 */

static int q5k_q(const uint8_t *b, int i) { /* kquants.h:185-190: Q4_K's nibble (qs at +48) | bit j of qh[l] << 4 */
    int j = i / 32, l = i % 32;
    return ((b[48 + 32 * (j / 2) + l] >> (4 * (j % 2))) & 15) | ((b[16 + l] >> j) & 1) << 4;
}

static int q6k_q(const uint8_t *b, int i) { /* kquants.h:192-198 */
    int n = i / 128, p = i / 32 % 4, l = i % 32;
    return ((b[64 * n + 32 * (p & 1) + l] >> (4 * (p >> 1))) & 15) | ((b[128 + 32 * n + l] >> (2 * p)) & 3) << 4;
}

static int q3k_q(const uint8_t *b, int i) { /* kquants.h:200-206: q' = q + 4 = 2 bits of qs (+32) | hmask bit i / 32 << 2 */
    int n = i / 128, p = i / 32 % 4, l = i % 32;
    return ((b[32 + 32 * n + l] >> (2 * p)) & 3) | ((b[l] >> (i / 32)) & 1) << 2;
}

static int q3k_scale(const uint8_t *b, int j) { /* kquants.h:207-212: the 6-bit scale (before the - 32) of sub-block j */
    const uint8_t *sc = b + 96;
    return (j < 8 ? sc[j] & 15 : sc[j - 8] >> 4) | ((sc[8 + j % 4] >> (2 * (j / 4))) & 3) << 4;
}

static int kq_bytes(int type) {
    /* kquants.h:9-33; iquants.h:140-154 */
    switch (type) {
    case T_Q4_K: return 144;
    case T_Q5_K: return 176;
    case T_Q3_K: return 110;
    case T_Q2_K: return 84;
    case T_IQ4_XS: return 136;
    case T_IQ2_XXS: return 66;
    case T_IQ2_XS: return 74;
    case T_IQ2_S: return 82;
    case T_IQ3_XXS: return 98;
    case T_IQ3_S: return 110;
    case T_IQ1_S: return 50;
    case T_IQ1_M: return 56;
    }
    return 210;
}

/* ------------------------------------------------------------------ the codebook i-quants (iquants.h:8-57) */

static uint32_t u32le(const uint8_t *p) { uint32_t v; memcpy(&v, p, 4); return v; }
static unsigned ksigns(unsigned s) { return s | (__builtin_popcount(s) & 1u) << 7; } /* iquants.h:9, :197 */

static uint16_t iq1m_d16(const uint8_t *b) { /* iquants.h:200-205: the fp16 d in the 4 scale words' top nibbles */
    uint16_t sc0 = u16(b + 48), sc1 = u16(b + 50), sc2 = u16(b + 52), sc3 = u16(b + 54);
    return (uint16_t)((sc0 >> 12) | ((sc1 >> 8) & 0x00f0) | ((sc2 >> 4) & 0x0f00) | (sc3 & 0xf000));
}

/* group ib (32 values) of a block in its integer form (iquants.h:33-47): v[32], S[h] for the two halves of 16, D */
static void cb_group(int type, const uint8_t *b, int ib, int v[32], int S[2], float *D) {
    if (type == T_IQ2_XXS) { /* a0: 4 grid indices; a1: 4 x 7 sign bits, ls in the top 4 (iquants.h:12-13) */
        uint32_t a0 = u32le(b + 2 + 8 * ib), a1 = u32le(b + 6 + 8 * ib);
        for (int l = 0; l < 4; l++) {
            uint64_t g = gw_iq2_entry(gw_iq2xxs_codes, (int)(a0 >> 8 * l & 255));
            unsigned sg = ksigns(a1 >> 7 * l & 127);
            for (int j = 0; j < 8; j++) v[8 * l + j] = (int)(g >> 8 * j & 255) * (sg >> j & 1 ? -1 : 1);
        }
        S[0] = S[1] = 2 * (int)(a1 >> 28) + 1;
        *D = or_fp16_to_f32(u16(b)) * 0.125f;
    } else if (type == T_IQ2_XS || type == T_IQ2_S) { /* iquants.h:14-17 */
        for (int l = 0; l < 4; l++) {
            uint64_t g;
            unsigned sg;
            if (type == T_IQ2_XS) {
                int q = u16(b + 2 + 2 * (4 * ib + l));
                g = gw_iq2_entry(gw_iq2xs_codes, q & 511);
                sg = ksigns((unsigned)q >> 9);
            } else {
                g = gw_iq2_entry(gw_iq2s_codes, b[2 + 4 * ib + l] | (b[66 + ib] << (8 - 2 * l) & 0x300));
                sg = b[34 + 4 * ib + l];
            }
            for (int j = 0; j < 8; j++) v[8 * l + j] = (int)(g >> 8 * j & 255) * (sg >> j & 1 ? -1 : 1);
        }
        int sc = b[(type == T_IQ2_XS ? 66 : 74) + ib];
        S[0] = 2 * (sc & 15) + 1;
        S[1] = 2 * (sc >> 4) + 1;
        *D = or_fp16_to_f32(u16(b)) * 0.125f;
    } else if (type == T_IQ3_XXS) { /* iquants.h:18-19: qs[8 ib + t] the index of values 4 t ..; then per group a u32 */
        uint32_t a = u32le(b + 66 + 4 * ib);
        for (int l = 0; l < 4; l++) {
            unsigned sg = ksigns(a >> 7 * l & 127);
            for (int hh = 0; hh < 2; hh++) {
                uint32_t g = gw_iq3xxs_entry(b[2 + 8 * ib + 2 * l + hh]);
                for (int j = 0; j < 4; j++) v[8 * l + 4 * hh + j] = (int)(g >> 8 * j & 255) * (sg >> (4 * hh + j) & 1 ? -1 : 1);
            }
        }
        S[0] = S[1] = 2 * (int)(a >> 28) + 1;
        *D = or_fp16_to_f32(u16(b)) * 0.25f;
    } else if (type == T_IQ3_S) { /* iquants.h:20-21: qh bit t of group ib = index bit 8 of step t; raw signs */
        int qh = b[66 + ib];
        for (int l = 0; l < 4; l++) {
            unsigned sg = b[74 + 4 * ib + l];
            for (int hh = 0; hh < 2; hh++) {
                uint32_t g = gw_iq3s_entry(b[2 + 8 * ib + 2 * l + hh] | (qh << (8 - 2 * l - hh) & 256));
                for (int j = 0; j < 4; j++) v[8 * l + 4 * hh + j] = (int)(g >> 8 * j & 255) * (sg >> (4 * hh + j) & 1 ? -1 : 1);
            }
        }
        S[0] = S[1] = 1 + 2 * (b[106 + ib / 2] >> 4 * (ib % 2) & 15);
        *D = or_fp16_to_f32(u16(b));
    } else if (type == T_IQ1_S) { /* iquants.h:22-24: v = 8 grid + (delta < 0 ? -1 : 1) */
        int qh = u16(b + 34 + 2 * ib), dl = qh & 0x8000 ? -1 : 1;
        for (int l = 0; l < 4; l++) {
            uint64_t g = gw_iq1s_entry(b[2 + 4 * ib + l] | (qh >> 3 * l & 7) << 8);
            for (int j = 0; j < 8; j++) v[8 * l + j] = 8 * (int)(int8_t)(g >> 8 * j) + dl;
        }
        S[0] = S[1] = 2 * (qh >> 12 & 7) + 1;
        *D = or_fp16_to_f32(u16(b)) * 0.125f;
    } else { /* IQ1_M, iquants.h:25-27: per chunk of 8 its delta sign; 3-bit scales per 16 */
        int sc = u16(b + 48 + 2 * (ib / 2));
        for (int l = 0; l < 4; l++) {
            int q = b[32 + 2 * ib + l / 2] >> 4 * (l % 2), dl = q & 8 ? -1 : 1;
            uint64_t g = gw_iq1s_entry(b[4 * ib + l] | (q & 7) << 8);
            for (int j = 0; j < 8; j++) v[8 * l + j] = 8 * (int)(int8_t)(g >> 8 * j) + dl;
        }
        S[0] = 2 * (sc >> (6 * (ib % 2)) & 7) + 1;
        S[1] = 2 * (sc >> (6 * (ib % 2) + 3) & 7) + 1;
        *D = or_fp16_to_f32(iq1m_d16(b)) * 0.125f;
    }
}

static void cb_dequant(int type, const uint8_t *b, float *y) {
    /* iquants.h:217-345 (ggml's dequantize_row_*): one block, each type's own expression */
    float d = or_fp16_to_f32(type == T_IQ1_M ? iq1m_d16(b) : u16(b));
    for (int ib = 0; ib < 8; ib++) {
        if (type == T_IQ1_S || type == T_IQ1_M) { /* d (2 s + 1) (grid + delta), delta = +-0.125 */
            for (int l = 0; l < 4; l++) {
                int idx, s3;
                float delta;
                if (type == T_IQ1_S) {
                    int qh = u16(b + 34 + 2 * ib);
                    idx = b[2 + 4 * ib + l] | (qh >> 3 * l & 7) << 8;
                    s3 = qh >> 12 & 7;
                    delta = qh & 0x8000 ? -0.125f : 0.125f;
                } else {
                    int sc = u16(b + 48 + 2 * (ib / 2)), q = b[32 + 2 * ib + l / 2] >> 4 * (l % 2);
                    idx = b[4 * ib + l] | (q & 7) << 8;
                    s3 = sc >> (6 * (ib % 2) + 3 * (l / 2)) & 7;
                    delta = q & 8 ? -0.125f : 0.125f;
                }
                float dl = d * (float)(2 * s3 + 1);
                uint64_t g = gw_iq1s_entry(idx);
                for (int j = 0; j < 8; j++) y[32 * ib + 8 * l + j] = dl * ((float)(int8_t)(g >> 8 * j) + delta);
            }
            continue;
        }
        int v[32], S[2];
        float D;
        cb_group(type, b, ib, v, S, &D); /* (the grid values with their signs; the scales below from the block) */
        for (int i = 0; i < 32; i++) {
            int h = i / 16, gv = v[i] < 0 ? -v[i] : v[i];
            float sg = v[i] < 0 ? -1.f : 1.f, y0;
            if (type == T_IQ2_XXS) /* d (0.5 + ls) 0.25 */
                y0 = d * (0.5f + (float)(u32le(b + 6 + 8 * ib) >> 28)) * 0.25f;
            else if (type == T_IQ2_XS || type == T_IQ2_S) /* d (0.5 + sc) 0.25, sc the nibble of the half */
                y0 = d * (0.5f + (float)(b[(type == T_IQ2_XS ? 66 : 74) + ib] >> 4 * h & 15)) * 0.25f;
            else if (type == T_IQ3_XXS) /* d (0.5 + ls) 0.5 */
                y0 = d * (0.5f + (float)(u32le(b + 66 + 4 * ib) >> 28)) * 0.5f;
            else /* IQ3_S: d (1 + 2 sc) */
                y0 = d * (float)(1 + 2 * (b[106 + ib / 2] >> 4 * (ib % 2) & 15));
            y[32 * ib + i] = y0 * (float)gv * sg;
        }
    }
}

static int q2k_q(const uint8_t *b, int i) { /* iquants.h:10-11: 2 bits 2 (i / 32 % 4) of qs[32 (i / 128) + i % 32] */
    return (b[16 + 32 * (i / 128) + i % 32] >> (2 * (i / 32 % 4))) & 3;
}

static int iq4xs_ls(const uint8_t *b, int ib) { /* iquants.h:28-29: the 6-bit scale of group ib (before the - 32) */
    return ((b[4 + ib / 2] >> (4 * (ib % 2))) & 15) | ((u16(b + 2) >> (2 * ib)) & 3) << 4;
}

static int iq4xs_v(const uint8_t *b, int i) { /* iquants.h:29: value i's code, qs[16 ib + j] low nibble j, high 16 + j */
    int ib = i / 32, l = i % 32;
    return kv_iq4nl[(b[8 + 16 * ib + l % 16] >> (4 * (l / 16))) & 15];
}

void or_kq_dequant_row(int type, const uint8_t *blk, int n, float *y) {
    /* kquants.h:222-251 */
    for (int s = 0; s < n / 256; s++, y += 256) {
        const uint8_t *b = blk + (size_t)s * kq_bytes(type);
        if (type == T_Q4_K || type == T_Q5_K) {
            float d = or_fp16_to_f32(u16(b)), dmin = or_fp16_to_f32(u16(b + 2));
            for (int j = 0; j < 8; j++) {
                int sc, m;
                q4k_scale_min(b + 4, j, &sc, &m);
                float d1 = d * sc, m1 = dmin * m;
                for (int l = 0; l < 32; l++)
                    y[32 * j + l] = d1 * (type == T_Q5_K ? q5k_q(b, 32 * j + l) : q4k_q(b, 32 * j + l)) - m1;
            }
        } else if (type == T_Q3_K) {
            float d = or_fp16_to_f32(u16(b + 108));
            for (int j = 0; j < 16; j++) {
                float dl = d * (float)(q3k_scale(b, j) - 32);
                for (int l = 0; l < 16; l++) y[16 * j + l] = dl * (float)(q3k_q(b, 16 * j + l) - 4);
            }
        } else if (type == T_Q2_K) { /* iquants.h:224-231 (ggml's dequantize_row_q2_K): (d sc) q - dmin m per 16 */
            float d = or_fp16_to_f32(u16(b + 80)), dmin = or_fp16_to_f32(u16(b + 82));
            for (int i = 0; i < 256; i++) {
                float dl = d * (float)(b[i / 16] & 15), ml = dmin * (float)(b[i / 16] >> 4);
                y[i] = dl * (float)q2k_q(b, i) - ml;
            }
        } else if (IS_CB(type)) {
            cb_dequant(type, b, y);
        } else if (type == T_IQ4_XS) { /* iquants.h:330-340 (ggml's dequantize_row_iq4_xs): (d (ls - 32)) v */
            float d = or_fp16_to_f32(u16(b));
            for (int ib = 0; ib < 8; ib++) {
                float dl = d * (float)(iq4xs_ls(b, ib) - 32);
                for (int l = 0; l < 32; l++) y[32 * ib + l] = dl * (float)iq4xs_v(b, 32 * ib + l);
            }
        } else {
            float d = or_fp16_to_f32(u16(b + 208));
            for (int i = 0; i < 256; i++) y[i] = d * (float)(int8_t)b[192 + i / 16] * (float)(q6k_q(b, i) - 32);
        }
    }
}

void or_kq_act_prep(float *xf, const int8_t *xq, const float *xs, int n) {
    /* kquants.h:392-400 */
    for (int g = 0; g < n / 32; g++) {
        int32_t sum = 0;
        for (int i = 0; i < 32; i++) sum += xq[32 * g + i];
        xf[g] = xs[g] * (float)sum;
    }
}

static float kq_dot_row(int type, const uint8_t *row, const int8_t *x, const float *xs, const float *xf, int K) {
    /* the definition, kquants.h:86-109, on the file's blocks of one weight row */
    float val = 0;
    for (int s = 0; s < K / 256; s++) {
        const uint8_t *b = row + (size_t)s * kq_bytes(type);
        for (int j = 0; j < 8; j++) {
            int g = 8 * s + j;
            const int8_t *xg = x + 32 * g;
            if (type == T_Q4_K || type == T_Q5_K) { /* Q5_K: Q4_K's fold with its 5-bit q (kquants.h:95) */
                int sc, m;
                q4k_scale_min(b + 4, j, &sc, &m);
                int32_t isum = 0;
                for (int i = 0; i < 32; i++) isum += (type == T_Q5_K ? q5k_q(b, 32 * j + i) : q4k_q(b, 32 * j + i)) * xg[i];
                float ds = or_fp16_to_f32(u16(b)) * (float)sc, dm = or_fp16_to_f32(u16(b + 2)) * (float)m;
                float a = (ds * xs[g]) * (float)isum;
                float bb = dm * xf[g];
                val = val + (a - bb);
            } else if (type == T_Q3_K) { /* Q6_K's fold with q' - 4 and the signed scales sc - 32 (kquants.h:101-104) */
                int32_t I = 0;
                for (int h = 0; h < 2; h++) {
                    int jj = 2 * j + h;
                    int32_t t = 0, xsum = 0;
                    for (int i = 0; i < 16; i++) {
                        t += q3k_q(b, 16 * jj + i) * xg[16 * h + i];
                        xsum += xg[16 * h + i];
                    }
                    I += (q3k_scale(b, jj) - 32) * (t - 4 * xsum);
                }
                float d = or_fp16_to_f32(u16(b + 108));
                val = val + (d * xs[g]) * (float)I;
            } else if (type == T_Q2_K) { /* iquants.h:49-57: I = sc_0 T_0 + sc_1 T_1, M = m_0 X_0 + m_1 X_1 */
                int32_t I = 0, Mi = 0;
                for (int h = 0; h < 2; h++) {
                    int jj = 2 * j + h;
                    int32_t t = 0, xsum = 0;
                    for (int i = 0; i < 16; i++) {
                        t += q2k_q(b, 16 * jj + i) * xg[16 * h + i];
                        xsum += xg[16 * h + i];
                    }
                    I += (b[jj] & 15) * t;
                    Mi += (b[jj] >> 4) * xsum;
                }
                float d = or_fp16_to_f32(u16(b + 80)), dmin = or_fp16_to_f32(u16(b + 82));
                val = val + ((d * xs[g]) * (float)I - (dmin * xs[g]) * (float)Mi);
            } else if (IS_CB(type)) { /* iquants.h:49-55: I = S_0 T_0 + S_1 T_1 (exact int), val = val + (D xs) I */
                int v[32], S[2];
                float D;
                cb_group(type, b, j, v, S, &D);
                int32_t I = 0;
                for (int h = 0; h < 2; h++) {
                    int32_t t = 0;
                    for (int i = 0; i < 16; i++) t += v[16 * h + i] * xg[16 * h + i];
                    I += S[h] * t;
                }
                val = val + (D * xs[g]) * (float)I;
            } else if (type == T_IQ4_XS) { /* iquants.h:49-55: I = S_0 T_0 + S_1 T_1, S = ls - 32 on both halves, D = d */
                int32_t I = 0, S = iq4xs_ls(b, j) - 32;
                for (int h = 0; h < 2; h++) {
                    int32_t t = 0;
                    for (int i = 0; i < 16; i++) t += iq4xs_v(b, 32 * j + 16 * h + i) * xg[16 * h + i];
                    I += S * t;
                }
                val = val + (or_fp16_to_f32(u16(b)) * xs[g]) * (float)I;
            } else {
                int32_t I = 0;
                for (int h = 0; h < 2; h++) {
                    int jj = 2 * j + h;
                    int32_t t = 0, xsum = 0;
                    for (int i = 0; i < 16; i++) {
                        t += q6k_q(b, 16 * jj + i) * xg[16 * h + i];
                        xsum += xg[16 * h + i];
                    }
                    I += (int32_t)(int8_t)b[192 + jj] * (t - 32 * xsum);
                }
                float d = or_fp16_to_f32(u16(b + 208));
                val = val + (d * xs[g]) * (float)I;
            }
        }
    }
    return val;
}

void or_kq_matmul(int type, float *out, const uint8_t *blocks, const int8_t *xq, const float *xs, int M, int N, int K) {
    size_t rb = (size_t)(K / 256) * kq_bytes(type);
    float *xf = malloc((size_t)(K / 32) * sizeof(float));
    for (int m = 0; m < M; m++) {
        or_kq_act_prep(xf, xq + (size_t)m * K, xs + (size_t)m * (K / 32), K);
        for (int n = 0; n < N; n++)
            out[(size_t)m * N + n] = kq_dot_row(type, blocks + (size_t)n * rb, xq + (size_t)m * K, xs + (size_t)m * (K / 32), xf, K);
    }
    free(xf);
}

/* --------------------------------------------------------------------------------------- attention */

float or_exp_att(float x) {
    /* forward.c:1301-1321 (= att512_exp, kernels_avx512.h:1163-1181): Cephes-style, x clamped at -86 */
    x = x > -86.0f ? x : -86.0f;
    float n = rintf(x * 1.44269504088896341f);
    float r = fmaf(n, -0.693359375f, x);
    r = fmaf(n, 2.12194440e-4f, r);
    float z = r * r;
    float y = 1.9875691500e-4f;
    y = fmaf(y, r, 1.3981999507e-3f);
    y = fmaf(y, r, 8.3334519073e-3f);
    y = fmaf(y, r, 4.1665795894e-2f);
    y = fmaf(y, r, 1.6666665459e-1f);
    y = fmaf(y, r, 5.0000001201e-1f);
    y = fmaf(y, z, r);
    y = y + 1.0f;
    uint32_t bits;
    memcpy(&bits, &y, 4);
    bits += (uint32_t)(int32_t)n << 23;
    memcpy(&y, &bits, 4);
    return y;
}

size_t or_kv_tile(int t, int h, int n_kv, int hd) {
    return (((size_t)(t / ATT_P) * n_kv + h) * ATT_P + (size_t)(t % ATT_P / ATT_T) * ATT_T) * hd;
}

/* The 16-bit caches' layouts inside a tile (forward.c:1901-1951): f16 K at [i][j], V rows [j][i]; bf16 K in dim pairs,
 * dims 2p, 2p + 1 of position j at 32 p + 2 j (+ 1), V rows with dims 32 c + l, 32 c + 16 + l at 32 c + 2 l (+ 1) */
static size_t kv_k_at(int bf, int i, int j) { return bf ? (size_t)(i & ~1) * ATT_T + 2 * j + (i & 1) : (size_t)i * ATT_T + j; }
static size_t kv_v_at(int bf, int i, int j, int hd) {
    return (size_t)j * hd + (bf ? (size_t)((i & ~31) + 2 * (i & 15) + ((i >> 4) & 1)) : (size_t)i);
}
static float kv_f32(int bf, uint16_t h) { /* exact */
    if (!bf) return or_fp16_to_f32(h);
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t or_f32_bf16(float f) {
    /* kernels_avx512.h:60-69: round to nearest even; NaN stays a quiet NaN */
    uint32_t u;
    memcpy(&u, &f, 4);
    uint32_t r = (u + 0x7fffu + ((u >> 16) & 1)) >> 16;
    return (uint16_t)((u & 0x7fffffffu) > 0x7f800000u ? (u >> 16) | 0x40 : r);
}

/* ---- the 8-bit / 4-bit KV caches (RQ_KV_Q8, RQ_KV_Q4, RQ_KV_Q4K4; forward.c:1609-1790). A position's key and value
 * rows are rotated, x' = H D x (D: signs kvq_neg, H: the unnormalized Walsh-Hadamard butterflies in the order h = 1, 2,
 * .., each output one fp32 add or subtract), then quantized per group of 32 dims from the group's values alone:
 *   q8: d = bf16 of max |x'| / 127 with its magnitude rounded up; n = rint(x' (1 / d)) in -127..127
 *   q4: m = the x' of largest |x'| (the first), d = bf16 of m / -8, magnitude rounded up; n = rint(x' (1 / d)) in -8..7
 *   (the reference's source writes x' / d; its build, which parity follows, multiplies by the reciprocal)
 *   (d zero or a bf16 denormal: the group is zero). Read back n d, exact.
 * The attention runs on q' = H D q / hd and the values read back (the fp32 attention), and its output o' comes back as
 * o = D H o' / hd. Tile layouts (16 positions j, hd dims i; the bf16 scales after the codes):
 *   K q8 [i][j] int8, scales at 16 hd: [c][j];  K q4: byte [p][j] = (n_2p + 8) | (n_2p+1 + 8) << 4, scales at 8 hd: [c][j]
 *   V q8 [j][i] int8, scales at 16 hd: [j][c];  V q4: byte [j][c][l] = (n_32c+l + 8) | (n_32c+16+l + 8) << 4, scales at
 *   8 hd: [j][c] */
enum { KVQ_Q8 = 3, KVQ_Q4 = 8, KVQ_Q4K4 = 9, KVQ_F32 = 16 };
/* KVQ_F32: the f32 cache (RQ_KV_F32) kept in the same byte tiles: 64 hd bytes, K [i][j], V [j][i] floats, not rotated
 * (kv_store's fp32 case, forward.c:1945-1950); its attention the fp32 one of the 16-bit caches (forward.c:1827-1857) */
static int kvq_fmt(int kvt, int is_v) { return kvt == KVQ_Q4K4 ? KVQ_Q4 : kvt == KVQ_Q4 && !is_v ? KVQ_Q8 : kvt; }
static size_t kvq_tile_bytes(int fmt, int hd) { return (size_t)hd * (fmt == KVQ_F32 ? 64 : fmt == KVQ_Q4 ? 9 : 17); }
static int kvq_neg(int i) { return (int)(((uint32_t)i * 0x9E3779B9u) >> 31); } /* forward.c:1632 */

static void kvq_rot(float *x, int n, int inv) {
    /* forward.c:1634-1652: x <- H D x, or (inv) D H x */
    if (!inv)
        for (int i = 0; i < n; i++) x[i] = kvq_neg(i) ? -x[i] : x[i];
    for (int h = 1; h < n; h *= 2)
        for (int i0 = 0; i0 < n; i0 += 2 * h)
            for (int i = i0; i < i0 + h; i++) {
                const float a = x[i], b = x[i + h];
                x[i] = a + b;
                x[i + h] = a - b;
            }
    if (inv)
        for (int i = 0; i < n; i++) x[i] = kvq_neg(i) ? -x[i] : x[i];
}

static void kvq_scale_by(float *x, int n) { /* forward.c:1654-1658: times 2^-log2(n), exact */
    const float f = 1.0f / (float)n;
    for (int i = 0; i < n; i++) x[i] = x[i] * f;
}

static uint16_t kvq_scale(float d) {
    /* forward.c:1682-1689: bf16 of d with its magnitude rounded up, the sign kept; 0 for a zero or denormal result */
    uint32_t u;
    memcpy(&u, &d, 4);
    const uint32_t r = (u >> 16) + ((u & 0xffffu) != 0);
    return (r & 0x7f80u) ? (uint16_t)r : 0;
}

static float bf16_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static void kvq_store(int fmt, uint8_t *tile, int j, int hd, const float *x0, int is_v) {
    /* forward.c:1691-1738: row x0 of position j into a q8 / q4 tile (kvq_group per 32 dims, then the layout); an f32
     * tile takes the row as it is */
    if (fmt == KVQ_F32) {
        for (int i = 0; i < hd; i++) memcpy(tile + 4 * (is_v ? (size_t)j * hd + i : (size_t)i * ATT_T + j), &x0[i], 4);
        return;
    }
    float x[256];
    memcpy(x, x0, (size_t)hd * sizeof(float));
    kvq_rot(x, hd, 0);
    const int q4 = fmt == KVQ_Q4, ng = hd / 32;
    uint8_t *sc = tile + (size_t)(q4 ? 8 : 16) * hd;
    for (int c = 0; c < ng; c++) {
        const float *g = x + 32 * c;
        float a = 0.0f, m = 0.0f;
        for (int i = 0; i < 32; i++)
            if (fabsf(g[i]) > a) {
                a = fabsf(g[i]);
                m = g[i];
            }
        const uint16_t s = kvq_scale(q4 ? m / -8.0f : a / 127.0f);
        const float d = bf16_f32(s), r = 1.0f / d;
        int8_t n[32];
        const int lo = q4 ? -8 : -127, hi = q4 ? 7 : 127;
        for (int i = 0; i < 32; i++) {
            /* rint(x' / d) as the reference's build computes it: x' times the one reciprocal 1 / d of the group (the
             * compiled kvq_group divides once and multiplies; the two differ where x' / d lies within an ulp of a half) */
            const float t = s ? rintf(g[i] * r) : 0.0f;
            n[i] = (int8_t)(t < (float)lo ? lo : t > (float)hi ? hi : (int)t);
        }
        const size_t so = 2 * (is_v ? (size_t)j * ng + c : (size_t)c * ATT_T + j);
        memcpy(sc + so, &s, 2);
        for (int l = 0; l < 32; l++) {
            if (!is_v && !q4) tile[(size_t)(32 * c + l) * ATT_T + j] = (uint8_t)n[l];
            if (is_v && !q4) tile[(size_t)j * hd + 32 * c + l] = (uint8_t)n[l];
        }
        for (int l = 0; l < 16; l++) {
            if (!is_v && q4) tile[(size_t)(16 * c + l) * ATT_T + j] = (uint8_t)((n[2 * l] + 8) | (n[2 * l + 1] + 8) << 4);
            if (is_v && q4) tile[(size_t)j * (hd / 2) + 16 * c + l] = (uint8_t)((n[l] + 8) | (n[l + 16] + 8) << 4);
        }
    }
}

static float kvq_val(int fmt, const uint8_t *tile, int i, int j, int hd, int is_v) {
    /* forward.c:1740-1768: dim i of position j read back, n d (exact); an f32 tile's value as stored */
    if (fmt == KVQ_F32) {
        float f;
        memcpy(&f, tile + 4 * (is_v ? (size_t)j * hd + i : (size_t)i * ATT_T + j), 4);
        return f;
    }
    const int q4 = fmt == KVQ_Q4, ng = hd / 32, c = i / 32;
    const uint8_t *sc = tile + (size_t)(q4 ? 8 : 16) * hd;
    uint16_t s;
    memcpy(&s, sc + 2 * (is_v ? (size_t)j * ng + c : (size_t)c * ATT_T + j), 2);
    int n;
    if (!is_v) n = q4 ? ((tile[(size_t)(i / 2) * ATT_T + j] >> (4 * (i & 1))) & 15) - 8 : (int8_t)tile[(size_t)i * ATT_T + j];
    else n = q4 ? ((tile[(size_t)j * (hd / 2) + c * 16 + i % 16] >> (4 * ((i / 16) & 1))) & 15) - 8 : (int8_t)tile[(size_t)j * hd + i];
    return (float)n * bf16_f32(s);
}

/* the cache value of dim i, position t of kv head h (K: is_v 0); kvt 0 / 1: the 16-bit caches (f16 / bf16; c16 the
 * layer's base), else a quantized type (cq the layer's base, tiles of kvq_tile_bytes) */
static float kv_get(int kvt, const uint16_t *c16, const uint8_t *cq, int t, int h, int n_kv, int hd, int i, int is_v) {
    const int j = t % ATT_T;
    if (kvt == 0 || kvt == 1) {
        const uint16_t *tl = c16 + or_kv_tile(t, h, n_kv, hd);
        return kv_f32(kvt, tl[is_v ? kv_v_at(kvt, i, j, hd) : kv_k_at(kvt, i, j)]);
    }
    const int fmt = kvq_fmt(kvt, is_v);
    const size_t nt = or_kv_tile(t, h, n_kv, hd) / ((size_t)ATT_T * hd);
    return kvq_val(fmt, cq + nt * kvq_tile_bytes(fmt, hd), i, j, hd, is_v);
}

static void attention_block_t(int kvt, float *o, float *ml, const float *q, const uint16_t *kc, const uint16_t *vc,
                              const uint8_t *kq, const uint8_t *vq, int n, int b, int h, int n_kv, int hd, float scale) {
    /* attention_vec (forward.c:1346-1403) on block b of kv head h: positions t0 .. t0 + nb - 1; the cache's values read
     * exactly (kv_block_f32, forward.c:1433-1451; the quantized caches: kvq_block_f32, n d), the fp32 attention */
    int t0 = b * ATT_P, nb = n - t0 < ATT_P ? n - t0 : ATT_P;
    float S[ATT_P] = { 0 };
    for (int t = 0; t < nb; t++) {
        float a = 0;
        for (int i0 = 0; i0 < hd; i0 += ATT_DC) {
            float c = 0;
            for (int i = i0; i < i0 + ATT_DC; i++) c = fmaf(q[i], kv_get(kvt, kc, kq, t0 + t, h, n_kv, hd, i, 0), c);
            a = i0 > 0 ? a + c : c;
        }
        S[t] = a * scale;
    }
    float m = S[0];
    for (int t = 1; t < nb; t++)
        if (S[t] > m) m = S[t];
    float sum[ATT_T];
    for (int j = 0; j < ATT_T; j++) sum[j] = 0.0f;
    for (int t = 0; t < (nb + ATT_T - 1) / ATT_T * ATT_T; t++) {
        float e = t < nb ? or_exp_att(S[t] - m) : 0.0f;
        if (t < nb) S[t] = e;
        sum[t % ATT_T] = sum[t % ATT_T] + e;
    }
    for (int w = ATT_T / 2; w >= 1; w /= 2)
        for (int j = 0; j < w; j++) sum[j] = sum[j] + sum[j + w];
    ml[0] = m;
    ml[1] = sum[0];
    for (int i = 0; i < hd; i++) o[i] = 0.0f;
    for (int t = 0; t < nb; t++)
        for (int i = 0; i < hd; i++) o[i] = fmaf(S[t], kv_get(kvt, vc, vq, t0 + t, h, n_kv, hd, i, 1), o[i]);
}

static void attention_block(int bf, float *o, float *ml, const float *q, const uint16_t *kc, const uint16_t *vc, int n, int b,
                            int h, int n_kv, int hd, float scale) {
    attention_block_t(bf, o, ml, q, kc, vc, NULL, NULL, n, b, h, n_kv, hd, scale);
}

void or_attention_block(float *o, float *ml, const float *q, const uint16_t *kc, const uint16_t *vc, int n, int b, int h,
                        int n_kv, int hd, float scale) {
    attention_block(0, o, ml, q, kc, vc, n, b, h, n_kv, hd, scale);
}

void or_att_combine(float *out, int nb, const float *part, size_t stride, int hd) {
    /* forward.c:1405-1431 */
    if (nb == 1) {
        float inv = 1.0f / part[hd + 1];
        for (int i = 0; i < hd; i++) out[i] = part[i] * inv;
        return;
    }
    float M = part[hd];
    for (int b = 1; b < nb; b++)
        if (part[b * stride + hd] > M) M = part[b * stride + hd];
    float L = 0.0f;
    for (int i = 0; i < hd; i++) out[i] = 0.0f;
    for (int b = 0; b < nb; b++) {
        const float *o = part + b * stride;
        float c = or_exp_att(o[hd] - M);
        L = fmaf(c, o[hd + 1], L);
        for (int i = 0; i < hd; i++) out[i] = fmaf(c, o[i], out[i]);
    }
    float inv = 1.0f / L;
    for (int i = 0; i < hd; i++) out[i] = out[i] * inv;
}

/* ---- the bf16 dot-product attention (the KV types with KV_DOT 4: RQ_KV_BF16_DOT 5, RQ_KV_F16_DOT 6, RQ_KV_Q8_DOT 7,
 * RQ_KV_Q4_DOT 12, RQ_KV_Q4K4_DOT 13; kernels_avx512.h:1439-1475, forward.c:1452-1606). q, K, V and the softmax weights
 * rounded to bf16 (vcvtneps2bf16: a denormal input flushed to a zero of its sign, then nearest even); each product pair
 * as vdpbf16ps's lane, two fmas with the odd element first; every operation with denormal inputs read as zero and
 * denormal results flushed (the call's FTZ / DAZ). A bf16-dot cache stores bf16 values, V in position pairs (dim i of
 * positions 2m, 2m + 1 of a tile at 2m hd + 2 i, + 1); an f16-dot cache f16 values, read as bf16 of them; the
 * quantized dot caches their values read back, rounded to bf16 */
static float ftz(float x) { return fabsf(x) < FLT_MIN ? copysignf(0.0f, x) : x; }
static float fma_ftz(float a, float b, float c) { return ftz(fmaf(ftz(a), ftz(b), ftz(c))); }
static float bf16_round(float x) { return bf16_f32(or_f32_bf16(ftz(x))); } /* (kernels_avx512.h:71-77) */
static size_t kv_v_dot_at(int i, int j, int hd) { return (size_t)(j & ~1) * hd + 2 * (size_t)i + (j & 1); }

/* a dot cache's value of dim i, position t as the products read it (K: is_v 0); kt: the full type */
static float kv_get_dot(int kt, const uint16_t *c16, const uint8_t *cq, int t, int h, int n_kv, int hd, int i, int is_v) {
    const int base = kt & ~4, j = t % ATT_T;
    if (base == 1) { /* bf16-dot: K as the bf16 cache, V in position pairs */
        const uint16_t *tl = c16 + or_kv_tile(t, h, n_kv, hd);
        return bf16_f32(tl[is_v ? kv_v_dot_at(i, j, hd) : kv_k_at(1, i, j)]);
    }
    if (base == 2) return bf16_round(kv_get(0, c16, cq, t, h, n_kv, hd, i, is_v)); /* f16-dot */
    return bf16_round(kv_get(base, c16, cq, t, h, n_kv, hd, i, is_v));
}

static void attention_block_dot(int kt, float *o, float *ml, const float *qb, const uint16_t *kc, const uint16_t *vc,
                                const uint8_t *kq, const uint8_t *vq, int n, int b, int h, int n_kv, int hd, float scale) {
    /* attention_vec_dot (forward.c:1488-1549) on block b of kv head h; qb: q rounded to bf16 */
    int t0 = b * ATT_P, nb = n - t0 < ATT_P ? n - t0 : ATT_P;
    float S[ATT_P] = { 0 };
    for (int t = 0; t < nb; t++) {
        float a = 0;
        for (int i0 = 0; i0 < hd; i0 += ATT_DC) {
            float c = 0;
            for (int i = i0; i < i0 + ATT_DC; i += 2) { /* (dim pairs, the odd one first) */
                c = fma_ftz(qb[i + 1], kv_get_dot(kt, kc, kq, t0 + t, h, n_kv, hd, i + 1, 0), c);
                c = fma_ftz(qb[i], kv_get_dot(kt, kc, kq, t0 + t, h, n_kv, hd, i, 0), c);
            }
            a = i0 > 0 ? ftz(a + c) : c;
        }
        S[t] = ftz(a * scale);
    }
    float m = S[0];
    for (int t = 1; t < nb; t++)
        if (S[t] > m) m = S[t];
    float sum[ATT_T];
    for (int j = 0; j < ATT_T; j++) sum[j] = 0.0f;
    for (int t = 0; t < (nb + ATT_T - 1) / ATT_T * ATT_T; t++) {
        const float w = bf16_round(t < nb ? or_exp_att(S[t] - m) : 0.0f);
        if (t < nb) S[t] = w;
        sum[t % ATT_T] = sum[t % ATT_T] + w;
    }
    for (int w = ATT_T / 2; w >= 1; w /= 2)
        for (int j = 0; j < w; j++) sum[j] = sum[j] + sum[j + w];
    ml[0] = m;
    ml[1] = sum[0];
    for (int i = 0; i < hd; i++) o[i] = 0.0f;
    for (int t = 0; t < nb; t += 2) /* (position pairs, the odd one first; past the last: +0, +0) */
        for (int i = 0; i < hd; i++) {
            const float w1 = t + 1 < nb ? S[t + 1] : 0.0f;
            const float v1 = t + 1 < nb ? kv_get_dot(kt, vc, vq, t0 + t + 1, h, n_kv, hd, i, 1) : 0.0f;
            o[i] = fma_ftz(S[t], kv_get_dot(kt, vc, vq, t0 + t, h, n_kv, hd, i, 1), fma_ftz(w1, v1, o[i]));
        }
}

static void attention_t(int kvt, float *out, const float *q, const uint16_t *kc, const uint16_t *vc, const uint8_t *kq,
                        const uint8_t *vq, int n, int h, int n_kv, int hd, float scale) {
    /* attention_kv (forward.c:1871-1892): one block directly, else the partials of every block, combined */
    int nb = (n + ATT_P - 1) / ATT_P;
    size_t st = (size_t)hd + 16;
    float *part = malloc((size_t)nb * st * sizeof(float));
    float qb[256];
    if (kvt & 4) /* (a dot type: q rounded to bf16, forward.c:1599) */
        for (int i = 0; i < hd; i++) qb[i] = bf16_round(q[i]);
    for (int b = 0; b < nb; b++) {
        if (kvt & 4) attention_block_dot(kvt, part + b * st, part + b * st + hd, qb, kc, vc, kq, vq, n, b, h, n_kv, hd, scale);
        else attention_block_t(kvt, part + b * st, part + b * st + hd, q, kc, vc, kq, vq, n, b, h, n_kv, hd, scale);
    }
    or_att_combine(out, nb, part, st, hd);
    free(part);
}

static void attention(int bf, float *out, const float *q, const uint16_t *kc, const uint16_t *vc, int n, int h, int n_kv,
                      int hd, float scale) {
    attention_t(bf, out, q, kc, vc, NULL, NULL, n, h, n_kv, hd, scale);
}

void or_attention(float *out, const float *q, const uint16_t *kc, const uint16_t *vc, int n, int h, int n_kv, int hd,
                  float scale) {
    attention(0, out, q, kc, vc, n, h, n_kv, hd, scale);
}

/* ------------------------------------------------------------------------------- norms, RoPE, SwiGLU */

float or_rsqrt_ref(float t) {
    /* the reference's 1.0f / sqrtf(t) as gcc -Ofast compiles it (forward.c:896, :137): r0 = rsqrtss(t), this host's
     * estimate, then one Newton step r = fma(t r0, r0, -3) (r0 * -0.5) (the constants of our build's object code) */
    float r0 = _mm_cvtss_f32(_mm_rsqrt_ss(_mm_set_ss(t)));
    float b = fmaf(t * r0, r0, -3.0f);
    return b * (r0 * -0.5f);
}

float or_rms_scale(const float *x, int n) {
    /* rmsnorm's scale (forward.c:886-901) in the operation order gcc -Ofast gives the reference (its rmsnorm and every
     * inlined copy): 16 lanes, lane j an fma chain over x[j], x[j + 16], ... from 0; the fixed tree (lanes j + 8, then
     * + 4, + 2, + 1); t = fma(ss, 1 / n, 1e-6) (1 / n an IEEE division); or_rsqrt_ref(t) (n % 16 == 0) */
    float s[16];
    for (int j = 0; j < 16; j++) s[j] = 0.0f;
    for (int j = 0; j < n; j++) s[j % 16] = fmaf(x[j], x[j], s[j % 16]);
    for (int w = 8; w >= 1; w /= 2)
        for (int j = 0; j < w; j++) s[j] = s[j] + s[j + w];
    float inv_n = 1.0f / (float)n;
    float t = fmaf(s[0], inv_n, 1e-6f);
    return or_rsqrt_ref(t);
}

void or_rmsnorm(float *o, const float *x, const float *w, int n) {
    /* forward.c:886-901: o = (w * x) * scale (the compiled order of weight[j] * (ss * x[j])) */
    float r = or_rms_scale(x, n);
    for (int j = 0; j < n; j++) o[j] = (w[j] * x[j]) * r;
}

void or_rope_row(float *cs, int hd, int pos, float log_theta) {
    /* forward.c:1248-1264 with the libm calls of the reference's build there: glibc's scalar expf, and one sincosf
     * for the cosf / sinf pair */
    for (int j = 0; j < hd / 2; j++) {
        float freq = expf(log_theta * (-(float)j / (hd / 2))), c, sn;
        sincosf(pos * freq, &sn, &c);
        cs[j] = c;
        cs[j + hd / 2] = sn;
    }
}

void or_qk_norm_rope(float *v, int n_heads, const float *w, int hd, const float *cs) {
    /* forward.c:1266-1284 (rope_dim = head_dim for Qwen3); the rotation as compiled: x' = fma(x, c, -(y * s)),
     * y' = fma(x, s, y * c) */
    for (int h = 0; h < n_heads; h++) {
        float *q = v + (size_t)h * hd;
        or_rmsnorm(q, q, w, hd);
        for (int j = 0; j < hd / 2; j++) {
            float c = cs[j], s = cs[j + hd / 2], x = q[j], y = q[j + hd / 2];
            float ys = y * s, yc = y * c;
            q[j] = fmaf(x, c, -ys);
            q[j + hd / 2] = fmaf(x, s, yc);
        }
    }
}

float or_silu_exp(float x) {
    /* SiLU's exponential: the reference calls glibc's (vector) expf at min(-h, 80) (forward.c:1953-1958); here the
     * Cephes-style exp of the attention (exp_att) with the argument clamped to [-86, 80] (80: the reference's clamp;
     * below -86, 1 + e rounds to 1 either way) */
    x = x < 80.0f ? x : 80.0f;
    return or_exp_att(x);
}

static int swiglu_host = -1; /* -1: the reference's operations where this host has them (AVX-512) */

void or_set_swiglu_host(int on) { swiglu_host = on; }

__m512 _ZGVeN16v_expf(__m512); /* glibc libmvec: the vector expf gcc calls in the reference's SwiGLU loop */

__attribute__((target("avx512f"))) static void swiglu_host16(float *hb, const float *hb2, int n) {
    /* forward.c:1953-1958 as our build of the reference runs it, 16 values at a time: x = min(-h, 80), e = libmvec
     * expf(x), d = e + 1, r0 = rcp14(d) (this host's estimate), r = (r0 + r0) - (r0 d) r0, out = (h h2) r */
    for (int i = 0; i < n; i += 16) {
        __m512 h = _mm512_loadu_ps(hb + i), h2 = _mm512_loadu_ps(hb2 + i);
        __m512 x = _mm512_min_ps(_mm512_sub_ps(_mm512_setzero_ps(), h), _mm512_set1_ps(80.0f));
        __m512 d = _mm512_add_ps(_ZGVeN16v_expf(x), _mm512_set1_ps(1.0f));
        __m512 p = _mm512_mul_ps(h, h2);
        __m512 r0 = _mm512_rcp14_ps(d);
        __m512 t = _mm512_mul_ps(r0, _mm512_mul_ps(r0, d));
        __m512 r = _mm512_sub_ps(_mm512_add_ps(r0, r0), t);
        _mm512_storeu_ps(hb + i, _mm512_mul_ps(p, r));
    }
}

void or_swiglu(float *hb, const float *hb2, int n) {
    /* forward.c:1953-1958 in the compiled order: (h * h2) * (1 / (1 + e)), e = exp(min(-h, 80)). On an AVX-512 host
     * (default; or_set_swiglu_host(1)): the reference's own operations here, libmvec's vector expf and rcp14 + Newton
     * (n % 16 == 0), which the device reproduces from tables measured on the host. or_set_swiglu_host(0) or no
     * AVX-512: the portable definition, e = or_silu_exp, 1 / (1 + e) an IEEE division */
    if (swiglu_host < 0) swiglu_host = __builtin_cpu_supports("avx512f");
    if (swiglu_host && n % 16 == 0) {
        swiglu_host16(hb, hb2, n);
        return;
    }
    for (int i = 0; i < n; i++) {
        float h = hb[i];
        float e = or_silu_exp(-h);
        float r = 1.0f / (1.0f + e);
        hb[i] = (h * hb2[i]) * r;
    }
}

/* ------------------------------------------------------------------------------------------ model */

typedef struct { int type, rows, cols; const uint8_t *data; } OrMat;

struct OrModel {
    int dim, hidden, L, nh, nkv, hd, vocab, kv_len, cap;
    float log_theta, att_scale;
    uint8_t *file;
    OrMat embd, out, *wq, *wk, *wv, *wo, *w1, *w2, *w3;
    const float *final_norm, **att_norm, **ffn_norm, **q_norm, **k_norm;
};

struct OrSeq {
    const OrModel *m;
    int len, bf; /* bf: a bf16 cache (RQ_KV_BF16), else f16 */
    int qt;      /* a quantized cache: RQ_KV_Q8, RQ_KV_Q4 or RQ_KV_Q4K4 (kq / vq), else 0 (kc / vc) */
    int dot;     /* the bf16 dot-product attention (the type's KV_DOT bit) */
    uint16_t *kc, *vc;
    uint8_t *kq, *vq;
    size_t kq_layer, vq_layer; /* bytes per layer of kq / vq */
};

typedef struct { const char *name; size_t nlen; uint64_t ne[4]; uint32_t nd, type; uint64_t off; } GT;

static int rd(const uint8_t *f, size_t sz, size_t *p, void *dst, size_t n) {
    if (*p + n > sz) return 0;
    memcpy(dst, f + *p, n);
    *p += n;
    return 1;
}

static size_t row_bytes(int type, int k) {
    return type == T_Q8_0 ? (size_t)k / 32 * 34 : IS_KQ(type) ? (size_t)k / 256 * kq_bytes(type) : (size_t)k * 4;
}

OrModel *or_model_load(const char *path, int cap, char *err, size_t errlen) {
    /* a GGUF v3 file as gw_synth writes it (and llama.cpp's qwen3 files): metadata + tensor table, read whole */
#define FAIL(...) do { snprintf(err, errlen, __VA_ARGS__); goto fail; } while (0)
    OrModel *m = calloc(1, sizeof(OrModel));
    GT *T = NULL;
    FILE *fp = fopen(path, "rb");
    if (!m || !fp) { snprintf(err, errlen, "cannot open %s", path); if (fp) fclose(fp); free(m); return NULL; }
    fseek(fp, 0, SEEK_END);
    size_t sz = (size_t)ftell(fp);
    fseek(fp, 0, SEEK_SET);
    m->file = malloc(sz);
    if (!m->file || fread(m->file, 1, sz, fp) != sz) { fclose(fp); FAIL("read failed"); }
    fclose(fp);
    const uint8_t *f = m->file;
    size_t p = 0;
    uint32_t magic, ver;
    uint64_t nt, nkv;
    if (!rd(f, sz, &p, &magic, 4) || magic != 0x46554747u || !rd(f, sz, &p, &ver, 4) || !rd(f, sz, &p, &nt, 8) ||
        !rd(f, sz, &p, &nkv, 8))
        FAIL("not a GGUF file");
    uint64_t align = 32;
    int64_t meta[8] = { 0 };
    float theta = 1e6f;
    static const char *keys[8] = { "qwen3.block_count", "qwen3.embedding_length", "qwen3.feed_forward_length",
                                   "qwen3.attention.head_count", "qwen3.attention.head_count_kv", "qwen3.context_length",
                                   "qwen3.attention.key_length", "general.alignment" };
    static const size_t vsz[13] = { 1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8 };
    for (uint64_t i = 0; i < nkv; i++) {
        uint64_t kl;
        if (!rd(f, sz, &p, &kl, 8) || p + kl > sz) FAIL("bad metadata");
        const char *key = (const char *)f + p;
        p += kl;
        uint32_t ty, aty = 0;
        uint64_t cnt = 1;
        if (!rd(f, sz, &p, &ty, 4)) FAIL("bad metadata");
        size_t vpos = p;
        if (ty == 9) { if (!rd(f, sz, &p, &aty, 4) || !rd(f, sz, &p, &cnt, 8)) FAIL("bad metadata"); }
        uint32_t et = ty == 9 ? aty : ty;
        for (uint64_t j = 0; j < cnt; j++) {
            if (et == 8) { uint64_t sl; if (!rd(f, sz, &p, &sl, 8) || p + sl > sz) FAIL("bad metadata"); p += sl; }
            else if (et < 13 && vsz[et]) p += vsz[et];
            else FAIL("bad metadata type");
        }
        if (ty == 9) continue;
        for (int k = 0; k < 8; k++)
            if (kl == strlen(keys[k]) && !memcmp(key, keys[k], kl)) {
                uint64_t v = 0;
                memcpy(&v, f + vpos, vsz[ty] < 8 ? vsz[ty] : 8);
                meta[k] = (int64_t)v;
            }
        if (kl == 20 && !memcmp(key, "qwen3.rope.freq_base", 20)) memcpy(&theta, f + vpos, 4);
    }
    if (meta[7]) align = (uint64_t)meta[7];
    T = calloc(nt, sizeof(GT));
    for (uint64_t i = 0; i < nt; i++) {
        uint64_t nl;
        if (!rd(f, sz, &p, &nl, 8) || p + nl > sz) FAIL("bad tensor table");
        T[i].name = (const char *)f + p;
        T[i].nlen = nl;
        p += nl;
        if (!rd(f, sz, &p, &T[i].nd, 4) || T[i].nd < 1 || T[i].nd > 4) FAIL("bad tensor table");
        for (uint32_t d = 0; d < 4; d++) {
            T[i].ne[d] = 1;
            if (d < T[i].nd && !rd(f, sz, &p, &T[i].ne[d], 8)) FAIL("bad tensor table");
        }
        if (!rd(f, sz, &p, &T[i].type, 4) || !rd(f, sz, &p, &T[i].off, 8)) FAIL("bad tensor table");
    }
    size_t data = (p + align - 1) / align * align;
    m->L = (int)meta[0]; m->dim = (int)meta[1]; m->hidden = (int)meta[2]; m->nh = (int)meta[3]; m->nkv = (int)meta[4];
    m->hd = meta[6] ? (int)meta[6] : m->dim / m->nh;
    int ctx = (int)meta[5];
    m->cap = cap > 0 && cap < ctx ? cap : ctx;
    m->kv_len = (m->cap + ATT_P - 1) / ATT_P * ATT_P;
    m->log_theta = (float)log((double)theta);
    m->att_scale = or_rsqrt_ref((float)m->hd); /* forward.c:137 as compiled */
    if (m->L < 1 || m->dim < 32 || m->nh < 1 || m->nkv < 1 || m->nh % m->nkv) FAIL("bad hyperparameters");
#define FIND(nm, dst, rows_, cols_) do { int found_ = 0; for (uint64_t i_ = 0; i_ < nt; i_++) { \
        if (T[i_].nlen == strlen(nm) && !memcmp(T[i_].name, nm, T[i_].nlen)) { \
            (dst).type = (int)T[i_].type; (dst).cols = (int)T[i_].ne[0]; (dst).rows = (int)(T[i_].nd > 1 ? T[i_].ne[1] : 1); \
            (dst).data = f + data + T[i_].off; found_ = 1; \
            if ((rows_) && ((dst).rows != (rows_) || (dst).cols != (cols_))) FAIL("tensor %s: bad shape", nm); \
            if (data + T[i_].off + (size_t)(dst).rows * row_bytes((dst).type, (dst).cols) > sz) FAIL("tensor %s truncated", nm); } } \
        if (!found_) FAIL("tensor %s missing", nm); } while (0)
    FIND("token_embd.weight", m->embd, 0, 0);
    m->vocab = m->embd.rows;
    int has_out = 0;
    for (uint64_t i = 0; i < nt; i++) has_out |= T[i].nlen == 13 && !memcmp(T[i].name, "output.weight", 13);
    if (has_out) FIND("output.weight", m->out, m->vocab, m->dim);
    else m->out = m->embd;
    OrMat nv;
    FIND("output_norm.weight", nv, 0, 0);
    m->final_norm = (const float *)nv.data;
    int L = m->L, qd = m->nh * m->hd, kvd = m->nkv * m->hd;
    m->wq = calloc(L, sizeof(OrMat)); m->wk = calloc(L, sizeof(OrMat)); m->wv = calloc(L, sizeof(OrMat));
    m->wo = calloc(L, sizeof(OrMat)); m->w1 = calloc(L, sizeof(OrMat)); m->w2 = calloc(L, sizeof(OrMat));
    m->w3 = calloc(L, sizeof(OrMat));
    m->att_norm = calloc(L, sizeof(float *)); m->ffn_norm = calloc(L, sizeof(float *));
    m->q_norm = calloc(L, sizeof(float *)); m->k_norm = calloc(L, sizeof(float *));
    char nm[96];
    for (int l = 0; l < L; l++) {
        snprintf(nm, sizeof nm, "blk.%d.attn_q.weight", l); FIND(nm, m->wq[l], qd, m->dim);
        snprintf(nm, sizeof nm, "blk.%d.attn_k.weight", l); FIND(nm, m->wk[l], kvd, m->dim);
        snprintf(nm, sizeof nm, "blk.%d.attn_v.weight", l); FIND(nm, m->wv[l], kvd, m->dim);
        snprintf(nm, sizeof nm, "blk.%d.attn_output.weight", l); FIND(nm, m->wo[l], m->dim, qd);
        snprintf(nm, sizeof nm, "blk.%d.ffn_gate.weight", l); FIND(nm, m->w1[l], m->hidden, m->dim);
        snprintf(nm, sizeof nm, "blk.%d.ffn_down.weight", l); FIND(nm, m->w2[l], m->dim, m->hidden);
        snprintf(nm, sizeof nm, "blk.%d.ffn_up.weight", l); FIND(nm, m->w3[l], m->hidden, m->dim);
        snprintf(nm, sizeof nm, "blk.%d.attn_norm.weight", l); FIND(nm, nv, 0, 0); m->att_norm[l] = (const float *)nv.data;
        snprintf(nm, sizeof nm, "blk.%d.ffn_norm.weight", l); FIND(nm, nv, 0, 0); m->ffn_norm[l] = (const float *)nv.data;
        snprintf(nm, sizeof nm, "blk.%d.attn_q_norm.weight", l); FIND(nm, nv, 0, 0); m->q_norm[l] = (const float *)nv.data;
        snprintf(nm, sizeof nm, "blk.%d.attn_k_norm.weight", l); FIND(nm, nv, 0, 0); m->k_norm[l] = (const float *)nv.data;
    }
    free(T);
    return m;
fail:
    free(T);
    or_model_free(m);
    return NULL;
#undef FIND
#undef FAIL
}

void or_model_free(OrModel *m) {
    if (!m) return;
    free(m->file);
    free(m->wq); free(m->wk); free(m->wv); free(m->wo); free(m->w1); free(m->w2); free(m->w3);
    free(m->att_norm); free(m->ffn_norm); free(m->q_norm); free(m->k_norm);
    free(m);
}

void or_model_dims(const OrModel *m, int *d) {
    d[0] = m->dim; d[1] = m->hidden; d[2] = m->L; d[3] = m->nh; d[4] = m->nkv; d[5] = m->hd; d[6] = m->vocab; d[7] = m->kv_len;
}

float or_model_att_scale(const OrModel *m) { return m->att_scale; }

OrSeq *or_seq_new(const OrModel *m) {
    OrSeq *s = calloc(1, sizeof(OrSeq));
    size_t n = (size_t)m->L * m->kv_len * m->nkv * m->hd;
    s->m = m;
    s->kc = calloc(n, 2);
    s->vc = calloc(n, 2);
    if (!s->kc || !s->vc) { or_seq_free(s); return NULL; }
    return s;
}

OrSeq *or_seq_new_kv(const OrModel *m, int bf16) {
    /* a sequence whose cache is bf16 (RQ_KV_BF16: the same tiles, the bf16 layouts) or f16 */
    OrSeq *s = or_seq_new(m);
    if (s) s->bf = bf16 != 0;
    return s;
}

OrSeq *or_seq_new_type(const OrModel *m, int kv_type) {
    /* a sequence of cache type kv_type (runq.h:214): RQ_KV_F32 0, RQ_KV_F16 2, RQ_KV_BF16 1, RQ_KV_Q8 3, RQ_KV_Q4 8,
     * RQ_KV_Q4K4 9, and the dot-product types of all but f32 (+ 4: 5, 6, 7, 12, 13) */
    if (kv_type == 4) return NULL;
    const int base = kv_type & ~4, dot = (kv_type & 4) != 0;
    if (base == 1 || base == 2) {
        OrSeq *s = or_seq_new_kv(m, base == 1);
        if (s) s->dot = dot;
        return s;
    }
    if (base != KVQ_Q8 && base != KVQ_Q4 && base != KVQ_Q4K4 && base != 0) return NULL;
    kv_type = base ? base : KVQ_F32;
    OrSeq *s = calloc(1, sizeof(OrSeq));
    if (!s) return NULL;
    s->dot = dot;
    const size_t tiles = (size_t)m->kv_len / ATT_T * m->nkv;
    s->m = m;
    s->qt = kv_type;
    s->kq_layer = tiles * kvq_tile_bytes(kvq_fmt(kv_type, 0), m->hd);
    s->vq_layer = tiles * kvq_tile_bytes(kvq_fmt(kv_type, 1), m->hd);
    s->kq = calloc((size_t)m->L, s->kq_layer);
    s->vq = calloc((size_t)m->L, s->vq_layer);
    if (!s->kq || !s->vq) { or_seq_free(s); return NULL; }
    return s;
}

void or_seq_free(OrSeq *s) {
    if (!s) return;
    free(s->kc);
    free(s->vc);
    free(s->kq);
    free(s->vq);
    free(s);
}

int or_seq_len(const OrSeq *s) { return s->len; }
void or_seq_truncate(OrSeq *s, int n) { if (n >= 0 && n <= s->len) s->len = n; }
void or_seq_set_len(OrSeq *s, int n) { s->len = n; }

void or_seq_copy(OrSeq *dst, const OrSeq *src, int n) {
    if (src->qt) { /* (the tiles holding positions 0 .. n - 1, whole: later positions are stored before they are read) */
        const size_t tb_k = kvq_tile_bytes(kvq_fmt(src->qt, 0), src->m->hd), tb_v = kvq_tile_bytes(kvq_fmt(src->qt, 1), src->m->hd);
        for (int l = 0; l < src->m->L; l++)
            for (int t = 0; t < n; t += ATT_T)
                for (int h = 0; h < src->m->nkv; h++) {
                    const size_t nt = or_kv_tile(t, h, src->m->nkv, src->m->hd) / ((size_t)ATT_T * src->m->hd);
                    memcpy(dst->kq + l * src->kq_layer + nt * tb_k, src->kq + l * src->kq_layer + nt * tb_k, tb_k);
                    memcpy(dst->vq + l * src->vq_layer + nt * tb_v, src->vq + l * src->vq_layer + nt * tb_v, tb_v);
                }
        dst->len = n;
        return;
    }
    size_t per = (size_t)src->m->kv_len * src->m->nkv * src->m->hd;
    for (int l = 0; l < src->m->L; l++)
        for (int t = 0; t < n; t++)
            for (int h = 0; h < src->m->nkv; h++) {
                size_t o = (size_t)l * per + or_kv_tile(t, h, src->m->nkv, src->m->hd);
                int j = t % ATT_T, hd = src->m->hd, bf = src->bf;
                for (int i = 0; i < hd; i++) {
                    dst->kc[o + kv_k_at(bf, i, j)] = src->kc[o + kv_k_at(bf, i, j)];
                    dst->vc[o + kv_v_at(bf, i, j, hd)] = src->vc[o + kv_v_at(bf, i, j, hd)];
                }
            }
    dst->len = n;
}

const uint16_t *or_seq_cache(const OrSeq *s, int layer, int v) {
    if (s->qt) return NULL;
    return (v ? s->vc : s->kc) + (size_t)layer * s->m->kv_len * s->m->nkv * s->m->hd;
}

const uint8_t *or_seq_cache_q(const OrSeq *s, int layer, int v) {
    /* a quantized cache's layer base (the tiles of kvq_tile_bytes each), else NULL */
    if (!s->qt) return NULL;
    return v ? s->vq + layer * s->vq_layer : s->kq + layer * s->kq_layer;
}
uint16_t *or_seq_cache_mut(OrSeq *s, int layer, int v) {
    return (v ? s->vc : s->kc) + (size_t)layer * s->m->kv_len * s->m->nkv * s->m->hd;
}

static void matvec(float *out, const OrMat *w, const int8_t *xq, const float *xs) {
    /* matvec_rows (forward.c:983-1010) for one activation row: Q8_0 via dot_q8, K-quants via the definition */
    if (w->type == T_Q8_0) {
        int K = w->cols, G = K / 32;
        int8_t *q = malloc((size_t)K);
        float *s = malloc((size_t)G * sizeof(float));
        for (int n = 0; n < w->rows; n++) {
            or_q8_from_blocks(q, s, w->data + (size_t)n * G * 34, (size_t)G);
            out[n] = or_dot_q8(q, s, xq, xs, K);
        }
        free(q);
        free(s);
    } else {
        or_kq_matmul(w->type, out, w->data, xq, xs, 1, w->rows, w->cols);
    }
}

static void embed(float *x, const OrMat *t, int token, int dim) {
    /* embed_row (forward.c:839-881): Q8_0 x = (int8) q * d (one rounding), K-quants by kq_dequant_row */
    if (t->type == T_Q8_0) {
        const uint8_t *blk = t->data + (size_t)token * (dim / 32) * 34;
        for (int g = 0; g < dim / 32; g++, blk += 34) {
            float s = or_fp16_to_f32(u16(blk));
            for (int i = 0; i < 32; i++) x[g * 32 + i] = (float)(int8_t)blk[2 + i] * s;
        }
    } else if (t->type == T_F32) {
        memcpy(x, t->data + (size_t)token * dim * 4, (size_t)dim * 4);
    } else {
        or_kq_dequant_row(t->type, t->data + (size_t)token * row_bytes(t->type, dim), dim, x);
    }
}

int or_forward_token(const OrModel *m, OrSeq *s, int token, float *logits, float *trace) {
    /* decode_step + decode_worker (forward.c:2568-2813) for one row, the operations of each phase in order */
    int dim = m->dim, hd = m->hd, nh = m->nh, nkv = m->nkv, kv_mul = nh / nkv, qd = nh * hd, kvd = nkv * hd;
    int pos = s->len, H = m->hidden;
    if (pos >= m->cap || token < 0 || token >= m->vocab) return -1;
    int xsz = dim > qd ? dim : qd;
    float *x = calloc(dim, 4), *xb = calloc(xsz, 4), *q = calloc(qd, 4), *k = calloc(kvd, 4), *v = calloc(kvd, 4);
    float *hb = calloc(H, 4), *hb2 = calloc(H, 4), *cs = calloc(hd, 4), *att = calloc(qd, 4);
    int8_t *xq = calloc(H > xsz ? H : xsz, 1);
    float *xs = calloc((H > xsz ? H : xsz) / 32, 4);
    embed(x, &m->embd, token, dim);
    or_rope_row(cs, hd, pos, m->log_theta);
    size_t per = (size_t)m->kv_len * kvd;
    for (int l = 0; l < m->L; l++) {
        or_rmsnorm(xb, x, m->att_norm[l], dim);
        or_quantize(xq, xs, xb, dim);
        matvec(q, &m->wq[l], xq, xs);
        matvec(k, &m->wk[l], xq, xs);
        matvec(v, &m->wv[l], xq, xs);
        or_qk_norm_rope(q, nh, m->q_norm[l], hd, cs);
        or_qk_norm_rope(k, nkv, m->k_norm[l], hd, cs);
        if (s->qt) { /* kv_store's quantized rows (forward.c:1907-1913), attention on q' (forward.c:2679, :2712) */
            uint8_t *kq = s->kq + l * s->kq_layer, *vq = s->vq + l * s->vq_layer;
            const int fk = kvq_fmt(s->qt, 0), fv = kvq_fmt(s->qt, 1);
            for (int g = 0; g < nkv; g++) {
                const size_t nt = or_kv_tile(pos, g, nkv, hd) / ((size_t)ATT_T * hd);
                kvq_store(fk, kq + nt * kvq_tile_bytes(fk, hd), pos % ATT_T, hd, k + g * hd, 0);
                kvq_store(fv, vq + nt * kvq_tile_bytes(fv, hd), pos % ATT_T, hd, v + g * hd, 1);
            }
            for (int h = 0; h < nh; h++) {
                float qr[256];
                memcpy(qr, q + h * hd, (size_t)hd * sizeof(float));
                if (s->qt != KVQ_F32) {
                    kvq_rot(qr, hd, 0);
                    kvq_scale_by(qr, hd);
                }
                attention_t(s->qt | (s->dot ? 4 : 0), att + h * hd, qr, NULL, NULL, kq, vq, pos + 1, h / kv_mul, nkv, hd,
                            m->att_scale);
                if (s->qt != KVQ_F32) {
                    kvq_rot(att + h * hd, hd, 1);
                    kvq_scale_by(att + h * hd, hd);
                }
            }
        } else {
        uint16_t *kc = s->kc + (size_t)l * per, *vc = s->vc + (size_t)l * per;
        for (int g = 0; g < nkv; g++) { /* kv_store (forward.c:1901-1951), f16 or bf16, rounded to nearest even */
            size_t o = or_kv_tile(pos, g, nkv, hd);
            int j = pos % ATT_T, bf = s->bf;
            for (int i = 0; i < hd; i++) { /* (a bf16-dot cache: V in position pairs, forward.c:1916-1924) */
                kc[o + kv_k_at(bf, i, j)] = bf ? or_f32_bf16(k[g * hd + i]) : or_f32_f16(k[g * hd + i]);
                vc[o + (bf && s->dot ? kv_v_dot_at(i, j, hd) : kv_v_at(bf, i, j, hd))] =
                    bf ? or_f32_bf16(v[g * hd + i]) : or_f32_f16(v[g * hd + i]);
            }
        }
        for (int h = 0; h < nh; h++) /* (the dot types: kt = 1 / 2 | 4) */
            attention_t(s->dot ? (s->bf ? 1 : 2) | 4 : s->bf, att + h * hd, q + h * hd, kc, vc, NULL, NULL, pos + 1, h / kv_mul,
                        nkv, hd, m->att_scale);
        }
        or_quantize(xq, xs, att, qd);
        matvec(xb, &m->wo[l], xq, xs);
        for (int i = 0; i < dim; i++) x[i] += xb[i];
        or_rmsnorm(xb, x, m->ffn_norm[l], dim);
        or_quantize(xq, xs, xb, dim);
        matvec(hb, &m->w1[l], xq, xs);
        matvec(hb2, &m->w3[l], xq, xs);
        or_swiglu(hb, hb2, H);
        or_quantize(xq, xs, hb, H);
        matvec(xb, &m->w2[l], xq, xs);
        for (int i = 0; i < dim; i++) x[i] += xb[i];
        if (trace) memcpy(trace + (size_t)l * dim, x, (size_t)dim * 4);
    }
    if (logits) {
        or_rmsnorm(x, x, m->final_norm, dim);
        or_quantize(xq, xs, x, dim);
        matvec(logits, &m->out, xq, xs);
    }
    s->len = pos + 1;
    free(x); free(xb); free(q); free(k); free(v); free(hb); free(hb2); free(cs); free(att); free(xq); free(xs);
    return 0;
}
