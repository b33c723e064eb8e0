/* Seeded synthetic Qwen3-shaped GGUF files (random-init weights) for the parity tests and the benchmark.
 *
 * Every matmul tensor is N(0, std) before quantization (std 0.02), the norms are a constant (1.0), the
 * metadata is what the reference's GGUF reader checks for a qwen3 file (gguf.c:230-336: block_count,
 * embedding_length, feed_forward_length, head counts, context_length, key/value length, rope.freq_base,
 * layer_norm_rms_epsilon 1e-6) and the tensor names are llama.cpp's (model.c:269-299). A tokenizer block only where
 * cfg->tokenizer asks for one (a small byte-level BPE vocabulary, below); without it readers load the file without a
 * tokenizer (RqModelOpts.no_tokenizer).
 *
 * Values: row r of tensor t draws from its own splitmix64 stream seeded by (seed, t, r), Box-Muller in
 * double precision, so a file is a pure function of (shape, types, seed) whatever the thread count.
 * Encoders (ggml block formats, restated; the layouts are the ones kquants.h:9-33 documents):
 *   Q8_0: d = amax / 127 (fp16), q = round(x / d) clamped to [-127, 127]
 *   Q4_K: 8 sub-blocks of 32, per sub-block scale / offset from its range, 6-bit sc and m against d / dmin
 *   Q6_K: 16 sub-blocks of 16, int8 sub-scales against d, q in 0..63 (value q - 32)
 *   Q5_K: as Q4_K with q in 0..31 (bit 4 in qh)
 *   Q3_K: 16 sub-blocks of 16, 6-bit scales sc (value (d (sc - 32)) q) with sc - 32 in 0..31 here, q in -4..3
 *   Q2_K (iquants.h:10-11): 16 sub-blocks of 16, 4-bit scale sc and min m per sub-block (value (d sc) q - dmin m),
 *     q in 0..3
 *   IQ4_XS (iquants.h:28-30): 8 groups of 32, 6-bit ls (value (d (ls - 32)) kvalues_iq4nl[q]) with ls - 32 in 0..31
 *     for even groups and -31..0 for odd ones (both signs of the scale), q the nearest of the 16 code values
 *   the codebook i-quants IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ1_S, IQ1_M (iquants.h:12-27): every grid index,
 *     sign bit, scale and delta drawn uniformly from a stream seeded by the row's values (so every codebook entry and
 *     sign pattern occurs), then d set so the block's rms equals the values' (a search for the nearest codebook
 *     entries would not change what the parity tests check)
 * Any valid block decodes the same way on both sides, so these simple encoders suffice for parity. */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "gw_synth.h"
#include "gw_iq_tables.h"

enum { T_F32 = 0, T_Q8_0 = 8, T_Q2_K = 10, T_Q3_K = 11, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14, T_IQ2_XXS = 16, T_IQ2_XS = 17,
       T_IQ3_XXS = 18, T_IQ1_S = 19, T_IQ3_S = 21, T_IQ2_S = 22, T_IQ4_XS = 23, T_IQ1_M = 29 };
#define IS_CB(t) ((t) == T_IQ2_XXS || (t) == T_IQ2_XS || (t) == T_IQ2_S || (t) == T_IQ3_XXS || (t) == T_IQ3_S || \
                  (t) == T_IQ1_S || (t) == T_IQ1_M)
#define IS_SB(t) (((t) >= T_Q2_K && (t) <= T_Q6_K) || (t) == T_IQ4_XS || IS_CB(t)) /* (super-blocks of 256) */

/* bytes per super-block of the codebook i-quants (iquants.h:140-154) */
static int cb_bytes(int t) {
    return t == T_IQ2_XXS ? 66 : t == T_IQ2_XS ? 74 : t == T_IQ2_S ? 82 : t == T_IQ3_XXS ? 98 : t == T_IQ3_S ? 110
         : t == T_IQ1_S ? 50 : 56;
}

/* IQ4_XS's code values (ggml's kvalues_iq4nl) */
static const int8_t kv_iq4nl[16] = { -127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113 };

static uint16_t f32_to_f16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to inf */
    if (a < 0x38800000u) { /* subnormal half: m * 2^-24 */
        float af;
        memcpy(&af, &a, 4);
        return (uint16_t)(sign | (uint32_t)nearbyintf(af * 16777216.0f));
    }
    uint32_t n = a - 0x38000000u;
    return (uint16_t)(sign | ((n + 0xfffu + ((n >> 13) & 1)) >> 13));
}

static float f16_to_f32(uint16_t h) {
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

static uint64_t splitmix(uint64_t *s) {
    uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

static void normal_row(float *y, int n, uint64_t seed, uint64_t tensor, uint64_t row, float std) {
    uint64_t s = seed * 0x2545f4914f6cdd1dull ^ (tensor + 1) * 0x9e3779b97f4a7c15ull ^ (row + 1) * 0xd1b54a32d192ed03ull;
    splitmix(&s);
    for (int i = 0; i < n; i += 2) {
        double u1 = ((splitmix(&s) >> 11) + 1.0) * (1.0 / 9007199254740992.0); /* (0, 1] */
        double u2 = (splitmix(&s) >> 11) * (1.0 / 9007199254740992.0);
        double r = sqrt(-2.0 * log(u1)), th = 6.283185307179586 * u2;
        y[i] = (float)(std * r * cos(th));
        if (i + 1 < n) y[i + 1] = (float)(std * r * sin(th));
    }
}

size_t gw_synth_row_bytes(int type, int k) {
    if (type == T_Q8_0) return (size_t)k / 32 * 34;
    if (type == T_Q4_K) return (size_t)k / 256 * 144;
    if (type == T_Q5_K) return (size_t)k / 256 * 176;
    if (type == T_Q3_K) return (size_t)k / 256 * 110;
    if (type == T_Q6_K) return (size_t)k / 256 * 210;
    if (type == T_IQ4_XS) return (size_t)k / 256 * 136;
    if (type == T_Q2_K) return (size_t)k / 256 * 84;
    if (IS_CB(type)) return (size_t)k / 256 * (size_t)cb_bytes(type);
    return (size_t)k * 4;
}

static void enc_q8_0(uint8_t *o, const float *x, int k) {
    for (int g = 0; g < k / 32; g++, o += 34, x += 32) {
        float amax = 0;
        for (int i = 0; i < 32; i++) amax = fabsf(x[i]) > amax ? fabsf(x[i]) : amax;
        float d = amax / 127.0f, id = d > 0 ? 1.0f / d : 0.0f;
        uint16_t h = f32_to_f16_rne(d);
        memcpy(o, &h, 2);
        for (int i = 0; i < 32; i++) {
            float v = roundf(x[i] * id);
            v = v > 127 ? 127 : v < -127 ? -127 : v;
            o[2 + i] = (uint8_t)(int8_t)v;
        }
    }
}

static void enc_q45_k(uint8_t *o, const float *x, int k, int q5) {
    /* Q4_K (q5 = 0: 144-byte blocks, q 0..15) or Q5_K (176 bytes, q 0..31: the 5th bit in qh, the nibbles at +48) */
    const int qmax = q5 ? 31 : 15, bytes = q5 ? 176 : 144, qs = q5 ? 48 : 16;
    for (int sb = 0; sb < k / 256; sb++, o += bytes, x += 256) {
        float sc[8], mn[8], smax = 0, mmax = 0;
        for (int j = 0; j < 8; j++) {
            float lo = x[32 * j], hi = x[32 * j];
            for (int i = 1; i < 32; i++) {
                lo = x[32 * j + i] < lo ? x[32 * j + i] : lo;
                hi = x[32 * j + i] > hi ? x[32 * j + i] : hi;
            }
            if (lo > 0) lo = 0; /* w = s * q - m with m >= 0 */
            sc[j] = (hi - lo) / (float)qmax;
            mn[j] = -lo;
            smax = sc[j] > smax ? sc[j] : smax;
            mmax = mn[j] > mmax ? mn[j] : mmax;
        }
        uint16_t hd = f32_to_f16_rne(smax / 63.0f), hm = f32_to_f16_rne(mmax / 63.0f);
        float d = f16_to_f32(hd), dmin = f16_to_f32(hm);
        int isc[8], im[8];
        for (int j = 0; j < 8; j++) {
            int a = d > 0 ? (int)lroundf(sc[j] / d) : 0, b = dmin > 0 ? (int)lroundf(mn[j] / dmin) : 0;
            isc[j] = a < 0 ? 0 : a > 63 ? 63 : a;
            im[j] = b < 0 ? 0 : b > 63 ? 63 : b;
        }
        memcpy(o, &hd, 2);
        memcpy(o + 2, &hm, 2);
        uint8_t *s = o + 4;
        for (int j = 0; j < 4; j++) {
            s[j] = (uint8_t)((isc[j] & 63) | (isc[j + 4] >> 4) << 6);
            s[j + 4] = (uint8_t)((im[j] & 63) | (im[j + 4] >> 4) << 6);
            s[j + 8] = (uint8_t)((isc[j + 4] & 15) | (im[j + 4] & 15) << 4);
        }
        uint8_t q[256];
        for (int j = 0; j < 8; j++) {
            float ds = d * isc[j], dm = dmin * im[j];
            for (int i = 0; i < 32; i++) {
                int v = ds > 0 ? (int)lroundf((x[32 * j + i] + dm) / ds) : 0;
                q[32 * j + i] = (uint8_t)(v < 0 ? 0 : v > qmax ? qmax : v);
            }
        }
        for (int c = 0; c < 4; c++)
            for (int l = 0; l < 32; l++)
                o[qs + 32 * c + l] = (uint8_t)((q[64 * c + l] & 15) | (q[64 * c + 32 + l] & 15) << 4);
        if (q5) {
            for (int l = 0; l < 32; l++) {
                uint8_t h = 0;
                for (int j = 0; j < 8; j++) h |= (uint8_t)(((q[32 * j + l] >> 4) & 1) << j);
                o[16 + l] = h;
            }
        }
    }
}

static void enc_q3_k(uint8_t *o, const float *x, int k) {
    for (int sb = 0; sb < k / 256; sb++, o += 110, x += 256) {
        float ss[16], smax = 0;
        for (int j = 0; j < 16; j++) {
            float amax = 0;
            for (int i = 0; i < 16; i++) amax = fabsf(x[16 * j + i]) > amax ? fabsf(x[16 * j + i]) : amax;
            ss[j] = amax / 4.0f;
            smax = ss[j] > smax ? ss[j] : smax;
        }
        uint16_t hd = f32_to_f16_rne(smax / 31.0f);
        float d = f16_to_f32(hd);
        int isc[16];
        uint8_t q[256]; /* q' = q + 4, 0..7 */
        for (int j = 0; j < 16; j++) {
            int a = d > 0 ? (int)lroundf(ss[j] / d) : 0;
            isc[j] = a < 0 ? 0 : a > 31 ? 31 : a;
            float dl = d * (float)isc[j];
            for (int i = 0; i < 16; i++) {
                int v = dl > 0 ? (int)lroundf(x[16 * j + i] / dl) : 0;
                v = v < -4 ? -4 : v > 3 ? 3 : v;
                q[16 * j + i] = (uint8_t)(v + 4);
            }
        }
        memset(o, 0, 110);
        for (int i = 0; i < 256; i++) {
            int n = i / 128, p = i / 32 % 4, l = i % 32;
            o[32 + 32 * n + l] |= (uint8_t)((q[i] & 3) << (2 * p));
            o[l] |= (uint8_t)(((q[i] >> 2) & 1) << (i / 32));
        }
        uint8_t *sc = o + 96;
        for (int j = 0; j < 16; j++) {
            int v = isc[j] + 32; /* the stored 6-bit scale */
            if (j < 8) sc[j] |= (uint8_t)(v & 15);
            else sc[j - 8] |= (uint8_t)((v & 15) << 4);
            sc[8 + j % 4] |= (uint8_t)(((v >> 4) & 3) << (2 * (j / 4)));
        }
        memcpy(o + 108, &hd, 2);
    }
}

static void enc_q6_k(uint8_t *o, const float *x, int k) {
    for (int sb = 0; sb < k / 256; sb++, o += 210, x += 256) {
        float ss[16], smax = 0;
        for (int j = 0; j < 16; j++) {
            float amax = 0;
            for (int i = 0; i < 16; i++) amax = fabsf(x[16 * j + i]) > amax ? fabsf(x[16 * j + i]) : amax;
            ss[j] = amax / 31.0f;
            smax = ss[j] > smax ? ss[j] : smax;
        }
        uint16_t hd = f32_to_f16_rne(smax / 127.0f);
        float d = f16_to_f32(hd);
        int8_t isc[16];
        uint8_t q[256];
        for (int j = 0; j < 16; j++) {
            int a = d > 0 ? (int)lroundf(ss[j] / d) : 0;
            isc[j] = (int8_t)(a > 127 ? 127 : a < 0 ? 0 : a);
            float ds = d * isc[j];
            for (int i = 0; i < 16; i++) {
                int v = ds > 0 ? (int)lroundf(x[16 * j + i] / ds) + 32 : 32;
                q[16 * j + i] = (uint8_t)(v < 0 ? 0 : v > 63 ? 63 : v);
            }
        }
        uint8_t *ql = o, *qh = o + 128;
        for (int n = 0; n < 2; n++)
            for (int l = 0; l < 32; l++) {
                const uint8_t *qq = q + 128 * n;
                ql[64 * n + l] = (uint8_t)((qq[l] & 15) | (qq[64 + l] & 15) << 4);
                ql[64 * n + 32 + l] = (uint8_t)((qq[32 + l] & 15) | (qq[96 + l] & 15) << 4);
                qh[32 * n + l] = (uint8_t)((qq[l] >> 4) | (qq[32 + l] >> 4) << 2 | (qq[64 + l] >> 4) << 4 | (qq[96 + l] >> 4) << 6);
            }
        memcpy(o + 192, isc, 16);
        memcpy(o + 208, &hd, 2);
    }
}

static void enc_q2_k(uint8_t *o, const float *x, int k) {
    /* 84 bytes: scales[16] (sc | m << 4), qs[64] (value i: 2 bits 2 (i / 32 % 4) of qs[32 (i / 128) + i % 32]), fp16 d,
     * fp16 dmin */
    for (int sb = 0; sb < k / 256; sb++, o += 84, x += 256) {
        float sc[16], mn[16], smax = 0, mmax = 0;
        for (int j = 0; j < 16; j++) {
            float lo = x[16 * j], hi = x[16 * j];
            for (int i = 1; i < 16; i++) {
                lo = x[16 * j + i] < lo ? x[16 * j + i] : lo;
                hi = x[16 * j + i] > hi ? x[16 * j + i] : hi;
            }
            if (lo > 0) lo = 0; /* w = s * q - m with m >= 0 */
            sc[j] = (hi - lo) / 3.0f;
            mn[j] = -lo;
            smax = sc[j] > smax ? sc[j] : smax;
            mmax = mn[j] > mmax ? mn[j] : mmax;
        }
        uint16_t hd = f32_to_f16_rne(smax / 15.0f), hm = f32_to_f16_rne(mmax / 15.0f);
        float d = f16_to_f32(hd), dmin = f16_to_f32(hm);
        memset(o, 0, 84);
        for (int j = 0; j < 16; j++) {
            int a = d > 0 ? (int)lroundf(sc[j] / d) : 0, b = dmin > 0 ? (int)lroundf(mn[j] / dmin) : 0;
            a = a > 15 ? 15 : a;
            b = b > 15 ? 15 : b;
            o[j] = (uint8_t)(a | b << 4);
            const float dl = d * (float)a, ml = dmin * (float)b;
            for (int i = 0; i < 16; i++) {
                const int e = 16 * j + i;
                int q = dl > 0 ? (int)lroundf((x[e] + ml) / dl) : 0;
                q = q < 0 ? 0 : q > 3 ? 3 : q;
                o[16 + 32 * (e / 128) + e % 32] |= (uint8_t)(q << (2 * (e / 32 % 4)));
            }
        }
        memcpy(o + 80, &hd, 2);
        memcpy(o + 82, &hm, 2);
    }
}

static void enc_iq4_xs(uint8_t *o, const float *x, int k) {
    /* 136 bytes: fp16 d, u16 scales_h (bits 2 ib, 2 ib + 1: ls >> 4), scales_l[4] (nibble ib % 2 of byte ib / 2: ls & 15),
     * qs[128] (qs[16 ib + j]: low nibble the code of value j of group ib, high nibble of value 16 + j) */
    for (int sb = 0; sb < k / 256; sb++, o += 136, x += 256) {
        float sg[8], smax = 0;
        for (int ib = 0; ib < 8; ib++) {
            float amax = 0;
            for (int i = 0; i < 32; i++) amax = fabsf(x[32 * ib + i]) > amax ? fabsf(x[32 * ib + i]) : amax;
            sg[ib] = amax / 113.0f;
            smax = sg[ib] > smax ? sg[ib] : smax;
        }
        uint16_t hd = f32_to_f16_rne(smax / 31.0f);
        float d = f16_to_f32(hd);
        memset(o, 0, 136);
        memcpy(o, &hd, 2);
        uint16_t sh = 0;
        for (int ib = 0; ib < 8; ib++) {
            int a = d > 0 ? (int)lroundf(sg[ib] / d) : 0;
            a = a > 31 ? 31 : a;
            const int S = ib & 1 ? -a : a, ls = S + 32;
            o[4 + ib / 2] |= (uint8_t)((ls & 15) << (4 * (ib % 2)));
            sh |= (uint16_t)(((ls >> 4) & 3) << (2 * ib));
            const float dl = d * (float)S;
            for (int i = 0; i < 32; i++) {
                const float t = dl != 0 ? x[32 * ib + i] / dl : 0.0f;
                int best = 0;
                for (int q = 1; q < 16; q++)
                    if (fabsf((float)kv_iq4nl[q] - t) < fabsf((float)kv_iq4nl[best] - t)) best = q;
                o[8 + 16 * ib + i % 16] |= (uint8_t)(best << (4 * (i / 16)));
            }
        }
        memcpy(o + 2, &sh, 2);
    }
}

static void put16(uint8_t *p, uint16_t v) { memcpy(p, &v, 2); }
static void put32(uint8_t *p, uint32_t v) { memcpy(p, &v, 4); }

static void enc_iq_cb(int type, uint8_t *o, const float *x, int k) {
    /* random valid blocks (see the header): fields drawn, the values' sum of squares of d = 1 accumulated as they are
     * drawn (w = (d * mult) S v), then d = rms(x) / rms(w at d = 1) */
    uint64_t st = 0x6a09e667f3bcc909ull;
    for (int i = 0; i < k; i++) {
        uint32_t u;
        memcpy(&u, &x[i], 4);
        st = (st ^ u) * 0x100000001b3ull;
    }
    const int bytes = cb_bytes(type);
    const double mult = type == T_IQ3_XXS ? 0.25 : type == T_IQ3_S ? 1.0 : 0.125;
    for (int sb = 0; sb < k / 256; sb++, o += bytes, x += 256) {
        memset(o, 0, (size_t)bytes);
        double ss = 0; /* sum of (S v)^2 */
        for (int ib = 0; ib < 8; ib++) {
            const uint32_t r0 = (uint32_t)splitmix(&st), r1 = (uint32_t)splitmix(&st);
            if (type == T_IQ2_XXS) { /* a0: 4 indices; a1: 4 x 7 sign bits, ls */
                put32(o + 2 + 8 * ib, r0);
                put32(o + 6 + 8 * ib, r1);
                const int S = 2 * (int)(r1 >> 28) + 1;
                for (int l = 0; l < 4; l++)
                    for (int j = 0; j < 8; j++) {
                        const double v = GW_IQ2_VAL((gw_iq2xxs_codes[r0 >> 8 * l & 255] >> 2 * j) & 3);
                        ss += (S * v) * (S * v);
                    }
            } else if (type == T_IQ2_XS || type == T_IQ2_S) {
                const int sc = (int)(r1 & 255);
                o[(type == T_IQ2_XS ? 66 : 74) + ib] = (uint8_t)sc;
                const uint32_t r2 = (uint32_t)splitmix(&st);
                for (int l = 0; l < 4; l++) {
                    int idx;
                    if (type == T_IQ2_XS) {
                        const uint16_t q = (uint16_t)(l < 2 ? r0 >> 16 * l : r2 >> 16 * (l - 2));
                        put16(o + 2 + 2 * (4 * ib + l), q);
                        idx = q & 511;
                    } else {
                        o[2 + 4 * ib + l] = (uint8_t)(r0 >> 8 * l);
                        o[34 + 4 * ib + l] = (uint8_t)(r2 >> 8 * l);
                        idx = o[2 + 4 * ib + l] | ((r1 >> (8 + 2 * l)) & 3) << 8;
                        o[66 + ib] |= (uint8_t)(((r1 >> (8 + 2 * l)) & 3) << 2 * l);
                    }
                    const int S = 2 * ((sc >> 4 * (l / 2)) & 15) + 1;
                    const uint16_t *cd = type == T_IQ2_XS ? gw_iq2xs_codes : gw_iq2s_codes;
                    for (int j = 0; j < 8; j++) {
                        const double v = GW_IQ2_VAL((cd[idx] >> 2 * j) & 3);
                        ss += (S * v) * (S * v);
                    }
                }
            } else if (type == T_IQ3_XXS) { /* qs: 8 indices of 4 values; a: 4 x 7 sign bits, ls */
                const uint32_t r2 = (uint32_t)splitmix(&st);
                put32(o + 2 + 8 * ib, r0);
                put32(o + 6 + 8 * ib, r2);
                put32(o + 66 + 4 * ib, r1);
                const int S = 2 * (int)(r1 >> 28) + 1;
                for (int t = 0; t < 8; t++) {
                    const int idx = o[2 + 8 * ib + t];
                    for (int j = 0; j < 4; j++) {
                        const double v = GW_IQ3XXS_VAL((gw_iq3xxs_codes[idx] >> 3 * j) & 7);
                        ss += (S * v) * (S * v);
                    }
                }
            } else if (type == T_IQ3_S) { /* qs, qh (index bit 8), raw signs, 4-bit scales */
                const uint32_t r2 = (uint32_t)splitmix(&st), r3 = (uint32_t)splitmix(&st);
                put32(o + 2 + 8 * ib, r0);
                put32(o + 6 + 8 * ib, r2);
                o[66 + ib] = (uint8_t)r1;
                put32(o + 74 + 4 * ib, r3);
                o[106 + ib / 2] |= (uint8_t)(((r1 >> 8) & 15) << 4 * (ib % 2));
                const int S = 2 * (int)((r1 >> 8) & 15) + 1;
                for (int t = 0; t < 8; t++) {
                    const int idx = o[2 + 8 * ib + t] | ((r1 >> t) & 1) << 8;
                    for (int j = 0; j < 4; j++) {
                        const double v = 2 * ((gw_iq3s_codes[idx] >> 3 * j) & 7) + 1;
                        ss += (S * v) * (S * v);
                    }
                }
            } else if (type == T_IQ1_S) { /* qs; qh: 4 x 3 index bits, the 3-bit scale, the delta's sign */
                put32(o + 2 + 4 * ib, r0);
                const uint16_t qh = (uint16_t)r1;
                put16(o + 34 + 2 * ib, qh);
                const int S = 2 * ((qh >> 12) & 7) + 1, dl = qh & 0x8000 ? -1 : 1;
                for (int l = 0; l < 4; l++) {
                    const int idx = (int)(r0 >> 8 * l & 255) | ((qh >> 3 * l) & 7) << 8;
                    for (int j = 0; j < 8; j++) {
                        const double v = 8 * (((gw_iq1s_codes[idx] >> 2 * j) & 3) - 1) + dl;
                        ss += (S * v) * (S * v);
                    }
                }
            } else { /* IQ1_M: qs; qh nibbles (3 index bits, the delta's sign) per chunk; 3-bit scales per 16 */
                put32(o + 4 * ib, r0);
                o[32 + 2 * ib] = (uint8_t)r1;
                o[33 + 2 * ib] = (uint8_t)(r1 >> 8);
                const int s6 = (int)((r1 >> 16) & 63); /* (the group's two 3-bit scales, into sc[ib / 2] below) */
                uint16_t scw;
                memcpy(&scw, o + 48 + 2 * (ib / 2), 2);
                scw |= (uint16_t)(s6 << 6 * (ib % 2));
                put16(o + 48 + 2 * (ib / 2), scw);
                for (int l = 0; l < 4; l++) {
                    const int q = (o[32 + 2 * ib + l / 2] >> 4 * (l % 2)) & 15, dl = q & 8 ? -1 : 1;
                    const int idx = (int)(r0 >> 8 * l & 255) | (q & 7) << 8, S = 2 * ((s6 >> 3 * (l / 2)) & 7) + 1;
                    for (int j = 0; j < 8; j++) {
                        const double v = 8 * (((gw_iq1s_codes[idx] >> 2 * j) & 3) - 1) + dl;
                        ss += (S * v) * (S * v);
                    }
                }
            }
        }
        double xs = 0;
        for (int i = 0; i < 256; i++) xs += (double)x[i] * x[i];
        const double rw = sqrt(ss / 256.0) * mult;
        uint16_t hd = f32_to_f16_rne(rw > 0 ? (float)(sqrt(xs / 256.0) / rw) : 0.0f);
        if (type == T_IQ1_M) { /* d in the top nibbles of sc[0..3] */
            for (int w = 0; w < 4; w++) {
                uint16_t scw;
                memcpy(&scw, o + 48 + 2 * w, 2);
                scw = (uint16_t)((scw & 0x0fff) | ((hd >> 4 * w) & 15) << 12);
                put16(o + 48 + 2 * w, scw);
            }
        } else put16(o, hd);
    }
}

void gw_synth_encode_row(int type, uint8_t *o, const float *x, int k) {
    if (type == T_Q8_0) enc_q8_0(o, x, k);
    else if (type == T_Q4_K) enc_q45_k(o, x, k, 0);
    else if (type == T_Q5_K) enc_q45_k(o, x, k, 1);
    else if (type == T_Q3_K) enc_q3_k(o, x, k);
    else if (type == T_Q6_K) enc_q6_k(o, x, k);
    else if (type == T_IQ4_XS) enc_iq4_xs(o, x, k);
    else if (type == T_Q2_K) enc_q2_k(o, x, k);
    else if (IS_CB(type)) enc_iq_cb(type, o, x, k);
    else memcpy(o, x, (size_t)k * 4);
}

/* ------------------------------------------------------------------------------------ GGUF writing */

typedef struct {
    char name[64];
    int type, rows, cols; /* ne = { cols, rows } (rows 0: a vector of cols values) */
    int norm;             /* a norm vector (constant value) */
    uint64_t off;
} SynTensor;

typedef struct { FILE *f; int err; } W;

static void w_bytes(W *w, const void *p, size_t n) {
    if (!w->err && fwrite(p, 1, n, w->f) != n) w->err = 1;
}
static void w_u32(W *w, uint32_t v) { w_bytes(w, &v, 4); }
static void w_u64(W *w, uint64_t v) { w_bytes(w, &v, 8); }
static void w_str(W *w, const char *s) { uint64_t n = strlen(s); w_u64(w, n); w_bytes(w, s, n); }
static void kv_u32(W *w, const char *k, uint32_t v) { w_str(w, k); w_u32(w, 4 /* GV_U32 */); w_u32(w, v); }
static void kv_f32(W *w, const char *k, float v) { w_str(w, k); w_u32(w, 6 /* GV_F32 */); w_bytes(w, &v, 4); }
static void kv_s(W *w, const char *k, const char *v) { w_str(w, k); w_u32(w, 8 /* GV_STR */); w_str(w, v); }

/* ------------------------------------------------------------------------- synthetic tokenizer (cfg->tokenizer) */

/* A small byte-level BPE vocabulary in the form llama.cpp's "gpt2" model with the "qwen2" pre-tokenizer stores it (the
 * metadata the reference's build_tokenizer_gguf reads, tokenizer.c:201-320): ids 0..255 the single bytes; then, for
 * a fixed list of English words, with and without a leading space, each word's prefixes of two bytes and more, each
 * made by the merge (its prefix one byte shorter, its last byte), merges in that order; then the added tokens
 * (ChatML's control tokens and the think tags). Token strings and merges are in GPT-2's byte-to-unicode form. */

static int gpt2_printable(int b) { return (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174 && b <= 255); }

static size_t gpt2_form(const unsigned char *p, size_t n, char *o) {
    /* GPT-2's map: a printable byte stands for its own code point, the other 68 bytes for 256, 257, .. in byte order;
     * UTF-8 encoded */
    size_t k = 0;
    for (size_t i = 0; i < n; i++) {
        int b = p[i], cp = b;
        if (!gpt2_printable(b)) {
            cp = 256;
            for (int x = 0; x < b; x++) cp += !gpt2_printable(x);
        }
        if (cp < 0x80) o[k++] = (char)cp;
        else {
            o[k++] = (char)(0xc0 | (cp >> 6));
            o[k++] = (char)(0x80 | (cp & 63));
        }
    }
    o[k] = 0;
    return k;
}

typedef struct {
    char **tok;     /* GPT-2 form of each token */
    int32_t *type;  /* 1 normal, 3 control, 4 user-defined */
    char **merge;   /* "left right", rank order */
    int n_tok, n_merge, eos;
} SynTok;

static const char *const syn_words[] = {
    "the", "and", "of", "to", "in", "is", "it", "you", "that", "was", "for", "on", "are", "with", "as", "this", "be",
    "at", "have", "from", "or", "one", "had", "by", "word", "but", "not", "what", "all", "were", "we", "when", "your",
    "can", "said", "there", "use", "an", "each", "which", "she", "do", "how", "their", "if", "will", "up", "other",
    "about", "out", "many", "then", "them", "these", "so", "some", "her", "would", "make", "like", "him", "into",
    "time", "has", "look", "two", "more", "write", "go", "see", "number", "no", "way", "could", "people", "my",
    "than", "first", "water", "been", "call", "who", "its", "now", "find", "long", "down", "day", "did", "get",
    "come", "made", "may", "part", "hello", "world", "answer", "question", "model", "token", "user", "assistant",
    "system", "think", "Hello", "The", "What", "Why", "12", "42", "2024", "\n\n", "  ", "...", ", ",
};

static void syn_tok_free(SynTok *t) {
    for (int i = 0; i < t->n_tok; i++) free(t->tok[i]);
    for (int i = 0; i < t->n_merge; i++) free(t->merge[i]);
    free(t->tok);
    free(t->type);
    free(t->merge);
    memset(t, 0, sizeof *t);
}

static int syn_tok_build(SynTok *t, int vocab) {
    /* -1: the vocabulary is too small (256 bytes + the added tokens) or no memory */
    static const char *const added[] = { "<|endoftext|>", "<|im_start|>", "<|im_end|>", "<think>", "</think>" };
    const int n_added = 5;
    if (vocab < 256 + n_added) return -1;
    memset(t, 0, sizeof *t);
    t->tok = calloc((size_t)vocab, sizeof(char *));
    t->type = calloc((size_t)vocab, sizeof(int32_t));
    t->merge = calloc((size_t)vocab, sizeof(char *));
    unsigned char **raw = calloc((size_t)vocab, sizeof(unsigned char *)); /* raw bytes of the regular tokens */
    int *rawn = calloc((size_t)vocab, sizeof(int));
    if (!t->tok || !t->type || !t->merge || !raw || !rawn) goto fail;
    char g[512];
    for (int b = 0; b < 256; b++) {
        unsigned char c = (unsigned char)b;
        gpt2_form(&c, 1, g);
        raw[b] = malloc(1);
        if (!(t->tok[b] = strdup(g)) || !raw[b]) goto fail;
        raw[b][0] = c;
        rawn[b] = 1;
        t->type[b] = 1;
    }
    int n = 256;
    for (size_t wi = 0; wi < sizeof syn_words / sizeof syn_words[0]; wi++)
        for (int sp = 0; sp < 2; sp++) {
            unsigned char w[64];
            int len = 0;
            if (sp) w[len++] = ' ';
            for (const char *q = syn_words[wi]; *q && len < 60; q++) w[len++] = (unsigned char)*q;
            for (int k = 2; k <= len && n < vocab - n_added; k++) {
                int have = 0;
                for (int i = 256; i < n && !have; i++) have = rawn[i] == k && !memcmp(raw[i], w, (size_t)k);
                if (have) continue;
                char a[256], c[16];
                gpt2_form(w, (size_t)(k - 1), a);
                gpt2_form(w + k - 1, 1, c);
                snprintf(g, sizeof g, "%s %s", a, c);
                if (!(t->merge[t->n_merge] = strdup(g))) goto fail;
                t->n_merge++;
                gpt2_form(w, (size_t)k, g);
                if (!(t->tok[n] = strdup(g)) || !(raw[n] = malloc((size_t)k))) goto fail;
                memcpy(raw[n], w, (size_t)k);
                rawn[n] = k;
                t->type[n++] = 1;
            }
        }
    for (int i = 0; i < n_added; i++) {
        if (!(t->tok[n] = strdup(added[i]))) goto fail;
        t->type[n] = i < 3 ? 3 : 4;
        if (i == 2) t->eos = n;
        n++;
    }
    t->n_tok = n;
    for (int i = 0; i < vocab; i++) free(raw[i]);
    free(raw);
    free(rawn);
    return 0;
fail:
    if (raw)
        for (int i = 0; i < vocab; i++) free(raw[i]);
    free(raw);
    free(rawn);
    t->n_tok = vocab; /* (free every slot) */
    syn_tok_free(t);
    return -1;
}

static void kv_arr_s(W *w, const char *k, char *const *v, int n) {
    w_str(w, k);
    w_u32(w, 9 /* GV_ARR */);
    w_u32(w, 8 /* GV_STR */);
    w_u64(w, (uint64_t)n);
    for (int i = 0; i < n; i++) w_str(w, v[i]);
}

static void kv_arr_i32(W *w, const char *k, const int32_t *v, int n) {
    w_str(w, k);
    w_u32(w, 9 /* GV_ARR */);
    w_u32(w, 5 /* GV_I32 */);
    w_u64(w, (uint64_t)n);
    w_bytes(w, v, (size_t)n * 4);
}

typedef struct {
    const SynTensor *t;
    int tindex;
    uint8_t *out; /* the chunk buffer: row r at out + (r - base) * row bytes */
    int base;
    uint64_t seed;
    float std;
    int r0, r1;
} Job;

static void *job_run(void *arg) {
    Job *j = arg;
    const SynTensor *t = j->t;
    float *row = malloc((size_t)t->cols * sizeof(float));
    if (!row) return (void *)1;
    size_t rb = gw_synth_row_bytes(t->type, t->cols);
    for (int r = j->r0; r < j->r1; r++) {
        normal_row(row, t->cols, j->seed, (uint64_t)j->tindex, (uint64_t)r, j->std);
        gw_synth_encode_row(t->type, j->out + (size_t)(r - j->base) * rb, row, t->cols);
    }
    free(row);
    return NULL;
}

int gw_synth_gguf(const char *path, const GwSynthCfg *c, unsigned long long seed, int nthreads) {
    if (!path || !c || c->dim <= 0 || c->n_layers <= 0 || c->n_heads <= 0 || c->n_kv_heads <= 0 || c->head_dim <= 0 ||
        c->hidden <= 0 || c->vocab <= 0 || c->n_heads % c->n_kv_heads)
        return -1;
    int L = c->n_layers, dim = c->dim, qd = c->n_heads * c->head_dim, kvd = c->n_kv_heads * c->head_dim;
    int td = c->type_default ? c->type_default : T_Q8_0;
#define TY(x) ((x) ? (x) : td)
    int nt = 3 + !c->tied + 11 * L, k = 0;
    SynTensor *T = calloc((size_t)nt, sizeof(SynTensor));
    if (!T) return -2;
#define ADD(nm, ty, r, cl, nrm) do { snprintf(T[k].name, sizeof(T[k].name), "%s", nm); T[k].type = (ty); T[k].rows = (r); \
        T[k].cols = (cl); T[k].norm = (nrm); k++; } while (0)
    char nm[64];
    ADD("token_embd.weight", TY(c->type_embd), c->vocab, dim, 0);
    ADD("output_norm.weight", T_F32, 0, dim, 1);
    if (!c->tied) ADD("output.weight", TY(c->type_out), c->vocab, dim, 0);
    for (int l = 0; l < L; l++) {
        snprintf(nm, sizeof nm, "blk.%d.attn_norm.weight", l); ADD(nm, T_F32, 0, dim, 1);
        snprintf(nm, sizeof nm, "blk.%d.attn_q.weight", l); ADD(nm, TY(c->type_q), qd, dim, 0);
        snprintf(nm, sizeof nm, "blk.%d.attn_k.weight", l); ADD(nm, TY(c->type_k), kvd, dim, 0);
        snprintf(nm, sizeof nm, "blk.%d.attn_v.weight", l); ADD(nm, TY(c->type_v), kvd, dim, 0);
        snprintf(nm, sizeof nm, "blk.%d.attn_output.weight", l); ADD(nm, TY(c->type_o), dim, qd, 0);
        snprintf(nm, sizeof nm, "blk.%d.attn_q_norm.weight", l); ADD(nm, T_F32, 0, c->head_dim, 1);
        snprintf(nm, sizeof nm, "blk.%d.attn_k_norm.weight", l); ADD(nm, T_F32, 0, c->head_dim, 1);
        snprintf(nm, sizeof nm, "blk.%d.ffn_norm.weight", l); ADD(nm, T_F32, 0, dim, 1);
        snprintf(nm, sizeof nm, "blk.%d.ffn_gate.weight", l); ADD(nm, TY(c->type_gate), c->hidden, dim, 0);
        snprintf(nm, sizeof nm, "blk.%d.ffn_up.weight", l); ADD(nm, TY(c->type_up), c->hidden, dim, 0);
        snprintf(nm, sizeof nm, "blk.%d.ffn_down.weight", l); ADD(nm, TY(c->type_down), dim, c->hidden, 0);
    }
    nt = k;
    const uint64_t align = 32;
    uint64_t off = 0;
    for (int i = 0; i < nt; i++) {
        if (IS_SB(T[i].type) && T[i].cols % 256) { free(T); return -1; }
        if (T[i].type == T_Q8_0 && T[i].cols % 32) { free(T); return -1; }
        T[i].off = off;
        uint64_t sz = T[i].rows ? (uint64_t)T[i].rows * gw_synth_row_bytes(T[i].type, T[i].cols) : (uint64_t)T[i].cols * 4;
        off += (sz + align - 1) / align * align;
    }
    SynTok tk;
    memset(&tk, 0, sizeof tk);
    if (c->tokenizer && syn_tok_build(&tk, c->vocab)) { free(T); return -1; }
    FILE *f = fopen(path, "wb");
    if (!f) { free(T); syn_tok_free(&tk); return -3; }
    static char buf[1 << 22];
    setvbuf(f, buf, _IOFBF, sizeof buf);
    W w = { f, 0 };
    w_u32(&w, 0x46554747u);
    w_u32(&w, 3);
    w_u64(&w, (uint64_t)nt);
    w_u64(&w, c->tokenizer ? 20 : 13);
    kv_s(&w, "general.architecture", "qwen3");
    kv_u32(&w, "general.alignment", (uint32_t)align);
    kv_u32(&w, "qwen3.block_count", (uint32_t)L);
    kv_u32(&w, "qwen3.embedding_length", (uint32_t)dim);
    kv_u32(&w, "qwen3.feed_forward_length", (uint32_t)c->hidden);
    kv_u32(&w, "qwen3.attention.head_count", (uint32_t)c->n_heads);
    kv_u32(&w, "qwen3.attention.head_count_kv", (uint32_t)c->n_kv_heads);
    kv_u32(&w, "qwen3.context_length", (uint32_t)(c->ctx_len > 0 ? c->ctx_len : 40960));
    kv_u32(&w, "qwen3.attention.key_length", (uint32_t)c->head_dim);
    kv_u32(&w, "qwen3.attention.value_length", (uint32_t)c->head_dim);
    kv_f32(&w, "qwen3.rope.freq_base", c->rope_theta > 0 ? c->rope_theta : 1e6f);
    kv_f32(&w, "qwen3.attention.layer_norm_rms_epsilon", 1e-6f);
    kv_s(&w, "general.name", "gwenedeg-amd synthetic");
    if (c->tokenizer) {
        kv_s(&w, "tokenizer.ggml.model", "gpt2");
        kv_s(&w, "tokenizer.ggml.pre", "qwen2");
        kv_arr_s(&w, "tokenizer.ggml.tokens", tk.tok, tk.n_tok);
        kv_arr_i32(&w, "tokenizer.ggml.token_type", tk.type, tk.n_tok);
        kv_arr_s(&w, "tokenizer.ggml.merges", tk.merge, tk.n_merge);
        kv_u32(&w, "tokenizer.ggml.eos_token_id", (uint32_t)tk.eos);
        /* (a ChatML template with enable_thinking: Qwen3's hybrid variant) */
        kv_s(&w, "tokenizer.chat_template",
             "{%- for message in messages %}{{- '<|im_start|>' + message.role + '\\n' + message.content + '<|im_end|>' + "
             "'\\n' }}{%- endfor %}{%- if add_generation_prompt %}{{- '<|im_start|>assistant\\n' }}{%- if enable_thinking "
             "is defined and enable_thinking is false %}{{- '<think>\\n\\n</think>\\n\\n' }}{%- endif %}{%- endif %}");
        syn_tok_free(&tk);
    }
    for (int i = 0; i < nt; i++) {
        w_str(&w, T[i].name);
        if (T[i].rows) {
            w_u32(&w, 2);
            w_u64(&w, (uint64_t)T[i].cols);
            w_u64(&w, (uint64_t)T[i].rows);
        } else {
            w_u32(&w, 1);
            w_u64(&w, (uint64_t)T[i].cols);
        }
        w_u32(&w, (uint32_t)T[i].type);
        w_u64(&w, T[i].off);
    }
    long pos = ftell(f);
    static const uint8_t zeros[64];
    if (pos % (long)align) w_bytes(&w, zeros, (size_t)(align - pos % align));
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 64) nthreads = 64;
    float std = c->std > 0 ? c->std : 0.02f, nv = c->norm_value != 0 ? c->norm_value : 1.0f;
    uint64_t written = 0;
    int rc = 0;
    for (int i = 0; i < nt && !w.err && !rc; i++) {
        if (written < T[i].off) { uint64_t pad = T[i].off - written; w_bytes(&w, zeros, (size_t)pad); written += pad; }
        if (!T[i].rows) {
            for (int j = 0; j < T[i].cols; j++) w_bytes(&w, &nv, 4);
            written += (uint64_t)T[i].cols * 4;
            continue;
        }
        size_t rb = gw_synth_row_bytes(T[i].type, T[i].cols), chunk_rows = (size_t)(256u << 20) / rb;
        if (chunk_rows < 1) chunk_rows = 1;
        if (chunk_rows > (size_t)T[i].rows) chunk_rows = (size_t)T[i].rows;
        uint8_t *out = malloc(chunk_rows * rb);
        if (!out) { rc = -2; break; }
        for (int r0 = 0; r0 < T[i].rows && !rc; r0 += (int)chunk_rows) {
            int r1 = r0 + (int)chunk_rows < T[i].rows ? r0 + (int)chunk_rows : T[i].rows, n = r1 - r0;
            int tn = nthreads < n ? nthreads : n;
            pthread_t th[64];
            Job jb[64];
            for (int q = 0; q < tn; q++) {
                jb[q] = (Job){ &T[i], i, out, r0, seed, std, r0 + (int)(n * (long)q / tn), r0 + (int)(n * (long)(q + 1) / tn) };
            }
            for (int q = 0; q < tn; q++)
                if (pthread_create(&th[q], NULL, job_run, &jb[q])) { rc = -4; tn = q; break; }
            for (int q = 0; q < tn; q++) {
                void *res = NULL;
                pthread_join(th[q], &res);
                if (res) rc = -2;
            }
            if (!rc) w_bytes(&w, out, (size_t)n * rb);
        }
        free(out);
        written += (uint64_t)T[i].rows * rb;
    }
    if (fclose(f)) w.err = 1;
    free(T);
    return rc ? rc : w.err ? -3 : 0;
}
