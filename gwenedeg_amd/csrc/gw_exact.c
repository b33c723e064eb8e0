/* The reference's host-specific floating point, measured on this host so that the device reproduces it bit for bit.
 *
 * The reference is built with gcc -Ofast (-ffast-math) for AVX-512, and three of its operations are not IEEE-defined:
 *   1.0f / sqrtf(t)  (rmsnorm forward.c:896, QK-norm, the attention scale forward.c:137): gcc expands it into
 *                    r0 = rsqrtss(t), the CPU's estimate, and one Newton step r = fma(t r0, r0, -3) (r0 * -0.5)
 *   SwiGLU's expf    (forward.c:1953-1958): the loop is vectorized, e = glibc libmvec's _ZGVeN16v_expf(min(-h, 80))
 *   SwiGLU's 1 / d   (d = 1 + e): a vector division, r0 = vrcp14ps(d) (the CPU's estimate) and the Newton step
 *                    r = (r0 + r0) - r0 (r0 d); out = (h h2) r
 * The estimates (rsqrtss, vrcp14ps) are table lookups inside the CPU, exact up to the power of 2, so a table of their
 * values measured here on one binade reproduces them everywhere (verified on seeded inputs before use; vrcp14ps's is
 * kept in the compact form of rcp_compact). libmvec's expf is glibc's published AVX-512 method (its
 * svml_s_expf16_core_avx512 and data table): n = fma(x, 1/ln2, 1.5 2^23) - 1.5 2^23 (round to nearest by the shifter),
 * r = fma(-n, ln2_hi, x), r = fma(-n, ln2_lo, r) (ln2 split as 0x3f317200 + 0x35bfbe8e), a degree-5 polynomial in
 * Horner form with fma (c0 = 1, c1 .. c5 below), scaled by 2^n through the exponent field. The device computes that
 * (gw_exp_mvec here, exp_mvec there, operation for operation); the library still calls the host's libmvec on every
 * float the SwiGLU can meet where a difference could arise (|x| in [2^-26, 32) negative, [2^-26, 128) positive: 64
 * binades) and compares: equal everywhere (the development host: 0 differences among 5.1e8 inputs), no table; else the
 * signed ulp differences (4 bits each, 256 MiB) go to the device too, as a host with another libmvec needs. Outside:
 * |x| < 2^-26 both give 1 (r = x, and 1 + c1 x rounds to 1), x <= -32 gives 1 + e = 1 exactly either way (e < 2^-24),
 * x is clamped at 80.
 *
 * The tables are the host's, not constants: the reference's own results differ between CPUs the same way. A host
 * without AVX-512 leaves them unset, and the device falls back to IEEE 1 / sqrtf and division and the Cephes exp
 * (then it matches the oracle's portable definition, not the reference's bits).
 */
#define _GNU_SOURCE
#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "gw_internal.h"

static inline float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t u_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

/* ------------------------------------------------------------------------------------------- rsqrtss */

static inline float host_rsqrtss(float x) { return _mm_cvtss_f32(_mm_rsqrt_ss(_mm_set_ss(x))); }

static float rsqrt_lookup(const float *tab, int bits, float t) {
    /* t > 0 normal: the table's value for t's exponent parity and leading mantissa bits, scaled by t's power of 4 */
    uint32_t u = u_of(t);
    int e = (int)(u >> 23) - 127, par = e & 1;
    float r1 = tab[(((uint32_t)par << 23) | (u & 0x7fffffu)) >> (24 - bits)];
    return f_of(u_of(r1) - (uint32_t)(((e - par) >> 1) << 23));
}

float gw_rsqrt_host(float t) {
    /* the reference's 1.0f / sqrtf(t) on this host (rsqrtss + gcc's Newton step; constants of its object code) */
    float r0 = host_rsqrtss(t);
    float b = fmaf(t * r0, r0, -3.0f);
    return b * (r0 * -0.5f);
}

static float rsq_tab[1 << GW_RSQRT_MAXBITS_H];
static int rsq_bits = -1;

static int rsqrt_measure(void) {
    /* the fewest leading bits (parity + mantissa) that reproduce rsqrtss on 2^20 seeded inputs over 120 binades */
    for (int bits = 10; bits <= GW_RSQRT_MAXBITS_H; bits++) {
        for (uint32_t i = 0; i < (1u << bits); i++) rsq_tab[i] = host_rsqrtss(f_of(0x3f800000u + (i << (24 - bits))));
        int ok = 1;
        for (uint64_t k = 1; k <= (1u << 20) && ok; k++) {
            uint64_t r = mix64(k * 0x9e3779b97f4a7c15ull);
            float t = f_of(((uint32_t)(127 + (int)(r % 120) - 60) << 23) | (uint32_t)((r >> 8) & 0x7fffffu));
            ok = u_of(rsqrt_lookup(rsq_tab, bits, t)) == u_of(host_rsqrtss(t));
        }
        if (ok) return bits;
    }
    return 0;
}

/* ------------------------------------------------------------------------ SwiGLU: vrcp14ps and libmvec expf */

__m512 _ZGVeN16v_expf(__m512);

#define EXP_E0 101   /* first tabulated biased exponent (2^-26) */
#define EXP_POS 33   /* binades of x > 0: exponents 101..133 ([2^-26, 128)) */
#define EXP_NEG 31   /* binades of x < 0: exponents 101..131 ((-32, -2^-26]) */

static float exp_cephes(float x) {
    /* the attention's Cephes-style exp (forward.c:1301-1321's operations) without its clamp, for x in [-86, 80]: the
     * portable SwiGLU's exp on a host without the tables */
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
    return f_of(u_of(y) + ((uint32_t)(int32_t)n << 23));
}

float gw_exp_mvec(float x) {
    /* libmvec's expf by its published method (see above), for x in [-32, 80]: the device's exp_mvec, operation for
     * operation */
    const float sh = 12582912.0f; /* 1.5 2^23 */
    float n = fmaf(x, f_of(0x3fb8aa3bu), sh) - sh;
    float r = fmaf(-n, f_of(0x3f317200u), x);
    r = fmaf(-n, f_of(0x35bfbe8eu), r);
    float p = f_of(0x3c07d9feu);
    p = fmaf(p, r, f_of(0x3d2b8392u));
    p = fmaf(p, r, f_of(0x3e2aacacu));
    p = fmaf(p, r, f_of(0x3effff34u));
    p = fmaf(p, r, f_of(0x3f7ffffeu));
    p = fmaf(p, r, 1.0f);
    return f_of(u_of(p) + ((uint32_t)(int32_t)n << 23));
}

static float *rcp_tab;       /* vrcp14ps of 1.m, 2^23 floats */
static uint64_t *rcp_blk;    /* the same in 2^16 words, one per block of 128 mantissas (RCP_BLK_BITS) */
static uint8_t *exp_delta;   /* 2^29 nibbles: libmvec expf - gw_exp_mvec in ulps, + 8 (NULL: no difference anywhere) */
static int swiglu_ok = -1;   /* -1 not measured, 0 not reproducible here, 1 tables ready */

typedef struct { int slot0, slot1, bad; long nz; } ExpJob;

__attribute__((target("avx512f"))) static void *exp_worker(void *arg) {
    ExpJob *j = arg;
    float xs[16] __attribute__((aligned(64))), ys[16] __attribute__((aligned(64)));
    for (int slot = j->slot0; slot < j->slot1 && !j->bad; slot++) {
        uint32_t sign = slot >= EXP_POS ? 0x80000000u : 0, e = (uint32_t)(EXP_E0 + (slot >= EXP_POS ? slot - EXP_POS : slot));
        for (uint32_t m = 0; m < (1u << 23) && !j->bad; m += 16) {
            for (int k = 0; k < 16; k++) xs[k] = f_of(sign | e << 23 | (m + (uint32_t)k));
            _mm512_store_ps(ys, _ZGVeN16v_expf(_mm512_load_ps(xs)));
            for (int k = 0; k < 16; k += 2) {
                /* (x > 80: never met, the argument is clamped; no difference stored) */
                int d0 = xs[k] > 80.0f ? 0 : (int)(u_of(ys[k]) - u_of(gw_exp_mvec(xs[k])));
                int d1 = xs[k + 1] > 80.0f ? 0 : (int)(u_of(ys[k + 1]) - u_of(gw_exp_mvec(xs[k + 1])));
                if (d0 < -7 || d0 > 7 || d1 < -7 || d1 > 7) { j->bad = 1; break; }
                j->nz += (d0 != 0) + (d1 != 0);
                exp_delta[(((size_t)slot << 23) | (m + (uint32_t)k)) >> 1] = (uint8_t)((d0 + 8) | (d1 + 8) << 4);
            }
        }
    }
    return NULL;
}

__attribute__((target("avx512f"))) static float host_rcp14(float x) {
    return _mm512_cvtss_f32(_mm512_rcp14_ps(_mm512_set1_ps(x)));
}

static int rcp_compact(void) {
    /* vrcp14ps on [1, 2) is a non-increasing step function of the mantissa whose values lie in [0.5, 1] with at most
     * one step inside any block of 128 consecutive mantissas (measured here, not assumed: any block with two is a
     * failure): per block b, a = its first value, c = its value after the step, p = the step's offset (128: none),
     * packed as (a - 0.5's bits) | (c - 0.5's bits) << 24 | p << 48; then every mantissa checked against the table */
    rcp_blk = malloc(sizeof(uint64_t) << (23 - RCP_BLK_BITS));
    if (!rcp_blk) return 1;
    const uint32_t B = 1u << RCP_BLK_BITS, half = 0x3f000000u;
    for (uint32_t b = 0; b < (1u << (23 - RCP_BLK_BITS)); b++) {
        const uint32_t m0 = b << RCP_BLK_BITS, a = u_of(rcp_tab[m0]);
        uint32_t p = B, c = a;
        for (uint32_t o = 1; o < B; o++) {
            const uint32_t v = u_of(rcp_tab[m0 + o]);
            if (v == c) continue;
            if (p != B || v > c) return 1; /* (a second step, or not non-increasing) */
            p = o, c = v;
        }
        if (a < half || a > 0x3f800000u || c < half) return 1;
        rcp_blk[b] = (uint64_t)(a - half) | (uint64_t)(c - half) << 24 | (uint64_t)p << 48;
    }
    for (uint32_t m = 0; m < (1u << 23); m++) {
        const uint64_t w = rcp_blk[m >> RCP_BLK_BITS];
        const uint32_t o = m & (B - 1), v = 0x3f000000u + (uint32_t)(o < ((w >> 48) & 0xffu) ? w : w >> 24) % (1u << 24);
        if (v != u_of(rcp_tab[m])) return 1;
    }
    return 0;
}

static int swiglu_measure(void) {
    if (!__builtin_cpu_supports("avx512f")) return 0;
    rcp_tab = malloc((size_t)4 << 23);
    exp_delta = malloc((size_t)1 << 28);
    if (!rcp_tab || !exp_delta) return 0;
    for (uint32_t m = 0; m < (1u << 23); m++) rcp_tab[m] = host_rcp14(f_of(0x3f800000u | m));
    if (rcp_compact()) return 0;
    for (uint64_t k = 1; k <= (1u << 20); k++) { /* exact up to the power of 2, on d in [1, 2^120) */
        uint64_t r = mix64(k * 0xd1b54a32d192ed03ull);
        float d = f_of(((uint32_t)(127 + (int)(r % 120)) << 23) | (uint32_t)((r >> 8) & 0x7fffffu));
        uint32_t v = u_of(d);
        if (u_of(rcp_tab[v & 0x7fffffu]) - (((v >> 23) - 127) << 23) != u_of(host_rcp14(d))) return 0;
    }
    enum { NT = 16 };
    pthread_t th[NT];
    ExpJob job[NT];
    int ns = EXP_POS + EXP_NEG, bad = 0, started = 0;
    long nz = 0;
    for (int i = 0; i < NT; i++) {
        job[i] = (ExpJob){ ns * i / NT, ns * (i + 1) / NT, 0, 0 };
        if (pthread_create(&th[i], NULL, exp_worker, &job[i])) { exp_worker(&job[i]); continue; }
        started |= 1 << i;
    }
    for (int i = 0; i < NT; i++) {
        if (started & (1 << i)) pthread_join(th[i], NULL);
        bad |= job[i].bad;
        nz += job[i].nz;
    }
    if (!bad && !nz) { /* libmvec's expf is gw_exp_mvec for every input: no table */
        free(exp_delta);
        exp_delta = NULL;
    }
    return !bad;
}

/* ------------------------------------------------------------------------------ per-device installation */

static int dev_done[64];
static void *dev_rcp[64], *dev_exp[64];
static pthread_mutex_t mu = PTHREAD_MUTEX_INITIALIZER;

int gw_exact_init(char *err, size_t errlen) {
    /* the tables measured once per process, installed once per device (the current one) */
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return gw_hip_fail(err, errlen, "hipGetDevice", e);
    pthread_mutex_lock(&mu);
    int rc = RQ_OK;
    if (rsq_bits < 0) rsq_bits = rsqrt_measure();
    if (swiglu_ok < 0) swiglu_ok = swiglu_measure();
    if (dev < 64 && !dev_done[dev]) {
        void *rp = NULL, *ep = NULL;
        if (swiglu_ok) {
            const size_t rb = sizeof(uint64_t) << (23 - RCP_BLK_BITS);
            e = hipMalloc(&rp, rb);
            if (e == hipSuccess && exp_delta) e = hipMalloc(&ep, (size_t)1 << 28);
            if (e == hipSuccess) e = hipMemcpy(rp, rcp_blk, rb, hipMemcpyHostToDevice);
            if (e == hipSuccess && exp_delta) e = hipMemcpy(ep, exp_delta, (size_t)1 << 28, hipMemcpyHostToDevice);
            if (e != hipSuccess) {
                if (rp) hipFree(rp);
                if (ep) hipFree(ep);
                rc = gw_hip_fail(err, errlen, "the SwiGLU tables", e);
            }
        }
        if (rc == RQ_OK) {
            int k = gw_k_set_exact(rsq_tab, rsq_bits, (const uint64_t *)rp, (const uint8_t *)ep);
            if (!k) k = gw_v_set_exact(rsq_tab, rsq_bits, (const uint64_t *)rp, (const uint8_t *)ep);
            if (k) rc = gw_hip_fail(err, errlen, "hipMemcpyToSymbol (exact tables)", (hipError_t)k);
            else {
                dev_done[dev] = 1;
                dev_rcp[dev] = rp;
                dev_exp[dev] = ep;
            }
        }
    }
    pthread_mutex_unlock(&mu);
    return rc;
}

float gw_swiglu_tab_host(float h, float h2) {
    /* the device's swiglu_ref with the tables, on the host (checked against the reference's operations by the tests);
     * the portable definition without them */
    if (swiglu_ok < 0) swiglu_ok = swiglu_measure();
    if (swiglu_ok <= 0) {
        float x = -h;
        x = x < 80.0f ? x : 80.0f;
        x = x > -86.0f ? x : -86.0f;
        return (h * h2) * (1.0f / (1.0f + exp_cephes(x)));
    }
    float p = h * h2, x = -h;
    x = x < 80.0f ? x : 80.0f;
    uint32_t u = u_of(x), E = (u >> 23) & 0xffu;
    float d = 1.0f;
    if (!(u >> 31) || E < 132u) {
        float e = gw_exp_mvec(x);
        if (exp_delta && E >= 101u) {
            uint32_t slot = (u >> 31) ? 33u + (E - 101u) : E - 101u, idx = slot << 23 | (u & 0x7fffffu);
            int dl = (int)((exp_delta[idx >> 1] >> ((idx & 1u) * 4u)) & 15u) - 8;
            e = f_of(u_of(e) + (uint32_t)dl);
        }
        d = e + 1.0f;
    }
    uint32_t v = u_of(d);
    float r0 = f_of(gw_rcp_bits(rcp_blk, v));
    float t = r0 * (r0 * d);
    float r = (r0 + r0) - t;
    return p * r;
}

int gw_exact_mode(void) {
    /* bit 0: the reference's 1 / sqrtf reproduced; bit 1: its SwiGLU reproduced (after gw_exact_init); bit 2: with
     * libmvec's expf computed by its method everywhere (no difference table) */
    return (rsq_bits > 0) | (swiglu_ok > 0) << 1 | (swiglu_ok > 0 && !exp_delta) << 2;
}
