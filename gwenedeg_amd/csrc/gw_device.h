// Device helpers shared by the gfx950 kernel files: fp16 conversions, the reference's exp, wave reductions, the
// rmsnorm scale and the per-32 quantization (the arithmetic each cites, operation for operation).
#ifndef GW_DEVICE_H
#define GW_DEVICE_H

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

// a kernel launch that records the pending timing pair of gw_time_next_launch, if any (hipExtLaunchKernel's start /
// stop events: the dispatch's own timestamps)
#define GW_LAUNCH(K, G, B, LDS, S, ...)                                                                                 \
    do {                                                                                                                \
        hipEvent_t e0_, e1_;                                                                                            \
        gw_take_launch_events(&e0_, &e1_);                                                                              \
        hipExtLaunchKernelGGL(K, G, B, (uint32_t)(LDS), S, e0_, e1_, 0, __VA_ARGS__);                                   \
    } while (0)

#define ATT_T 16
#define ATT_P 256

// The reference's host-specific operations, reproduced from tables measured on the host (gw_exact.c; installed into
// every file of kernels by gw_exact_init through gw_k_set_exact / gw_v_set_exact):
//   rsqrt_ref(t): its 1.0f / sqrtf(t) = r0 = rsqrtss(t) (the CPU's estimate: gw_rsqrt_tab, 2^bits values for t in
//     [1, 4) by exponent parity and leading mantissa bits, exact up to the power of 4) and one Newton step
//     r = fma(t r0, r0, -3) (r0 * -0.5); bits 0: IEEE 1 / sqrtf
//   swiglu_ref(h, h2): its SwiGLU (forward.c:1953-1958, vectorized): x = min(-h, 80), e = libmvec expf(x) (exp_mvec:
//     its published method, equal to the host's on every input the host checked; else plus the measured ulp difference,
//     gw_exp_delta), d = 1 + e, r0 = vrcp14ps(d) (by mantissa from gw_rcp_blk, one
//     64-bit word per 128 mantissas: vrcp14ps on [1, 2) is a non-increasing step function with at most one step per
//     such block, checked for every mantissa on the host; exact up to the power of 2), r = (r0 + r0) - r0 (r0 d),
//     (h h2) r; without the tables (a host without AVX-512): (h h2) * (1 / (1 + exp_att(min(-h, 80)))), the portable
//     definition
#define GW_RSQRT_MAXBITS 14
static __constant__ float gw_rsqrt_tab[1 << GW_RSQRT_MAXBITS];
static __constant__ int gw_rsqrt_bits;
static __constant__ const uint64_t *gw_rcp_blk;
static __constant__ const uint8_t *gw_exp_delta;

__device__ __forceinline__ float rsqrt_ref(float t) {
    const int bits = gw_rsqrt_bits;
    if (!bits) return 1.0f / sqrtf(t);
    uint32_t u = __float_as_uint(t);
    int e = (int)(u >> 23) - 127, par = e & 1;
    float r1 = gw_rsqrt_tab[(((uint32_t)par << 23) | (u & 0x7fffffu)) >> (24 - bits)];
    float r0 = __uint_as_float(__float_as_uint(r1) - (uint32_t)(((e - par) >> 1) << 23));
    float a = t * r0;
    float b = __builtin_fmaf(a, r0, -3.0f);
    return b * (r0 * -0.5f);
}

__device__ __forceinline__ float h2f(uint16_t h) {
    // IEEE half -> float (exact; v_cvt_f32_f16)
    return __half2float(__ushort_as_half(h));
}

__device__ __forceinline__ uint16_t f2h_ref(float f) {
    // fp32 -> f16 as the reference's f32_f16 (forward.c:1325-1344): RNE, >= 65520 saturates to 65504, NaN quiet
    uint32_t u = __float_as_uint(f);
    uint32_t sign = (u >> 16) & 0x8000u, a = u & 0x7fffffffu;
    uint32_t n = a - 0x38000000u;
    uint32_t h = (n + 0xfffu + ((n >> 13) & 1)) >> 13;
    float fs = __uint_as_float(a < 0x38800000u ? a : 0u);
    uint32_t sub = (uint32_t)rintf(fs * 16777216.0f);
    h = a < 0x38800000u ? sub : h;
    h = a >= 0x477ff000u ? 0x7bffu : h;
    h = a > 0x7f800000u ? (0x7e00u | ((a >> 13) & 0x3ffu)) : h;
    return (uint16_t)(sign | h);
}

__device__ __forceinline__ uint16_t f2bf_ref(float f) {
    // fp32 -> bf16 as the reference's f32_bf16 (kernels_avx512.h:60-69): round to nearest even, NaN quiet
    uint32_t u = __float_as_uint(f);
    uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
    return (uint16_t)((u & 0x7fffffffu) > 0x7f800000u ? (u >> 16) | 0x40u : r);
}

__device__ __forceinline__ float bf2f(uint32_t h) { return __uint_as_float(h << 16); } // (h < 2^16: exact)

// The 16-bit KV caches inside a tile of 16 positions j (forward.c:1901-1951): f16 K at [i][j], V rows [j][i]; bf16
// (RQ_KV_BF16) K in dim pairs, dims 2p, 2p + 1 of position j at 32 p + 2 j (+ 1), V rows with dims 32 c + l and
// 32 c + 16 + l (l < 16) at 32 c + 2 l (+ 1). Offsets in 16-bit elements
__device__ __forceinline__ int kv_k_at(bool bf, int i, int j) { return bf ? (i & ~1) * 16 + 2 * j + (i & 1) : i * 16 + j; }
__device__ __forceinline__ int kv_v_col(bool bf, int i) { return bf ? (i & ~31) + 2 * (i & 15) + ((i >> 4) & 1) : i; }

__device__ __forceinline__ float exp_att(float x) {
    // forward.c:1301-1321 (att512_exp): Cephes-style expf, x clamped at -86
    x = x > -86.0f ? x : -86.0f;
    float n = rintf(x * 1.44269504088896341f);
    float r = __builtin_fmaf(n, -0.693359375f, x);
    r = __builtin_fmaf(n, 2.12194440e-4f, r);
    float z = r * r;
    float y = 1.9875691500e-4f;
    y = __builtin_fmaf(y, r, 1.3981999507e-3f);
    y = __builtin_fmaf(y, r, 8.3334519073e-3f);
    y = __builtin_fmaf(y, r, 4.1665795894e-2f);
    y = __builtin_fmaf(y, r, 1.6666665459e-1f);
    y = __builtin_fmaf(y, r, 5.0000001201e-1f);
    y = __builtin_fmaf(y, z, r);
    y = y + 1.0f;
    return __uint_as_float(__float_as_uint(y) + ((uint32_t)(int32_t)n << 23));
}

__device__ __forceinline__ float silu_exp(float x) { return exp_att(x < 80.0f ? x : 80.0f); }

__device__ __forceinline__ float exp_mvec(float x) {
    // glibc libmvec's expf (its AVX-512 method: shifter rounding, ln2 in two parts, degree-5 Horner polynomial, 2^n by
    // the exponent field), for x in [-32, 80]: gw_exact.c's gw_exp_mvec, operation for operation
    const float sh = 12582912.0f;
    float n = __builtin_fmaf(x, __uint_as_float(0x3fb8aa3bu), sh) - sh;
    float r = __builtin_fmaf(-n, __uint_as_float(0x3f317200u), x);
    r = __builtin_fmaf(-n, __uint_as_float(0x35bfbe8eu), r);
    float p = __uint_as_float(0x3c07d9feu);
    p = __builtin_fmaf(p, r, __uint_as_float(0x3d2b8392u));
    p = __builtin_fmaf(p, r, __uint_as_float(0x3e2aacacu));
    p = __builtin_fmaf(p, r, __uint_as_float(0x3effff34u));
    p = __builtin_fmaf(p, r, __uint_as_float(0x3f7ffffeu));
    p = __builtin_fmaf(p, r, 1.0f);
    return __uint_as_float(__float_as_uint(p) + ((uint32_t)(int32_t)n << 23));
}

__device__ __forceinline__ float swiglu_ref(float h, float h2) {
    const uint64_t *rt = gw_rcp_blk;
    const uint8_t *et = gw_exp_delta;
    if (!rt) {
        float ex = silu_exp(-h);
        float r = 1.0f / (1.0f + ex);
        return (h * h2) * r;
    }
    float p = h * h2;
    float x = -h;
    x = x < 80.0f ? x : 80.0f;
    uint32_t u = __float_as_uint(x), E = (u >> 23) & 0xffu;
    float d = 1.0f; // (x <= -32: e < 2^-24, 1 + e = 1)
    if (!(u >> 31) || E < 132u) {
        float e = exp_mvec(x);
        if (et && E >= 101u) { // (a host whose libmvec differs: the tabulated binades, |x| >= 2^-26)
            uint32_t slot = (u >> 31) ? 33u + (E - 101u) : E - 101u, idx = slot << 23 | (u & 0x7fffffu);
            int dl = (int)((et[idx >> 1] >> ((idx & 1u) * 4u)) & 15u) - 8;
            e = __uint_as_float(__float_as_uint(e) + (uint32_t)dl);
        }
        d = e + 1.0f;
    }
    const uint32_t v = __float_as_uint(d), m = v & 0x7fffffu;
    const uint64_t w = rt[m >> 7];
    const uint32_t a = (m & 127u) < (uint32_t)(w >> 48) ? (uint32_t)w : (uint32_t)(w >> 24);
    float r0 = __uint_as_float(0x3f000000u + (a & 0xffffffu) - (((v >> 23) - 127u) << 23));
    float t = r0 * (r0 * d);
    float r = (r0 + r0) - t;
    return p * r;
}

// swiglu_ref of N values in place (v[k] = swiglu_ref(v[k], v2[k])), the same operations, the branch on e a select and
// the N table reads issued together (as separate calls, each read waited for before the next value's); a host with a
// difference table (gw_exp_delta) or without the tables takes swiglu_ref per value
template <int N>
__device__ __forceinline__ void swiglu_ref_n(float (&v)[N], const float (&v2)[N]) {
    const uint64_t *rt = gw_rcp_blk;
    if (!rt || gw_exp_delta) {
        #pragma unroll
        for (int k = 0; k < N; k++) v[k] = swiglu_ref(v[k], v2[k]);
        return;
    }
    float d[N];
    uint64_t w[N];
    #pragma unroll
    for (int k = 0; k < N; k++) {
        float x = -v[k];
        x = x < 80.0f ? x : 80.0f;
        const uint32_t u = __float_as_uint(x), E = (u >> 23) & 0xffu;
        const float e = exp_mvec(x); // (x <= -32: unused, d = 1)
        d[k] = !(u >> 31) || E < 132u ? e + 1.0f : 1.0f;
    }
    #pragma unroll
    for (int k = 0; k < N; k++) w[k] = rt[(__float_as_uint(d[k]) & 0x7fffffu) >> 7];
    #pragma unroll
    for (int k = 0; k < N; k++) {
        const uint32_t b = __float_as_uint(d[k]), m = b & 0x7fffffu;
        const uint32_t a = (m & 127u) < (uint32_t)(w[k] >> 48) ? (uint32_t)w[k] : (uint32_t)(w[k] >> 24);
        const float r0 = __uint_as_float(0x3f000000u + (a & 0xffffffu) - (((b >> 23) - 127u) << 23));
        const float t = r0 * (r0 * d[k]);
        const float r = (r0 + r0) - t;
        v[k] = (v[k] * v2[k]) * r;
    }
}

__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

#define GW_RSRC_DW3 0x00020000 // buffer descriptor word 3 of gfx9-family targets (raw loads; out-of-range reads give 0)

// lane Q's value of each lane's quad of 4 neighbouring lanes (a DPP quad_perm move: no LDS, no address)
template <int Q>
__device__ __forceinline__ float quad_lane(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), Q * 0x55, 0xF, 0xF, false));
}

// The rmsnorm's 16 sum-of-squares chains (forward.c:886-901: chain j an fma chain over x[j], x[j + 16], ..., then the
// tree +8 +4 +2 +1) from the chains' LDS layout: value e of the row at [(e % 16) (4 NF + 4) + e / 16] (chain j's values
// contiguous, the 16 chains 4 banks apart), NF = rms_nf(n / 64) float4s per chain, zeros from n / 16 to 4 NF.
__host__ __device__ __forceinline__ int rms_nf(int n4) {
    return n4 <= 16 ? 16 : n4 <= 32 ? 32 : n4 <= 64 ? 64 : n4 <= 128 ? 128 : 256;
}

// one chain: ss = fma(v, v, ss) over its NF float4s in order, straight-line: a ring of 8 float4 reads at immediate
// offsets, each register's next read issued right after its four fmas, so a read has the other seven registers' 28 fmas
// to land. The reads, their waits and the fmas are inline asm in the order written (the compiler otherwise issued a
// chain's reads ahead of its fmas, even volatile ones); each wait names its register, so that register's fmas come
// after it. The zeros past the chain's end change no bit: fma(0, 0, ss) == ss for every ss >= 0. (Measured per chain
// of 64 float4s on one wave: 1.9 us for two sets of 16 reads taking turns, 1.1 us for this ring, 0.7 us for the fmas
// alone)
typedef float rms_f4 __attribute__((ext_vector_type(4)));
template <int NF>
__device__ __forceinline__ float rms_chain(const float4 *c) {
    const uint32_t base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)c;
    float ss = 0.0f;
    rms_f4 q[8];
    #pragma unroll
    for (int u = 0; u < 8; u++) asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(q[u]) : "v"(base), "i"(16 * u));
    #pragma unroll
    for (int i = 0; i < NF; i++) {
        // (reads issued after read i: i + 1 .. min(i + 7, NF - 1))
        const int later = NF - 1 - i < 7 ? NF - 1 - i : 7;
        asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(q[i & 7]) : "i"(later));
        const rms_f4 v = q[i & 7];
        asm volatile("v_fmac_f32 %0, %1, %1\n\tv_fmac_f32 %0, %2, %2\n\tv_fmac_f32 %0, %3, %3\n\tv_fmac_f32 %0, %4, %4"
                     : "+v"(ss) : "v"(v.x), "v"(v.y), "v"(v.z), "v"(v.w));
        if (i + 8 < NF) asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(q[i & 7]) : "v"(base), "i"(16 * (i + 8)));
    }
    return ss;
}

// the rmsnorm scale of a row of n floats (n % 64 == 0) in the chains' layout, by lanes 0..15 of the calling wave (all
// 64 lanes active), returned to every lane: the 16 chains, the tree by DPP row shifts (row_shl:w, lane j + w of the
// same 16-lane row: lane 0's value is that of ss + shfl_down(ss, w) for w = 8, 4, 2, 1), t = fma(ss, 1/n, 1e-6),
// rsqrt_ref(t)
__device__ __forceinline__ float rms_scale_t(const float *lds, int n) {
    const int lane = threadIdx.x & 63, NF = rms_nf(n >> 6);
    float ss = 0.0f;
    if (lane < 16) {
        const float4 *c = (const float4 *)lds + lane * (NF + 1);
        if (NF == 16) ss = rms_chain<16>(c);
        else if (NF == 32) ss = rms_chain<32>(c);
        else if (NF == 64) ss = rms_chain<64>(c);
        else if (NF == 128) ss = rms_chain<128>(c);
        else ss = rms_chain<256>(c);
    }
    ss = ss + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(ss), 0x108, 0xF, 0xF, true));
    ss = ss + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(ss), 0x104, 0xF, 0xF, true));
    ss = ss + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(ss), 0x102, 0xF, 0xF, true));
    ss = ss + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(ss), 0x101, 0xF, 0xF, true));
    float r = 0.0f;
    if (lane == 0) r = rsqrt_ref(__builtin_fmaf(ss, 1.0f / (float)n, 1e-6f));
    return __shfl(r, 0);
}

// rmsnorm scale of n floats in LDS (n % 128 == 0), computed by lanes 0..15 of the calling wave, returned to all lanes
// of that wave: forward.c:886-901 in the reference's compiled order (lane j: an fma chain over x[j], x[j + 16], ...,
// the tree +8 +4 +2 +1, t = fma(ss, 1/n, 1e-6), rsqrt_ref(t)); n % 16 == 0. The chain's next 16 LDS reads are
// issued before the current 16 fmas
__device__ __forceinline__ float rms_scale_lds(const float *xs_lds, int n) {
    int lane = threadIdx.x & 63;
    float s = 0.0f;
    if (lane < 16) {
        const float *p = xs_lds + lane;
        int len = n >> 4, j = 0; // the chain's length (n % 16 == 0)
        if (len >= 16) {
            float a[16];
            #pragma unroll
            for (int u = 0; u < 16; u++) a[u] = p[16 * u];
            for (j = 16; j + 16 <= len; j += 16) {
                float b[16];
                #pragma unroll
                for (int u = 0; u < 16; u++) b[u] = p[16 * (j + u)];
                #pragma unroll
                for (int u = 0; u < 16; u++) s = __builtin_fmaf(a[u], a[u], s);
                #pragma unroll
                for (int u = 0; u < 16; u++) a[u] = b[u];
            }
            #pragma unroll
            for (int u = 0; u < 16; u++) s = __builtin_fmaf(a[u], a[u], s);
        }
        for (; j < len; j++) s = __builtin_fmaf(p[16 * j], p[16 * j], s);
    }
    for (int w = 8; w >= 1; w >>= 1) {
        float o = __shfl_down(s, w);
        s = s + o;
    }
    float r = 0.0f;
    if (lane == 0) {
        float inv_n = 1.0f / (float)n;
        float t = __builtin_fmaf(s, inv_n, 1e-6f);
        r = rsqrt_ref(t);
    }
    return __shfl(r, 0);
}

// quantization with one lane per value: the 32 lanes of each half wave are one group of 32 consecutive values
// (forward.c:803-836: s = wmax * (1/127), inv = 127 / wmax, q = trunc(v * inv + copysign(0.49999997)), 0 if wmax = 0).
// The calling wave must have all 64 lanes active
__device__ __forceinline__ void quant_lane32(float v, int8_t *q, float *s) {
    float wmax = fabsf(v);
    #pragma unroll
    for (int o = 16; o >= 1; o >>= 1) {
        float t = __shfl_xor(wmax, o);
        wmax = t > wmax ? t : wmax;
    }
    if ((threadIdx.x & 31) == 0) *s = wmax * (1.0f / 127.0f);
    int32_t qi = 0;
    if (wmax > 0.0f) {
        float inv = 127.0f / wmax;
        float x = v * inv;
        qi = (int32_t)(x + copysignf(0.49999997f, x));
    }
    *q = (int8_t)qi;
}

#endif
