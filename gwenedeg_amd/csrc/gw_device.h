// Device helpers shared by the gfx950 kernel files: fp16 conversions, the reference's exp, wave reductions, the
// rmsnorm scale and the per-32 quantization (the arithmetic each cites, operation for operation).
#ifndef GW_DEVICE_H
#define GW_DEVICE_H

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#define ATT_T 16
#define ATT_P 256

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

__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

// rmsnorm scale of n floats in LDS (n % 128 == 0), computed by lanes 0..15 of the calling wave, returned to all lanes
// of that wave: forward.c:886-901 in the reference's compiled order (lane j: an fma chain over x[j], x[j + 16], ...,
// the tree +8 +4 +2 +1, t = fma(ss, 1/n, 1e-6), 1 / sqrt(t)); n % 16 == 0. The chain's next 16 LDS reads are
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
        r = 1.0f / sqrtf(t);
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
