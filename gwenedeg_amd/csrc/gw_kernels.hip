// gfx950 kernels of the forward hot path (decode GEMV, attention, norms, RoPE, SwiGLU, quantization) and their C-ABI
// launchers (gw_k_*: plain device pointers, sizes and a stream; declared in gw_internal.h).
//
// The arithmetic of every kernel is the reference's definition, operation for operation, so that results are
// bit-identical to the oracle's restatement of it (IEEE fp32, -ffp-contract=off: an FMA only where written):
//   quantize     forward.c:803-836       s = wmax * (1/127), inv = 127 / wmax, q = trunc(x * inv + copysign(0.49999997))
//   Q8_0 fold    forward.c:906-916,      exact int32 sum per group of 32; val = val + (ws * xs) * (float) isum, groups in
//                kernels_avx512.h:157    order (one lane folds one output)
//   rmsnorm      forward.c:886-901       16 fma chains (lane j: x[j], x[j+16], ...), the tree +8 +4 +2 +1,
//                                        t = fma(ss, 1/n, 1e-6), scale = rsqrt_ref(t) (the host CPU's rsqrtss +
//                                        gcc's Newton step), o = (w * x) * scale
//   RoPE         forward.c:1266-1284     x' = fma(x, c, -(y s)), y' = fma(x, s, y c); cos / sin from the host's table
//   attention    kernels_avx512.h:1109   per 256-position block: scores as 4 chunk fma chains of 32 dims added in order,
//                forward.c:1346-1431     times scale; m = max; e = exp_att(s - m); l = 16 lane chains + tree; o = fma
//                                        chain over positions in order; blocks combined in order (att_combine)
//   f16 KV       forward.c:1325-1344,    f32_f16's rounding; K transposed in 16-position tiles, V row-major
//                :1894-1951
//   SwiGLU       forward.c:1953-1958     swiglu_ref: the reference's vector expf and rcp14 + Newton (host tables)
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "gw_internal.h"

#include "gw_device.h"

// --------------------------------------------------------------------------------------- embedding

// x[b] = row tok[b] of a Q8_0 table (embed_row, forward.c:839-881): (int8) q * fp16 d, one rounding
__global__ __launch_bounds__(256) void k_embed_q8(float *__restrict__ x, int dim, const uint8_t *__restrict__ codes,
                                                  const uint16_t *__restrict__ scales, const int *__restrict__ tok) {
    int b = blockIdx.x, t = tok[b], i = blockIdx.y * 256 + threadIdx.x;
    const int8_t *q = (const int8_t *)codes + (size_t)t * dim;
    const uint16_t *s = scales + (size_t)t * (dim / 32);
    if (i < dim) x[(size_t)b * dim + i] = (float)q[i] * h2f(s[i >> 5]);
}

// ---------------------------------------------------- residual + rmsnorm + quantize (one row per block)

// row b (= sel[j] if sel, else j): x[b] += d[b] (if d), xn = rmsnorm(x[b], w); xq / xs row j = quantize(xn);
// hid row j = xn (if hid). 1024 threads, n % 32 == 0 and n <= 16384 (up to 4 float4 per thread, all loaded first);
// the row in LDS for the scale's 16 chains: in the chains' layout where n % 64 == 0 (TR: rms_scale_t), else as it is
// (rms_scale_lds)
#define NORM_T 1024
template <bool TR>
__global__ __launch_bounds__(NORM_T) void k_rmsnorm_quant(float *__restrict__ x, const float *__restrict__ d, int n,
                                                          const float *__restrict__ w, const int *__restrict__ sel,
                                                          int8_t *__restrict__ xq, float *__restrict__ xs, int ldq,
                                                          float *__restrict__ hid) {
    extern __shared__ float lds[];
    __shared__ float rsh;
    int j = blockIdx.x, b = sel ? sel[j] : j, t = threadIdx.x, n4 = n / 4;
    float4 *xr = (float4 *)(x + (size_t)b * n);
    const float4 *dr = d ? (const float4 *)(d + (size_t)b * n) : nullptr;
    const float4 *w4 = (const float4 *)w;
    float4 v[4], e[4], wv[4];
    #pragma unroll
    for (int k = 0; k < 4; k++) {
        int i = t + NORM_T * k;
        if (i < n4) {
            v[k] = xr[i];
            wv[k] = w4[i];
            if (dr) e[k] = dr[i];
        }
    }
    #pragma unroll
    for (int k = 0; k < 4; k++) {
        int i = t + NORM_T * k;
        if (i < n4) {
            if (dr) {
                v[k].x = v[k].x + e[k].x;
                v[k].y = v[k].y + e[k].y;
                v[k].z = v[k].z + e[k].z;
                v[k].w = v[k].w + e[k].w;
                xr[i] = v[k];
            }
            if (TR) { // (element 4 i + c: chain 4 (i % 4) + c, position i / 4)
                const int LS = 4 * rms_nf(n >> 6) + 4, p = i >> 2, c0 = 4 * (i & 3);
                lds[(c0 + 0) * LS + p] = v[k].x;
                lds[(c0 + 1) * LS + p] = v[k].y;
                lds[(c0 + 2) * LS + p] = v[k].z;
                lds[(c0 + 3) * LS + p] = v[k].w;
            } else {
                ((float4 *)lds)[i] = v[k];
            }
        }
    }
    if (TR) { // (the chains' zeros: positions n / 16 .. 4 NF - 1)
        const int NF = rms_nf(n >> 6), LS = 4 * NF + 4, zc = 4 * NF - (n >> 4);
        for (int z = t; z < 16 * zc; z += NORM_T) lds[(z / zc) * LS + (n >> 4) + z % zc] = 0.0f;
    }
    __syncthreads();
    if (t < 64) {
        float r = TR ? rms_scale_t(lds, n) : rms_scale_lds(lds, n);
        if (t == 0) rsh = r;
    }
    __syncthreads();
    float r = rsh;
    // quantize: element e = 4 i + c of float4 i = t + 1024 k; its group's 32 values are 8 consecutive threads' float4s:
    // the group max over those 8 lanes, one byte per value
    #pragma unroll
    for (int k = 0; k < 4; k++) {
        int i = t + NORM_T * k;
        if (i < n4) {
            float o[4] = { (wv[k].x * v[k].x) * r, (wv[k].y * v[k].y) * r, (wv[k].z * v[k].z) * r, (wv[k].w * v[k].w) * r };
            if (hid) ((float4 *)(hid + (size_t)j * n))[i] = make_float4(o[0], o[1], o[2], o[3]);
            float wm = fmaxf(fmaxf(fabsf(o[0]), fabsf(o[1])), fmaxf(fabsf(o[2]), fabsf(o[3])));
            #pragma unroll
            for (int sft = 4; sft >= 1; sft >>= 1) {
                float tt = __shfl_xor(wm, sft);
                wm = tt > wm ? tt : wm;
            }
            if ((t & 7) == 0) xs[(size_t)j * (ldq / 32) + (i >> 3)] = wm * (1.0f / 127.0f);
            uint32_t pk = 0;
            if (wm > 0.0f) {
                float inv = 127.0f / wm;
                #pragma unroll
                for (int c = 0; c < 4; c++) {
                    float y = o[c] * inv;
                    int32_t qi = (int32_t)(y + copysignf(0.49999997f, y));
                    pk |= ((uint32_t)qi & 0xffu) << (8 * c);
                }
            }
            *(uint32_t *)(xq + (size_t)j * ldq + 4 * i) = pk;
        }
    }
}

// ------------------------------------------------------------------------------------- Q8_0 GEMV

// ------------------------------------------------------------------- QK-norm + RoPE + KV cache store

// one 64-lane block per (row, head): heads 0..nh-1 the query heads (rmsnorm with qn, RoPE, in place), nh..nh+nkv-1
// the key heads (rmsnorm with kn, RoPE, f16 into the K cache), then the value heads (f16 into the V cache).
// qkv row b: [q (nh hd) | k (nkv hd) | v (nkv hd)]; rope: cos / sin rows per position (hd floats: cos then sin).
// Caches: row b's layer base kc[b] / vc[b] (f16, the tiled layout of forward.c:1894-1899)
// ---- the 8-bit / 4-bit KV caches (RQ_KV_Q8, RQ_KV_Q4, RQ_KV_Q4K4; forward.c:1609-1790). A position's key and value
// rows are rotated, x' = H D x (D: the signs kvq_neg, H: the unnormalized Walsh-Hadamard butterflies h = 1, 2, .. in that
// order, each output one fp32 add or subtract), then quantized per 32 dims from the group's values alone (q8: d = bf16
// of max |x'| / 127, its magnitude rounded up, n = rint(x' (1 / d)) in -127..127; q4: m = the first x' of largest |x'|,
// d = bf16 of m / -8 rounded up in magnitude, n = rint(x' (1 / d)) in -8..7; d zero or denormal: the group is zero), read
// back as n d (exact). The attention runs on q' = H D q / hd (rotated in k_qknorm_rope_store) and the values read
// back, and its output o' comes back as o = D H o' / hd (k_unrot_quant). Tiles (16 positions j x hd dims i):
//   K q8 [i][j] int8, the bf16 scales at 16 hd: [c][j];  K q4: byte [p][j] = (n_2p + 8) | (n_2p+1 + 8) << 4, scales at
//   8 hd; V q8 [j][i] int8, scales at 16 hd: [j][c];  V q4: byte [j][c][l] = (n_32c+l + 8) | (n_32c+16+l + 8) << 4,
//   scales at 8 hd: [j][c]
// The dot-product types (runq.h:214, KV_DOT 4: 5 bf16-dot, 6 f16-dot, 7 q8-dot, 12 q4-dot, 13 q4k4-dot) keep their base
// type's cache (kv_base), but for the bf16-dot V: position pairs, dim i of positions 2m, 2m + 1 of a tile at 2m hd + 2i
// (+ 1) (forward.c:1916-1924)
__device__ __forceinline__ bool kv_dot(int kvt) { return kvt == 5 || kvt == 6 || kvt == 7 || kvt == 12 || kvt == 13; }
__device__ __forceinline__ int kv_base(int kvt) { return kv_dot(kvt) ? kvt & ~4 : kvt; }
__device__ __forceinline__ bool kvq_type(int kvt) { const int b = kv_base(kvt); return b == 3 || b == 8 || b == 9; }
__device__ __forceinline__ bool kvq_q4(int kvt, bool is_v) { // (the half's format)
    const int b = kv_base(kvt);
    return b == 9 || (b == 8 && is_v);
}
__device__ __forceinline__ int kvq_tile_bytes(bool q4, int hd) { return hd * (q4 ? 9 : 17); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// x (hd values in LDS) <- H D x (inv false) or D H x (inv true) by the block's 64 threads
__device__ void kvq_rot_lds(float *x, int n, bool inv) {
    const int t = threadIdx.x;
    if (!inv) {
        for (int i = t; i < n; i += 64)
            if ((((uint32_t)i * 0x9E3779B9u) >> 31) != 0u) x[i] = -x[i];
        __syncthreads();
    }
    for (int h = 1; h < n; h *= 2) {
        for (int k = t; k < n / 2; k += 64) {
            const int i = (k / h) * 2 * h + k % h;
            const float a = x[i], b = x[i + h];
            x[i] = a + b;
            x[i + h] = a - b;
        }
        __syncthreads();
    }
    if (inv) {
        for (int i = t; i < n; i += 64)
            if ((((uint32_t)i * 0x9E3779B9u) >> 31) != 0u) x[i] = -x[i];
        __syncthreads();
    }
}

// the rotated row x (hd values in LDS) quantized into position j of a q8 / q4 tile (K: is_v false), by the block's 64
// threads; sc: LDS scratch of hd / 32 words
__device__ void kvq_store_lds(const float *x, int hd, bool q4, bool is_v, uint8_t *tile, int j, uint32_t *sc) {
    const int t = threadIdx.x, ng = hd >> 5;
    if (t < ng) { // the group's scale: the first value of largest magnitude (q4), the largest magnitude (q8)
        float a = 0.0f, m = 0.0f;
        for (int i = 0; i < 32; i++)
            if (fabsf(x[32 * t + i]) > a) {
                a = fabsf(x[32 * t + i]);
                m = x[32 * t + i];
            }
        const float d = q4 ? m / -8.0f : a / 127.0f;
        const uint32_t u = __float_as_uint(d), r = (u >> 16) + ((u & 0xffffu) != 0u);
        const uint16_t s16 = (r & 0x7f80u) ? (uint16_t)r : (uint16_t)0;
        sc[t] = s16;
        uint16_t *so = (uint16_t *)(tile + (size_t)(q4 ? 8 : 16) * hd) + (is_v ? j * ng + t : t * ATT_T + j);
        *so = s16;
    }
    __syncthreads();
    auto level = [&](int i) -> int { // (rint(x (1 / d)): the reference's build multiplies by the group's reciprocal)
        const uint32_t s16 = sc[i >> 5];
        const float d = bf16_to_f32((uint16_t)s16), tq = s16 ? __builtin_rintf(x[i] * (1.0f / d)) : 0.0f;
        const float lo = q4 ? -8.0f : -127.0f, hi = q4 ? 7.0f : 127.0f;
        return tq < lo ? (int)lo : tq > hi ? (int)hi : (int)tq;
    };
    if (!q4) {
        for (int i = t; i < hd; i += 64) tile[is_v ? (size_t)j * hd + i : (size_t)i * ATT_T + j] = (uint8_t)(int8_t)level(i);
    } else if (!is_v) {
        for (int p2 = t; p2 < hd / 2; p2 += 64)
            tile[(size_t)p2 * ATT_T + j] = (uint8_t)((level(2 * p2) + 8) | (level(2 * p2 + 1) + 8) << 4);
    } else {
        for (int k = t; k < hd / 2; k += 64) { // (byte 16 c + l of the position: dims 32 c + l and 32 c + 16 + l)
            const int c = k >> 4, l = k & 15;
            tile[(size_t)j * (hd / 2) + k] = (uint8_t)((level(32 * c + l) + 8) | (level(32 * c + 16 + l) + 8) << 4);
        }
    }
}

// the tile of position p, kv head g of a layer's quantized cache (base: the layer's first byte)
__device__ __forceinline__ uint8_t *kvq_tile(void *base, int p, int g, int nkv, int hd, bool q4) {
    const size_t nt = ((size_t)(p / ATT_P) * nkv + g) * (ATT_P / ATT_T) + (size_t)(p % ATT_P / ATT_T);
    return (uint8_t *)base + nt * (size_t)kvq_tile_bytes(q4, hd);
}

// rows' QK-norm + RoPE and the K / V store (forward.c:1266-1284, :1901-1951); kvt: each row's cache type (runq.h:214;
// NULL: all f16). A quantized row's query heads are rotated in place (q' = H D q / hd) and its key / value rows stored
// rotated and quantized
__global__ __launch_bounds__(64) void k_qknorm_rope_store(float *__restrict__ qkv, int ldqkv, int nh, int nkv, int hd,
                                                          const float *__restrict__ qn, const float *__restrict__ kn,
                                                          const float *__restrict__ rope, const int *__restrict__ pos,
                                                          uint16_t *const *__restrict__ kc, uint16_t *const *__restrict__ vc,
                                                          const int *__restrict__ kvt) {
    __shared__ float v[256];
    __shared__ uint32_t scw[8];
    int b = blockIdx.x, h = blockIdx.y, lane = threadIdx.x, p = pos[b];
    const int kt = kvt ? kvt[b] : 2;
    const bool bf = kv_base(kt) == 1, qz = kvq_type(kt), f32 = kt == 0; // (row b's cache: bf16 / quantized / f32)
    float *row = qkv + (size_t)b * ldqkv;
    int half = hd / 2;
    if (qz && h >= nh + nkv) { // value head: rotated and quantized
        int g = h - nh - nkv;
        const float *src = row + (size_t)(nh + nkv) * hd + g * hd;
        for (int i = lane; i < hd; i += 64) v[i] = src[i];
        __syncthreads();
        kvq_rot_lds(v, hd, false);
        kvq_store_lds(v, hd, kvq_q4(kt, true), true, kvq_tile(vc[b], p, g, nkv, hd, kvq_q4(kt, true)), p % ATT_T, scw);
        return;
    }
    if (h >= nh + nkv) { // value head: store
        int g = h - nh - nkv;
        const float *src = row + (size_t)(nh + nkv) * hd + g * hd;
        const size_t o = (((size_t)(p / ATT_P) * nkv + g) * ATT_P + (size_t)(p % ATT_P / ATT_T) * ATT_T) * hd;
        uint16_t *dst = vc[b] + o;
        const int j = p % ATT_T;
        if (f32) // (V [j][i] floats)
            for (int i = lane; i < hd; i += 64) ((float *)vc[b])[o + (size_t)j * hd + i] = src[i];
        else if (kt == 5) // (bf16-dot: position pairs)
            for (int i = lane; i < hd; i += 64) dst[(size_t)(j & ~1) * hd + 2 * i + (j & 1)] = f2bf_ref(src[i]);
        else
            for (int i = lane; i < hd; i += 64) dst[(size_t)j * hd + kv_v_col(bf, i)] = bf ? f2bf_ref(src[i]) : f2h_ref(src[i]);
        return;
    }
    float *src = row + (size_t)h * hd;
    for (int i = lane; i < hd; i += 64) v[i] = src[i];
    __syncthreads();
    float r = rms_scale_lds(v, hd);
    const float *w = h < nh ? qn : kn;
    const float *cs = rope + (size_t)p * hd;
    for (int i = lane; i < half; i += 64) {
        float x = (w[i] * v[i]) * r, y = (w[i + half] * v[i + half]) * r;
        float c = cs[i], s = cs[i + half];
        float ys = y * s, yc = y * c;
        float xo = __builtin_fmaf(x, c, -ys), yo = __builtin_fmaf(x, s, yc);
        if (qz) { // (rotated below: each thread rewrites only the values it read)
            v[i] = xo;
            v[i + half] = yo;
        } else if (h < nh) {
            src[i] = xo;
            src[i + half] = yo;
        } else {
            int g = h - nh;
            const size_t o = (((size_t)(p / ATT_P) * nkv + g) * ATT_P + (size_t)(p % ATT_P / ATT_T) * ATT_T) * hd;
            if (f32) { // (K [i][j] floats)
                ((float *)kc[b])[o + (size_t)i * ATT_T + p % ATT_T] = xo;
                ((float *)kc[b])[o + (size_t)(i + half) * ATT_T + p % ATT_T] = yo;
            } else {
                uint16_t *dst = kc[b] + o;
                dst[kv_k_at(bf, i, p % ATT_T)] = bf ? f2bf_ref(xo) : f2h_ref(xo);
                dst[kv_k_at(bf, i + half, p % ATT_T)] = bf ? f2bf_ref(yo) : f2h_ref(yo);
            }
        }
    }
    if (qz) {
        __syncthreads();
        kvq_rot_lds(v, hd, false);
        if (h < nh) { // q' = H D q / hd (1 / hd: a power of two, exact)
            const float f = 1.0f / (float)hd;
            for (int i = lane; i < hd; i += 64) src[i] = v[i] * f;
        } else {
            const int g = h - nh;
            kvq_store_lds(v, hd, kvq_q4(kt, false), false, kvq_tile(kc[b], p, g, nkv, hd, kvq_q4(kt, false)), p % ATT_T, scw);
        }
    }
}

// synthetic rows of the quantized and f32 caches (rq_seq_fill_synthetic): block (position p, kv head g, K / V) draws hd
// values (|K| < 3.9, |V| < 0.99) from a hash of (seed, p, g, K / V, dim) and stores them as k_qknorm_rope_store does
__global__ __launch_bounds__(64) void k_fill_synthetic_q(void *kc, void *vc, int kvt, int nkv, int hd, unsigned long long seed) {
    __shared__ float v[256];
    __shared__ uint32_t scw[8];
    const int p = blockIdx.x, g = blockIdx.y, isv = blockIdx.z;
    for (int i = threadIdx.x; i < hd; i += 64) {
        unsigned long long z = seed + (((unsigned long long)p * nkv + g) * 2 + isv) * 0x100000001b3ull + (unsigned long long)i * 0x9e3779b97f4a7c15ull;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        z ^= z >> 31;
        const float a = (float)(z & 0xffffff) * (1.0f / 16777216.0f);
        v[i] = (2.0f * a - 1.0f) * (isv ? 0.99f : 3.9f);
    }
    if (kvt == 0) { // (f32: K [i][j], V [j][i] floats, not rotated)
        float *t = (float *)(isv ? vc : kc) + (((size_t)(p / ATT_P) * nkv + g) * ATT_P + (size_t)(p % ATT_P / ATT_T) * ATT_T) * hd;
        for (int i = threadIdx.x; i < hd; i += 64) t[isv ? (size_t)(p % ATT_T) * hd + i : (size_t)i * ATT_T + p % ATT_T] = v[i];
        return;
    }
    __syncthreads();
    kvq_rot_lds(v, hd, false);
    const bool q4 = kvq_q4(kvt, isv != 0);
    kvq_store_lds(v, hd, q4, isv != 0, kvq_tile(isv ? vc : kc, p, g, nkv, hd, q4), p % ATT_T, scw);
}

// the rows of quantized caches: their attention output o' (att: rows of nh hd values) back to o = D H o' / hd, then
// quantized for wo as k_attn_combine_quant quantizes (aq / as rows of ldq codes); other rows are left as they are
__global__ __launch_bounds__(64) void k_unrot_quant(const float *__restrict__ att, int nh, int hd, const int *__restrict__ kvt,
                                                    int8_t *__restrict__ aq, float *__restrict__ as, int ldq) {
    __shared__ float v[256];
    const int b = blockIdx.x, h = blockIdx.y, t = threadIdx.x;
    if (!kvq_type(kvt[b])) return;
    const float *src = att + ((size_t)b * nh + h) * hd;
    for (int i = t; i < hd; i += 64) v[i] = src[i];
    __syncthreads();
    kvq_rot_lds(v, hd, true);
    const float f = 1.0f / (float)hd;
    for (int i = t; i < hd; i += 64) { // (hd % 64 == 0 or hd = 32: whole groups of 32 lanes)
        const int e = h * hd + i;
        if (i < hd) quant_lane32(v[i] * f, aq + (size_t)b * ldq + e, as + (size_t)b * (ldq / 32) + (e >> 5));
    }
}

// ----------------------------------------------------------------------------------------- attention

// Attention on the quantized caches: one block of AQ_T threads per item (first row r0, rows nr of one sequence, kv head
// g, key block kb; the items of k_attn_part) and each of its nq = nr kv_mul query vectors q' (rotated by
// k_qknorm_rope_store) that reaches the block: the fp32 attention of the oracle's attention_block on the values read
// back (n d, exact), as forward.c:1776-1803 runs it on kvq_block_f32's copy: scores by the chunk chains of 32 dims
// (a = c0 + c1 + c2 + c3, times scale), m the max, e = exp_att(s - m), l the 16 chains over positions j % 16 and the tree,
// o the fma chain over the positions. part[(row nh + h) pstride + kb (hd + 2)] = o, m, l. The block's K tiles are staged
// into LDS, then its V tiles over them. hd <= 128 (a power of two), nq <= NQM (8 or 16). The f32 cache (RQ_KV_F32: K [i][j], V
// [j][i] floats, not rotated) runs the same fp32 attention on its values, read from HBM where they lie (its 64 KB of K
// per block would not leave room in LDS for the rest); so do the 16-bit dot-product tiles (32 KB of K per block).
// DOT: the dot-product types (every row of the launch one), attention_vec_dot (forward.c:1488-1549, kernels_avx512.h:
// 1439-1475): q, the values (16-bit caches: bf16 as stored, f16 rounded to bf16; quantized: n d rounded to bf16) and the
// weights rounded to bf16; each product pair as vdpbf16ps's lane, two fmas with the odd element first (scores: dim
// pairs; o: position pairs, a last odd position paired with +0, +0); the call's FTZ / DAZ mode as ftz_f on each
// value read and on each fma's result (fma_fz)
#define AQ_T 512
__device__ __forceinline__ float ftz_f(float x) { return fabsf(x) < 1.17549435e-38f ? __builtin_copysignf(0.0f, x) : x; }
__device__ __forceinline__ float bf16_round(float x) { return bf16_to_f32(f2bf_ref(ftz_f(x))); } // (vcvtneps2bf16)
// fma_ftz on operands already flushed (a bf16_round result, a value as the products read it, an earlier fma_fz, zero):
// only the result needs the flush
__device__ __forceinline__ float fma_fz(float a, float b, float c) { return ftz_f(__builtin_fmaf(a, b, c)); }

// the block's work for one cache type (BT: the row's base type, kv_base; LDS from the kernel), every format decision made
// at compile time, so that a batch of operand loads is one straight run of loads
template <bool DOT, int BT, int NQM>
__device__ __forceinline__ void attn_q_body(const int4 it, const float *__restrict__ qkv, int ldqkv, int nh, int nkv, int hd,
                                            float scale, const int *__restrict__ pos, uint16_t *const *__restrict__ kc,
                                            uint16_t *const *__restrict__ vc, float *__restrict__ part, int pstride,
                                            uint8_t *tl, float *qs, float (*S)[ATT_P], float *ms, float *ls) {
    const int r0 = it.x, nr = it.y, g = it.z, kb = it.w, kv_mul = nh / nkv, nq = nr * kv_mul, t = threadIdx.x;
    const int ng = hd >> 5;
    constexpr int base = BT;
    constexpr bool b16 = DOT && (BT == 1 || BT == 2); // (a 16-bit dot cache: bf16-dot, f16-dot)
    constexpr bool f32 = !DOT && BT == 0;             // (the f32 cache: read from HBM, not staged; 64 KB per block)
    constexpr bool inplace = f32 || b16;              // (f32 and 16-bit dot tiles read where they lie: the LDS holds the
                                                      // 8-bit tiles only, and two blocks fit a CU)
    constexpr bool k4 = BT == 9, v4 = BT == 9 || BT == 8;
    const int tbk = f32 ? 64 * hd : b16 ? 32 * hd : kvq_tile_bytes(k4, hd);
    const int tbv = f32 ? 64 * hd : b16 ? 32 * hd : kvq_tile_bytes(v4, hd);
    auto npos = [&](int v) -> int { // positions of block kb vector v reaches (<= 0: none)
        const int n = pos[r0 + v / kv_mul] + 1 - kb * ATT_P;
        return n < ATT_P ? n : ATT_P;
    };
    auto tile_src = [&](uint16_t *const *c, bool q4, int tb) -> const uint4 * { // (the block's first tile, head g)
        if (!b16 && !f32) return (const uint4 *)kvq_tile(c[r0], kb * ATT_P, g, nkv, hd, q4);
        return (const uint4 *)((const uint8_t *)c[r0] + ((size_t)kb * nkv + g) * (ATT_P / ATT_T) * (size_t)tb);
    };
    // the value of dim i, position j of a staged K (is_v false) or V tile tb, as the products read it
    auto value = [&](const uint8_t *tb, int i, int j, bool is_v) -> float {
        if (f32) return ((const float *)tb)[is_v ? j * hd + i : i * ATT_T + j];
        if (b16) {
            const uint16_t *u = (const uint16_t *)tb;
            if (base == 1) return ftz_f(bf16_to_f32(u[is_v ? (j & ~1) * hd + 2 * i + (j & 1) : kv_k_at(true, i, j)]));
            return bf16_round(h2f(u[is_v ? j * hd + i : kv_k_at(false, i, j)]));
        }
        const bool q4 = is_v ? v4 : k4;
        const int c = i >> 5;
        float d;
        int n;
        if (!is_v) {
            d = bf16_to_f32(((const uint16_t *)(tb + (size_t)(q4 ? 8 : 16) * hd))[c * ATT_T + j]);
            n = q4 ? ((tb[(i >> 1) * ATT_T + j] >> (4 * (i & 1))) & 15) - 8 : (int)(int8_t)tb[i * ATT_T + j];
        } else {
            d = bf16_to_f32(((const uint16_t *)(tb + (size_t)(q4 ? 8 : 16) * hd))[j * ng + c]);
            n = q4 ? ((tb[(size_t)j * (hd / 2) + 16 * c + (i & 15)] >> (4 * ((i >> 4) & 1))) & 15) - 8
                   : (int)(int8_t)tb[(size_t)j * hd + i];
        }
        return DOT ? bf16_round((float)n * d) : (float)n * d;
    };
    // 1. the K tiles (the block's 16 tiles of head g are consecutive) and the query vectors
    const uint8_t *kt0 = inplace ? (const uint8_t *)tile_src(kc, k4, tbk) : tl;
    const uint8_t *vt0 = inplace ? (const uint8_t *)tile_src(vc, v4, tbv) : tl;
    {
        const uint4 *src = tile_src(kc, k4, tbk);
        if (!inplace)
            for (int i = t; i < ATT_T * tbk / 16; i += AQ_T) ((uint4 *)tl)[i] = src[i];
        for (int i = t; i < nq * hd; i += AQ_T) {
            const int v = i / hd, d = i % hd;
            const float q = qkv[(size_t)(r0 + v / kv_mul) * ldqkv + (size_t)(g * kv_mul + v % kv_mul) * hd + d];
            qs[d * NQM + v] = DOT ? bf16_round(q) : q;
        }
    }
    __syncthreads();
    // 2. scores: thread per (position, group of 4 vectors): each K value read once for the group's 4 chains
    // (vectors past nq, or positions past a vector's reach, computed on whatever LDS holds and not stored)
    for (int k = t; k < (nq + 3) / 4 * ATT_P; k += AQ_T) {
        const int v0 = 4 * (k / ATT_P), p = k % ATT_P;
        int reach = 0;
        #pragma unroll
        for (int u = 0; u < 4; u++)
            if (v0 + u < nq) reach = npos(v0 + u) > reach ? npos(v0 + u) : reach;
        if (p >= reach) continue;
        const uint8_t *tb = kt0 + (size_t)(p / ATT_T) * tbk;
        const int j = p % ATT_T;
        float a[4] = { 0.0f, 0.0f, 0.0f, 0.0f };
        for (int c = 0; c < ng; c++) {
            float cc[4] = { 0.0f, 0.0f, 0.0f, 0.0f };
            if (DOT) {
                for (int i = 32 * c; i < 32 * c + 32; i += 2) {
                    const float k1 = value(tb, i + 1, j, false), k0 = value(tb, i, j, false);
                    const float4 q1 = *(const float4 *)(qs + (i + 1) * NQM + v0), q0 = *(const float4 *)(qs + i * NQM + v0);
                    const float q1v[4] = { q1.x, q1.y, q1.z, q1.w }, q0v[4] = { q0.x, q0.y, q0.z, q0.w };
                    #pragma unroll
                    for (int u = 0; u < 4; u++) cc[u] = fma_fz(q0v[u], k0, fma_fz(q1v[u], k1, cc[u]));
                }
                #pragma unroll
                for (int u = 0; u < 4; u++) a[u] = c ? ftz_f(a[u] + cc[u]) : cc[u];
            } else {
                for (int i = 32 * c; i < 32 * c + 32; i++) {
                    const float kv = value(tb, i, j, false);
                    const float4 q = *(const float4 *)(qs + i * NQM + v0);
                    cc[0] = __builtin_fmaf(q.x, kv, cc[0]);
                    cc[1] = __builtin_fmaf(q.y, kv, cc[1]);
                    cc[2] = __builtin_fmaf(q.z, kv, cc[2]);
                    cc[3] = __builtin_fmaf(q.w, kv, cc[3]);
                }
                #pragma unroll
                for (int u = 0; u < 4; u++) a[u] = c ? a[u] + cc[u] : cc[u];
            }
        }
        #pragma unroll
        for (int u = 0; u < 4; u++)
            if (v0 + u < nq && p < npos(v0 + u)) S[v0 + u][p] = DOT ? ftz_f(a[u] * scale) : a[u] * scale;
    }
    __syncthreads();
    // 3. softmax: wave w takes vectors w, w + 8: m, the exponentials (DOT: rounded to bf16), l (lane j < 16: the chain
    // over positions j, j + 16, ...; then the tree)
    {
        const int wave = t >> 6, lane = t & 63;
        for (int v = wave; v < nq; v += AQ_T / 64) {
            const int n = npos(v);
            if (n <= 0) continue;
            float m = S[v][0];
            for (int p = lane; p < n; p += 64) m = S[v][p] > m ? S[v][p] : m;
            for (int o = 32; o >= 1; o >>= 1) {
                const float u = __shfl_xor(m, o);
                m = u > m ? u : m;
            }
            for (int p = lane; p < n; p += 64) {
                const float e = exp_att(S[v][p] - m);
                S[v][p] = DOT ? bf16_round(e) : e;
            }
            __builtin_amdgcn_wave_barrier();
            float sm = 0.0f;
            if (lane < 16)
                for (int p = lane; p < n; p += ATT_T) sm = sm + S[v][p];
            for (int w = 8; w >= 1; w >>= 1) {
                const float o = __shfl_down(sm, w);
                if (lane < w) sm = sm + o;
            }
            if (lane == 0) {
                ms[v] = m;
                ls[v] = sm;
            }
        }
    }
    __syncthreads();
    // 4. the V tiles over the K tiles
    if (!inplace) {
        const uint4 *src = tile_src(vc, v4, tbv);
        for (int i = t; i < ATT_T * tbv / 16; i += AQ_T) ((uint4 *)tl)[i] = src[i];
    }
    __syncthreads();
    // 5. o, thread per (dim, group of 4 vectors): each V value read once for the group's 4 fma chains over the positions
    // in order (DOT: over position pairs); the operands of 8 positions loaded before their fmas
    for (int k = t; k < (nq + 3) / 4 * hd; k += AQ_T) {
        const int v0 = 4 * (k / hd), i = k % hd, nv = nq - v0 < 4 ? nq - v0 : 4;
        int nu[4], nmin = ATT_P, nmax = 0;
        #pragma unroll
        for (int u = 0; u < 4; u++) {
            nu[u] = u < nv ? npos(v0 + u) : 0;
            if (u < nv) {
                nmin = nu[u] < nmin ? nu[u] : nmin;
                nmax = nu[u] > nmax ? nu[u] : nmax;
            }
        }
        if (nmax <= 0) continue;
        float o[4] = { 0.0f, 0.0f, 0.0f, 0.0f };
        int p = 0;
        for (; p + 8 <= nmin; p += 8) { // (p % 8 == 0: the 8 positions share a tile)
            const uint8_t *tb = vt0 + (size_t)(p / ATT_T) * tbv;
            const int j = p % ATT_T;
            float x[8], w[4][8];
            #pragma unroll
            for (int e = 0; e < 8; e++) {
                x[e] = value(tb, i, j + e, true);
                #pragma unroll
                for (int u = 0; u < 4; u++) w[u][e] = S[v0 + u][p + e]; // (rows past nq: in the array, not stored)
            }
            #pragma unroll
            for (int u = 0; u < 4; u++) {
                if (DOT) {
                    #pragma unroll
                    for (int e = 0; e < 8; e += 2) o[u] = fma_fz(w[u][e], x[e], fma_fz(w[u][e + 1], x[e + 1], o[u]));
                } else {
                    #pragma unroll
                    for (int e = 0; e < 8; e++) o[u] = __builtin_fmaf(w[u][e], x[e], o[u]);
                }
            }
        }
        if (DOT) {
            for (; p < nmax; p += 2) { // (p even: p and p + 1 share a tile; each vector to its own reach)
                const uint8_t *tb = vt0 + (size_t)(p / ATT_T) * tbv;
                const int j = p % ATT_T;
                const float x0 = value(tb, i, j, true), x1 = p + 1 < nmax ? value(tb, i, j + 1, true) : 0.0f;
                #pragma unroll
                for (int u = 0; u < 4; u++)
                    if (p < nu[u]) {
                        const float w1 = p + 1 < nu[u] ? S[v0 + u][p + 1] : 0.0f, v1 = p + 1 < nu[u] ? x1 : 0.0f;
                        o[u] = fma_fz(S[v0 + u][p], x0, fma_fz(w1, v1, o[u]));
                    }
            }
        } else {
            for (; p < nmax; p++) {
                const float x0 = value(vt0 + (size_t)(p / ATT_T) * tbv, i, p % ATT_T, true);
                #pragma unroll
                for (int u = 0; u < 4; u++)
                    if (p < nu[u]) o[u] = __builtin_fmaf(S[v0 + u][p], x0, o[u]);
            }
        }
        #pragma unroll
        for (int u = 0; u < 4; u++)
            if (u < nv && nu[u] > 0) {
                const int v = v0 + u;
                float *dst = part + ((size_t)(r0 + v / kv_mul) * nh + g * kv_mul + v % kv_mul) * pstride + (size_t)kb * (hd + 2);
                dst[i] = o[u];
                if (i == 0) {
                    dst[hd] = ms[v];
                    dst[hd + 1] = ls[v];
                }
            }
    }
}

template <bool DOT, int NQM> // (NQM: the query vectors an item may hold, 8 or 16; LDS sized by it: 8 lets 3 blocks share a CU)
__global__ __launch_bounds__(AQ_T) void k_attn_q(const int4 *__restrict__ items, const float *__restrict__ qkv, int ldqkv,
                                                 int nh, int nkv, int hd, float scale, const int *__restrict__ pos,
                                                 uint16_t *const *__restrict__ kc, uint16_t *const *__restrict__ vc,
                                                 const int *__restrict__ kvt, float *__restrict__ part, int pstride) {
    __shared__ __align__(16) uint8_t tl[ATT_T * 17 * 128]; // the block's 16 tiles of K, then of V (8-bit / 4-bit types)
    __shared__ __align__(16) float qs[128 * NQM]; // the query vectors, transposed: dim d of vector v at NQM d + v
    __shared__ float S[NQM][ATT_P];
    __shared__ float ms[NQM], ls[NQM];
    const int4 it = items[blockIdx.x];
    const int base = kv_base(kvt[it.x]); // (uniform over the block: one branch, then a body without type tests)
#define AQ_BODY(B) attn_q_body<DOT, B, NQM>(it, qkv, ldqkv, nh, nkv, hd, scale, pos, kc, vc, part, pstride, tl, qs, S, ms, ls)
    if constexpr (DOT) {
        if (base == 1) AQ_BODY(1);
        else if (base == 2) AQ_BODY(2);
        else if (base == 3) AQ_BODY(3);
        else if (base == 8) AQ_BODY(8);
        else AQ_BODY(9);
    } else {
        if (base == 0) AQ_BODY(0);
        else if (base == 3) AQ_BODY(3);
        else if (base == 8) AQ_BODY(8);
        else AQ_BODY(9);
    }
#undef AQ_BODY
}

// One block of 1024 threads per item (first row r0, rows nr of one sequence at consecutive positions, kv head g, key
// block kb): the partial result of block kb (forward.c:1346-1403 with ml) for each of the nq = nr * kv_mul query vectors
// that reach it: part[(row * nh + h) * pstride + kb * (hd + 2)] = o[hd] (unnormalized), m, l. Vector v = (row
// r0 + v / kv_mul, head g * kv_mul + v % kv_mul) over positions 0..pos(row). Steps:
//   stage: the block's K and V tiles (16-byte loads, all issued before any LDS write) and the query vectors into LDS;
//     K rows padded by 32 bytes per 32 dims, so the 4 chunks of a position read different banks
//   scores: lane (position p, chunk c): the fma chain over dims 32c .. 32c + 31 of every vector; the 4 chunks of a
//     position are neighbouring lanes, added in order (a = c0 + c1 + c2 + c3, left to right), times scale
//   softmax: one wave per vector: m = max, e = exp_att(s - m), l = 16 lane chains + the tree
//   o: lane (vector, dim pair): the fma chains over the positions in order, V from LDS (NQ = 16: its own buffer,
//     staged with K; else the K buffer, rewritten once the scores are done: a block's LDS stays under half a CU's)
// hd <= 128 (hd % 32 == 0), nq <= 16.
// a0..a7 += (q0..q7 of lane N of this lane's 16-lane row) * k: v_fmac_f32_dpp with row_newbcast, the broadcast folded
// into the fma (one rounding, as __builtin_fmaf; the compiler does not fold a separate DPP move into v_fmac). A VALU
// write of a DPP source needs 2 wait states before the read: the s_nop, whatever the compiler placed before the block
// (not volatile: the compiler schedules the K reads around the blocks)
template <int N>
__device__ __forceinline__ void fmac8_row(float &a0, float &a1, float &a2, float &a3, float &a4, float &a5, float &a6, float &a7,
                                          float q0, float q1, float q2, float q3, float q4, float q5, float q6, float q7, float k) {
    asm("s_nop 1\n\t"
                 "v_fmac_f32_dpp %0, %8, %16 row_newbcast:%17 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %1, %9, %16 row_newbcast:%17 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %2, %10, %16 row_newbcast:%17 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %3, %11, %16 row_newbcast:%17 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %4, %12, %16 row_newbcast:%17 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %5, %13, %16 row_newbcast:%17 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %6, %14, %16 row_newbcast:%17 row_mask:0xf bank_mask:0xf\n\t"
                 "v_fmac_f32_dpp %7, %15, %16 row_newbcast:%17 row_mask:0xf bank_mask:0xf"
                 : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(a4), "+v"(a5), "+v"(a6), "+v"(a7)
                 : "v"(q0), "v"(q1), "v"(q2), "v"(q3), "v"(q4), "v"(q5), "v"(q6), "v"(q7), "v"(k), "n"(N));
}

#define ATT_NQ 16
#define ATT_HDMAX 128
#define ATT_TH 1024
#define ATT_KROW 1056                   // LDS bytes of 32 K dims of a tile (32 x 32 + 32 padding)
#define ATT_KTILE (4 * ATT_KROW)        // LDS bytes of a K tile (hd <= 128)
#define ATT_QC 36                       // LDS floats per 32-dim chunk of a query vector (32 + 4 padding)
#define ATT_QS (4 * ATT_QC)             // LDS floats per query vector
template <int NQ, bool KB>
__device__ __forceinline__ void attn_part_body(const int4 *__restrict__ items, const float *__restrict__ qkv, int ldqkv, int nh,
                                               int nkv, int hd, float scale, const int *__restrict__ pos,
                                               uint16_t *const *__restrict__ kc, uint16_t *const *__restrict__ vc,
                                               float *__restrict__ part, int pstride) {
    // V staged in its own LDS buffer for NQ = 16 (prefill row blocks), else into the K buffer once the scores are done
    // (the block's LDS stays under half a CU's: two blocks per CU); its loads are issued with K's either way.
    // One LDS block: the query vectors, scores and lengths first (below 64 KiB, so every read of them is a base
    // register plus an immediate offset), then the K tiles, then (NQ = 16) V. V rows at a fixed 256-byte stride,
    // whatever hd: the o chains' reads are immediate offsets from one pointer. Up to 4 vectors (SE), the exponentials
    // go to their own array E, written by all 16 waves, and the sums l are added while the o chains run
    constexpr bool VL = NQ == 16, SE = NQ <= 4, DQ = NQ >= 8;
    constexpr int QS_B = NQ * ATT_QS * 4, S_B = NQ * ATT_P * 4, E_B = SE ? S_B : 0;
    constexpr int KS_OFF = (QS_B + S_B + E_B + NQ * 4 + 15) & ~15;
    __shared__ __align__(16) uint8_t lds[KS_OFF + 16 * ATT_KTILE + (VL ? ATT_P * 2 * ATT_HDMAX : 0)];
    float *const qs = (float *)lds;
    float (*const S)[ATT_P] = (float (*)[ATT_P])(lds + QS_B);
    float (*const E)[ATT_P] = (float (*)[ATT_P])(lds + QS_B + (SE ? S_B : 0)); // (the exponentials; S itself otherwise)
    int *const np = (int *)(lds + QS_B + S_B + E_B);
    uint8_t *const ks = lds + KS_OFF;
    uint8_t *const vs = lds + KS_OFF + 16 * ATT_KTILE; // (VL only)
    static_assert(QS_B + S_B + E_B + NQ * 4 <= 65536, "scores below 64 KiB");
    static_assert(!SE || 2 * sizeof(lds) <= 160 * 1024, "two blocks per CU");
    static_assert(16 * ATT_KTILE >= ATT_P * 2 * ATT_HDMAX, "V rows at 256 bytes fit the K buffer");
    int4 it = items[blockIdx.x];
    int r0 = it.x, nr = it.y, g = it.z, kb = it.w, kv_mul = nh / nkv, nq = nr * kv_mul, t = threadIdx.x;
    // (x / nchk = x vmg >> 16 and x / kv_mul = x kmg >> 16 for the x < 2^10 they divide here)
    const int TB = 32 * hd, nchk = hd / 32, vmg = (65536 + nchk - 1) / nchk, kmg = (65536 + kv_mul - 1) / kv_mul;
    const uint8_t *K = (const uint8_t *)(kc[r0] + ((size_t)kb * nkv + g) * ATT_P * hd);
    const uint8_t *V = (const uint8_t *)(vc[r0] + ((size_t)kb * nkv + g) * ATT_P * hd);
    int nmx = pos[r0 + nr - 1] + 1 - kb * ATT_P;
    nmx = nmx < ATT_P ? nmx : ATT_P;
    int nbytes = (nmx + ATT_T - 1) / ATT_T * TB; // the tiles holding positions < nmx
    // staging of K and V: 16 bytes per thread and round, up to 4 rounds (hd <= 128), loads issued before any use
    uint4 k0, k1, k2, k3, v0, v1, v2, v3;
#define ATT_LD(k, KR, VR)                                                                                                \
    if ((t + ATT_TH * k) * 16 < nbytes) {                                                                            \
        KR = *(const uint4 *)(K + (t + ATT_TH * k) * 16);                                                             \
        VR = *(const uint4 *)(V + (t + ATT_TH * k) * 16);                                                             \
    }
    ATT_LD(0, k0, v0) ATT_LD(1, k1, v1) ATT_LD(2, k2, v2) ATT_LD(3, k3, v3)
#undef ATT_LD
    for (int e = t; e < NQ * ATT_QS; e += ATT_TH) { // (padding and vectors past nq: zeros)
        int v = e / ATT_QS, c = e % ATT_QS / ATT_QC, i = e % ATT_QC, d = 32 * c + i, vr = v * kmg >> 16;
        qs[e] = v < nq && i < 32 && d < hd ? qkv[(size_t)(r0 + vr) * ldqkv + (size_t)(g * kv_mul + v - vr * kv_mul) * hd + d] : 0.0f;
    }
    if (t < NQ) {
        int n = t < nq ? pos[r0 + (t * kmg >> 16)] + 1 - kb * ATT_P : 0;
        np[t] = n < 0 ? 0 : n < ATT_P ? n : ATT_P;
    }
    // (V: 16-byte piece o of the block's rows, position o / (2 hd), into that position's 256-byte LDS row)
    auto vrow = [&](int o) __attribute__((always_inline)) -> int {
        const int pp = (o >> 6) * vmg >> 16;
        return pp * 2 * ATT_HDMAX + (o - pp * 64 * nchk);
    };
#define ATT_ST(k, KR, VR)                                                                                                \
    if ((t + ATT_TH * k) * 16 < nbytes) {                                                                            \
        int o = (t + ATT_TH * k) * 16, tile = ((t >> 6) + 16 * k) * vmg >> 16, w = o - tile * TB;                    \
        *(uint4 *)(ks + tile * ATT_KTILE + (w >> 10) * ATT_KROW + (w & 1023)) = KR;                                   \
        if (VL) *(uint4 *)(vs + vrow(o)) = VR;                                                                        \
    }
    ATT_ST(0, k0, v0) ATT_ST(1, k1, v1) ATT_ST(2, k2, v2) ATT_ST(3, k3, v3)
#undef ATT_ST
    __syncthreads();
    // scores, 8 or 16 vectors (DQ): lane 16 c + n of wave w takes position p = 16 w + n (the wave's tile w) and chunk
    // c; the lane holds q[v][32 c + n] and q[v][32 c + 16 + n] of every vector in registers, and dim i of the chunk's
    // chain takes the row's lane i % 16's (a DPP broadcast inside the fma): no query reads from LDS in the chains.
    // The chunks of position p are rows 0 .. 3 of lane n, added in order. Every lane of a wave whose tile holds a
    // position of the block runs the chains (no lane masked: a DPP source lane must be active); lanes past the block
    // or the head's chunks compute values never written
    if constexpr (DQ) {
        const int n = t & 15, c = (t >> 4) & 3, wv = __builtin_amdgcn_readfirstlane(t >> 6), p = 16 * wv + n;
        float qa[NQ], qb[NQ], acc[NQ];
        #pragma unroll
        for (int v = 0; v < NQ; v++) {
            qa[v] = qs[v * ATT_QS + c * ATT_QC + n];
            qb[v] = qs[v * ATT_QS + c * ATT_QC + 16 + n];
            acc[v] = 0.0f;
        }
        if (16 * wv < nmx) {
            const uint8_t *kt = ks + wv * ATT_KTILE + c * ATT_KROW + (KB ? 4 : 2) * n;
#define ATT_DQ(I, KF)                                                                                                   \
            {                                                                                                           \
                const float kf_ = (KF);                                                                                 \
                const float *qq = (I) < 16 ? qa : qb;                                                                   \
                fmac8_row<(I) & 15>(acc[0], acc[1], acc[2], acc[3], acc[4], acc[5], acc[6], acc[7], qq[0], qq[1], qq[2],  \
                                    qq[3], qq[4], qq[5], qq[6], qq[7], kf_);                                            \
                if constexpr (NQ > 8)                                                                                   \
                    fmac8_row<(I) & 15>(acc[8], acc[9], acc[10], acc[11], acc[12], acc[13], acc[14], acc[15], qq[8],      \
                                        qq[9], qq[10], qq[11], qq[12], qq[13], qq[14], qq[15], kf_);                    \
            }
            if constexpr (KB) { // (dims i, i + 1 of position p: one word at i 32 + 4 p of the chunk row, i even)
#define ATT_DQ2(I)                                                                                                      \
                {                                                                                                       \
                    const uint32_t w_ = *(const uint32_t *)(kt + (I) * 32);                                             \
                    ATT_DQ(I, bf2f(w_ & 0xffffu))                                                                       \
                    ATT_DQ((I) + 1, bf2f(w_ >> 16))                                                                     \
                }
                ATT_DQ2(0) ATT_DQ2(2) ATT_DQ2(4) ATT_DQ2(6) ATT_DQ2(8) ATT_DQ2(10) ATT_DQ2(12) ATT_DQ2(14)
                ATT_DQ2(16) ATT_DQ2(18) ATT_DQ2(20) ATT_DQ2(22) ATT_DQ2(24) ATT_DQ2(26) ATT_DQ2(28) ATT_DQ2(30)
#undef ATT_DQ2
            } else {
#define ATT_DQ1(I) ATT_DQ(I, h2f(*(const uint16_t *)(kt + (I) * 32)))
                ATT_DQ1(0) ATT_DQ1(1) ATT_DQ1(2) ATT_DQ1(3) ATT_DQ1(4) ATT_DQ1(5) ATT_DQ1(6) ATT_DQ1(7)
                ATT_DQ1(8) ATT_DQ1(9) ATT_DQ1(10) ATT_DQ1(11) ATT_DQ1(12) ATT_DQ1(13) ATT_DQ1(14) ATT_DQ1(15)
                ATT_DQ1(16) ATT_DQ1(17) ATT_DQ1(18) ATT_DQ1(19) ATT_DQ1(20) ATT_DQ1(21) ATT_DQ1(22) ATT_DQ1(23)
                ATT_DQ1(24) ATT_DQ1(25) ATT_DQ1(26) ATT_DQ1(27) ATT_DQ1(28) ATT_DQ1(29) ATT_DQ1(30) ATT_DQ1(31)
#undef ATT_DQ1
            }
#undef ATT_DQ
        }
        #pragma unroll
        for (int v = 0; v < NQ; v++) {
            float c1 = __shfl_down(acc[v], 16), c2 = __shfl_down(acc[v], 32), c3 = __shfl_down(acc[v], 48);
            float a = acc[v];
            if (nchk > 1) a = a + c1;
            if (nchk > 2) a = a + c2;
            if (nchk > 3) a = a + c3;
            if (c == 0 && p < nmx && v < nq) S[v][p] = a * scale;
        }
    } else { // scores, up to 4 vectors: lane (position p, chunk c), all NQ vectors (no per-vector branches in the chain)
        int p = t >> 2, c = t & 3;
        const uint8_t *kt = ks + (p / ATT_T) * ATT_KTILE + c * ATT_KROW + (p % ATT_T) * 2;
        const float *qc = qs + c * ATT_QC;
        float acc[NQ];
        #pragma unroll
        for (int v = 0; v < NQ; v++) acc[v] = 0.0f;
        if (p < nmx && c < nchk) {
            for (int i = 0; i < 32; i += 4) {
                float k[4];
                if (KB) { // (dims i, i + 1 of position p in one word at i 32 + 4 p of the chunk row; i + 2, i + 3 below)
                    const uint8_t *kw = kt + (p % ATT_T) * 2;
                    const uint32_t d0 = *(const uint32_t *)(kw + i * 32), d1 = *(const uint32_t *)(kw + (i + 2) * 32);
                    k[0] = bf2f(d0 & 0xffffu), k[1] = bf2f(d0 >> 16), k[2] = bf2f(d1 & 0xffffu), k[3] = bf2f(d1 >> 16);
                } else {
                    #pragma unroll
                    for (int u = 0; u < 4; u++) k[u] = h2f(*(const uint16_t *)(kt + (i + u) * 32));
                }
                float4 q4[NQ];
                #pragma unroll
                for (int v = 0; v < NQ; v++) q4[v] = *(const float4 *)(qc + v * ATT_QS + i);
                #pragma unroll
                for (int v = 0; v < NQ; v++) {
                    acc[v] = __builtin_fmaf(q4[v].x, k[0], acc[v]);
                    acc[v] = __builtin_fmaf(q4[v].y, k[1], acc[v]);
                    acc[v] = __builtin_fmaf(q4[v].z, k[2], acc[v]);
                    acc[v] = __builtin_fmaf(q4[v].w, k[3], acc[v]);
                }
            }
        }
        #pragma unroll
        for (int v = 0; v < NQ; v++) {
            float c1 = quad_lane<1>(acc[v]), c2 = quad_lane<2>(acc[v]), c3 = quad_lane<3>(acc[v]); // (chunks of lane c = 0)
            float a = acc[v];
            if (nchk > 1) a = a + c1;
            if (nchk > 2) a = a + c2;
            if (nchk > 3) a = a + c3;
            if (c == 0 && p < nmx && v < nq) S[v][p] = a * scale;
        }
    }
    __syncthreads();
    if (!VL) { // V into the K buffer (its readers are done), position p's row at p 256 bytes
#define ATT_SV(k, VR)                                                                                                    \
        if ((t + ATT_TH * k) * 16 < nbytes) *(uint4 *)(ks + vrow((t + ATT_TH * k) * 16)) = VR;
        ATT_SV(0, v0) ATT_SV(1, v1) ATT_SV(2, v2) ATT_SV(3, v3)
#undef ATT_SV
    }
    // (the wave and a wave's vector length as uniform values: scalar loop bounds, no exec-masked loops)
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63;
    // (a vector's part of block kb: m, l after its hd values o)
    auto mlp = [&](int v) __attribute__((always_inline)) -> float * {
        return part + ((size_t)(r0 + v / kv_mul) * nh + g * kv_mul + v % kv_mul) * pstride + (size_t)kb * (hd + 2) + hd;
    };
    if (SE) { // softmax: wave w takes vector w & 3 (its max over the block, each of its 4 waves alike), positions
              // 64 (w >> 2) + lane: E = exp_att(s - m); l is added after the barrier, beside the o chains
        const int v = wave & 3, p = 64 * (wave >> 2) + lane;
        if (v < nq && np[v] > 0) {
            const int n = np[v];
            float m = -3.402823466e38f;
            for (int q = lane; q < n; q += 64) m = fmaxf(m, S[v][q]);
            m = wave_max(m);
            if (p < n) E[v][p] = exp_att(S[v][p] - m);
            if (wave < 4 && lane == 0) mlp(v)[0] = m;
        }
    } else if (wave < nq && np[wave] > 0) { // softmax: wave v takes vector v
        int v = wave, n = np[v];
        float m = -3.402823466e38f;
        for (int p = lane; p < n; p += 64) m = fmaxf(m, S[v][p]);
        m = wave_max(m);
        for (int p = lane; p < n; p += 64) S[v][p] = exp_att(S[v][p] - m);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        float s = 0.0f;
        if (lane < 16) {
            int p = lane;
            for (; p + 48 < n; p += 64) {
                float e0 = S[v][p], e1 = S[v][p + 16], e2 = S[v][p + 32], e3 = S[v][p + 48];
                s = s + e0;
                s = s + e1;
                s = s + e2;
                s = s + e3;
            }
            for (; p < n; p += 16) s = s + S[v][p];
        }
        for (int w = 8; w >= 1; w >>= 1) {
            float o = __shfl_down(s, w);
            s = s + o;
        }
        if (lane == 0) {
            float *ml = mlp(v);
            ml[0] = m;
            ml[1] = s;
        }
    }
    __syncthreads();
    if (SE && wave >= 4 && wave < 8 && wave - 4 < nq && np[wave - 4] > 0) { // l of vector wave - 4: 16 lane chains
        const int v = wave - 4, n = np[v];                                  // over p = lane (mod 16), then the tree
        float s = 0.0f;
        if (lane < 16) {
            int p = lane;
            for (; p + 48 < n; p += 64) {
                float e0 = E[v][p], e1 = E[v][p + 16], e2 = E[v][p + 32], e3 = E[v][p + 48];
                s = s + e0;
                s = s + e1;
                s = s + e2;
                s = s + e3;
            }
            for (; p < n; p += 16) s = s + E[v][p];
        }
        for (int w = 8; w >= 1; w >>= 1) {
            float o = __shfl_down(s, w);
            s = s + o;
        }
        if (lane == 0) mlp(v)[1] = s;
    }
    // o: lane (vector v = wave, dim pair d2): the chains over the positions in order, V pairs from LDS, two register
    // sets of PB positions' loads per step
    {
        int v = wave, d2 = lane, i0 = 2 * d2;
        const int n = v < NQ ? __builtin_amdgcn_readfirstlane(np[v < NQ ? v : 0]) : 0;
        if (v < nq && i0 < hd && n > 0) {
            int p = 0;
            float o0 = 0.0f, o1 = 0.0f;
            // (the V rows' byte offset opaque to the compiler: one base register with immediate offsets, not a sum
            // folded into every read past 64 KiB (NQ = 16: V lies above the K tiles))
            int vo = (int)((VL ? vs : ks) - lds) + i0 * 2;
            asm volatile("" : "+v"(vo));
            const uint32_t *vb = (const uint32_t *)(lds + vo);
            constexpr int rs = ATT_HDMAX / 2; // (uint32 words per position's LDS row)
            constexpr int PB = VL ? 16 : 8; // (8: 64 registers, two blocks per CU)
            uint32_t va[PB], vbb[PB];
            float ea[PB], eb[PB];
            auto ld = [&](uint32_t (&vv)[PB], float (&ee)[PB], int q0) {
                #pragma unroll
                for (int u = 0; u < PB; u++) {
                    vv[u] = vb[(q0 + u) * rs];
                    ee[u] = E[v][q0 + u];
                }
            };
            auto fold = [&](const uint32_t (&vv)[PB], const float (&ee)[PB]) {
                #pragma unroll
                for (int u = 0; u < PB; u++) {
                    o0 = __builtin_fmaf(ee[u], KB ? bf2f(vv[u] & 0xffffu) : h2f((uint16_t)(vv[u] & 0xffff)), o0);
                    o1 = __builtin_fmaf(ee[u], KB ? bf2f(vv[u] >> 16) : h2f((uint16_t)(vv[u] >> 16)), o1);
                }
            };
            // (each step loads both sets, then folds them: no register set carried across steps, whose copies had
            // cost a fifth of the loop's instructions; the block's other waves cover the loads' latency)
            for (; p + 2 * PB <= n; p += 2 * PB) {
                ld(va, ea, p);
                ld(vbb, eb, p + PB);
                fold(va, ea);
                fold(vbb, eb);
            }
            if (p + PB <= n) {
                ld(va, ea, p);
                fold(va, ea);
                p += PB;
            }
            for (; p < n; p++) {
                uint32_t vv = vb[p * rs];
                float e = E[v][p];
                o0 = __builtin_fmaf(e, KB ? bf2f(vv & 0xffffu) : h2f((uint16_t)(vv & 0xffff)), o0);
                o1 = __builtin_fmaf(e, KB ? bf2f(vv >> 16) : h2f((uint16_t)(vv >> 16)), o1);
            }
            int row = r0 + v / kv_mul, h = g * kv_mul + v % kv_mul;
            float *o = part + ((size_t)row * nh + h) * pstride + (size_t)kb * (hd + 2);
            // (a V word holds dims i0, i0 + 1; in a bf16 row, dims 32 c + l and 32 c + 16 + l, d2 = 16 c + l)
            const int da = KB ? 32 * (d2 >> 4) + (d2 & 15) : i0, db = KB ? da + 16 : i0 + 1;
            o[da] = o0;
            o[db] = o1;
        }
    }
}

template <int NQ, bool KB>
__global__ __launch_bounds__(ATT_TH, NQ <= 4 ? 8 : 4) void k_attn_part(const int4 *__restrict__ items, const float *__restrict__ qkv, int ldqkv,
                                                      int nh, int nkv, int hd, float scale, const int *__restrict__ pos,
                                                      uint16_t *const *__restrict__ kc, uint16_t *const *__restrict__ vc,
                                                      float *__restrict__ part, int pstride) {
    attn_part_body<NQ, KB>(items, qkv, ldqkv, nh, nkv, hd, scale, pos, kc, vc, part, pstride);
}

// The attention of the one-row (decode) pass, one block of 1024 threads per (query vector v, kv head g, key block kb),
// with the row's QK-norm, RoPE and K / V store fused in (forward.c:1266-1284, :1901-1951). The row's position and its
// sequence's cache bases of the layer (kl, vl) are arguments (no memory round trip before the loads). The block normalizes and
// rotates its query head h = g kv_mul + v; the blocks of the last key block (the one holding the row's position pos)
// also compute the row's key and value of head g, write them into their own LDS copy of the block (so no block waits
// for another's store) and, for v = 0, into the cache. Then the partial result of block kb for vector v exactly as
// k_attn_part computes it: part[h pstride + kb (HD + 2)] = o[HD], m, l.
//   scores: thread (position p, chunk c): the fma chain over the chunk's 32 dims in order; the chunks added in order
//     (neighbouring lanes), times scale; softmax: m = max, e = exp_att(s - m), l = 16 lane chains + the tree (wave 15);
//     o: thread i < HD (a dim), the fma chain over the positions in order, two register sets of 16 positions'
//     loads alternating (a copy between sets would wait for the loads).
// 16 waves: the block's 2 x 32 HD bytes of K / V are loaded in HD / 32 rounds of 16 bytes per thread (a CU's loads in
// flight grow with its waves). Blocks b: XCD x = b % 8, y = b / 8, v = y % kv_mul, item = x + 8 (y / kv_mul) (an
// item's kv_mul blocks share an XCD and its L2); item = kb nkv + g. K / V blocks are loaded whole (the cache holds
// every 256-position block whole).
#define ATD_T 1024
#define ATD_KR 1056                 // LDS bytes of a K chunk row: 32 dims x 16 positions x 2 + 32 padding
#define ATD_KT (4 * ATD_KR + 32)    // LDS bytes of a K tile: the 4 tiles of a wave's 64 positions in distinct banks
template <int HD, bool KB>
__global__ __launch_bounds__(ATD_T) void k_attn_decode(const float *__restrict__ qkv, int nh, int nkv, float scale,
                                                       const float *__restrict__ qn, const float *__restrict__ kn,
                                                       const float *__restrict__ rope, int pos, uint16_t *__restrict__ kl,
                                                       uint16_t *__restrict__ vl, float *__restrict__ part, int pstride) {
    constexpr int NCH = HD / 32, TB = 32 * HD, NR = 256 * HD * 2 / (ATD_T * 16); // chunks, tile bytes, load rounds
    __shared__ __align__(16) uint8_t ks[16 * ATD_KT];
    __shared__ __align__(16) uint8_t vs[256 * HD * 2];
    __shared__ __align__(16) float qs[HD];
    __shared__ float qx[HD], kx[HD], S[256], red[20];
    const int kv_mul = nh / nkv, t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int x = blockIdx.x & 7, y = blockIdx.x >> 3, v = y % kv_mul, item = x + 8 * (y / kv_mul);
    const int nb = pos / ATT_P + 1;
    if (item >= nkv * nb) return;
    const int g = item % nkv, kb = item / nkv, h = g * kv_mul + v, half = HD / 2, pp = pos % ATT_P;
    const bool last = kb == nb - 1;
    const int n = last ? pp + 1 : ATT_P; // positions of this block up to pos
    // 1. the row's q, k and v heads (lane i % HD: no branch around the loads), issued before the cache loads
    const int ti = t % HD;
    const float qr = qkv[(size_t)h * HD + ti], kr = qkv[(size_t)(nh + g) * HD + ti], vr = qkv[(size_t)(nh + nkv + g) * HD + ti];
    // 2. the cache's K and V blocks (whole: NR rounds of 16 bytes per thread)
    const uint8_t *K = (const uint8_t *)(kl + ((size_t)kb * nkv + g) * ATT_P * HD);
    const uint8_t *V = (const uint8_t *)(vl + ((size_t)kb * nkv + g) * ATT_P * HD);
    static_assert(NR >= 1 && NR <= 4, "HD in 32, 64, 128");
    uint4 k0, k1, k2, k3, v0, v1, v2, v3; // (named: an array here is placed in scratch memory)
#define ATD_LD(k, KR, VR)                                                                                               \
    if constexpr (NR > k) {                                                                                         \
        KR = *(const uint4 *)(K + (size_t)(t + ATD_T * k) * 16);                                                     \
        VR = *(const uint4 *)(V + (size_t)(t + ATD_T * k) * 16);                                                     \
    }
    ATD_LD(0, k0, v0) ATD_LD(1, k1, v1) ATD_LD(2, k2, v2) ATD_LD(3, k3, v3)
#undef ATD_LD
    // 3. QK-norm + RoPE (k_qknorm_rope_store's arithmetic): the raw heads into LDS, the scales by waves 0 / 1
    if (t < HD) {
        qx[t] = qr;
        kx[t] = kr;
    }
    __syncthreads();
    if (wave == 0) {
        float r = rms_scale_lds(qx, HD);
        if (lane == 0) red[0] = r;
    } else if (wave == 1 && last) {
        float r = rms_scale_lds(kx, HD);
        if (lane == 0) red[1] = r;
    }
    // 4. the K / V blocks into LDS (K tiles: chunk rows ATD_KR apart, tiles ATD_KT apart; V rows as in the cache)
#define ATD_ST(k, KR, VR)                                                                                               \
    if constexpr (NR > k) {                                                                                         \
        int o = (t + ATD_T * k) * 16, tile = o / TB, w = o % TB;                                                     \
        *(uint4 *)(ks + tile * ATD_KT + (w >> 10) * ATD_KR + (w & 1023)) = KR;                                       \
        *(uint4 *)(vs + o) = VR;                                                                                     \
    }
    ATD_ST(0, k0, v0) ATD_ST(1, k1, v1) ATD_ST(2, k2, v2) ATD_ST(3, k3, v3)
#undef ATD_ST
    __syncthreads();
    const float *cs = rope + (size_t)pos * HD;
    if (t < half) {
        int i = t;
        float r = red[0];
        float xq = (qn[i] * qx[i]) * r, yq = (qn[i + half] * qx[i + half]) * r;
        float c = cs[i], s = cs[i + half];
        float ys = yq * s, yc = yq * c;
        qs[i] = __builtin_fmaf(xq, c, -ys);
        qs[i + half] = __builtin_fmaf(xq, s, yc);
        if (last) { // the row's key: into this block's LDS copy at pp, and (v = 0) into the cache
            float rk = red[1];
            float xk = (kn[i] * kx[i]) * rk, yk = (kn[i + half] * kx[i + half]) * rk;
            float ysk = yk * s, yck = yk * c;
            const float k0v = __builtin_fmaf(xk, c, -ysk), k1v = __builtin_fmaf(xk, s, yck);
            uint16_t kh0 = KB ? f2bf_ref(k0v) : f2h_ref(k0v), kh1 = KB ? f2bf_ref(k1v) : f2h_ref(k1v);
            int tile = pp / ATT_T, col = pp % ATT_T;
            *(uint16_t *)(ks + tile * ATD_KT + (i >> 5) * ATD_KR + kv_k_at(KB, i & 31, col) * 2) = kh0;
            *(uint16_t *)(ks + tile * ATD_KT + ((i + half) >> 5) * ATD_KR + kv_k_at(KB, (i + half) & 31, col) * 2) = kh1;
            if (v == 0) {
                uint16_t *kd = kl + (((size_t)kb * nkv + g) * ATT_P + (size_t)tile * ATT_T) * HD;
                kd[kv_k_at(KB, i, col)] = kh0;
                kd[kv_k_at(KB, i + half, col)] = kh1;
            }
        }
    }
    if (last && t < HD) { // the row's value
        uint16_t vh = KB ? f2bf_ref(vr) : f2h_ref(vr);
        *(uint16_t *)(vs + ((size_t)pp * HD + kv_v_col(KB, t)) * 2) = vh;
        if (v == 0) vl[(((size_t)kb * nkv + g) * ATT_P + pp) * HD + kv_v_col(KB, t)] = vh;
    }
    __syncthreads();
    // 5. scores: thread (p, c)
    const int p = t >> 2, c = t & 3;
    float acc = 0.0f;
    if (p < n && c < NCH) {
        const uint8_t *kt = ks + (p / ATT_T) * ATD_KT + c * ATD_KR + (p % ATT_T) * 2;
        const float *qc = qs + 32 * c;
        float kf[32];
        if (KB) { // (dims 2 q, 2 q + 1 of position p: one word at 2 q 32 + 4 p of the chunk row)
            #pragma unroll
            for (int q = 0; q < 16; q++) {
                const uint32_t w = *(const uint32_t *)(kt + (p % ATT_T) * 2 + q * 64);
                kf[2 * q] = bf2f(w & 0xffffu);
                kf[2 * q + 1] = bf2f(w >> 16);
            }
        } else {
            #pragma unroll
            for (int i = 0; i < 32; i++) kf[i] = h2f(*(const uint16_t *)(kt + i * 32));
        }
        #pragma unroll
        for (int i = 0; i < 32; i += 4) {
            float4 q4 = *(const float4 *)(qc + i);
            acc = __builtin_fmaf(q4.x, kf[i], acc);
            acc = __builtin_fmaf(q4.y, kf[i + 1], acc);
            acc = __builtin_fmaf(q4.z, kf[i + 2], acc);
            acc = __builtin_fmaf(q4.w, kf[i + 3], acc);
        }
    }
    float c1 = quad_lane<1>(acc), c2 = quad_lane<2>(acc), c3 = quad_lane<3>(acc);
    float a = acc;
    if (NCH > 1) a = a + c1;
    if (NCH > 2) a = a + c2;
    if (NCH > 3) a = a + c3;
    const float sc = c == 0 && p < n ? a * scale : -3.402823466e38f;
    // 6. softmax
    float m = wave_max(sc);
    if (lane == 0) red[4 + wave] = m;
    __syncthreads();
    m = red[4];
    #pragma unroll
    for (int w = 1; w < 16; w++) m = fmaxf(m, red[4 + w]);
    if (c == 0 && p < n) S[p] = exp_att(sc - m);
    __syncthreads();
    // 7. l (wave 15, lanes 0..15: chains over p = lane, lane + 16, ... then the tree) beside o (threads i < HD)
    if (wave == 15) {
        float s = 0.0f;
        if (lane < 16) {
            int q = lane;
            for (; q + 48 < n; q += 64) {
                float e0 = S[q], e1 = S[q + 16], e2 = S[q + 32], e3 = S[q + 48];
                s = s + e0;
                s = s + e1;
                s = s + e2;
                s = s + e3;
            }
            for (; q < n; q += 16) s = s + S[q];
        }
        for (int w = 8; w >= 1; w >>= 1) {
            float o = __shfl_down(s, w);
            s = s + o;
        }
        if (lane == 0) {
            float *ml = part + (size_t)h * pstride + (size_t)kb * (HD + 2) + HD;
            ml[0] = m;
            ml[1] = s;
        }
    } else if (t < HD) {
        const uint16_t *vcol = (const uint16_t *)vs + kv_v_col(KB, t);
        float o = 0.0f;
        int q = 0;
        uint16_t va[16], vb[16];
        float ea[16], eb[16];
        auto ld = [&](uint16_t (&vv)[16], float (&ee)[16], int q0) {
            #pragma unroll
            for (int u = 0; u < 16; u++) {
                vv[u] = vcol[(size_t)(q0 + u) * HD];
                ee[u] = S[q0 + u];
            }
        };
        auto fold = [&](const uint16_t (&vv)[16], const float (&ee)[16]) {
            #pragma unroll
            for (int u = 0; u < 16; u++) o = __builtin_fmaf(ee[u], KB ? bf2f(vv[u]) : h2f(vv[u]), o);
        };
        if (n >= 16) {
            ld(va, ea, 0);
            for (q = 16; q + 32 <= n; q += 32) {
                ld(vb, eb, q);
                fold(va, ea);
                ld(va, ea, q + 16);
                fold(vb, eb);
            }
            if (q + 16 <= n) {
                ld(vb, eb, q);
                fold(va, ea);
                fold(vb, eb);
                q += 16;
            } else {
                fold(va, ea);
            }
        }
        for (; q < n; q++) o = __builtin_fmaf(S[q], KB ? bf2f(vcol[(size_t)q * HD]) : h2f(vcol[(size_t)q * HD]), o);
        part[(size_t)h * pstride + (size_t)kb * (HD + 2) + t] = o;
    }
}

// the attention of each head of a row from its key blocks' partials, in block order (att_combine,
// forward.c:1405-1431), then the row's quantization for wo (aq row b, all_heads = nh * HD values, a multiple of 64).
// One wave per (row b, 64 consecutive values of the row: one head, or two of HD = 32); lane: value e, head h = e / HD,
// dim e % HD. Per head: M = max m_k, c_k = exp_att(m_k - M) (lanes over k in parallel, into LDS), L = the fma chain
// of c_k l_k in block order (every lane of the head alike, its LDS reads up to 16 ahead), inv = 1 / L; per value the fma
// chain of c_k o_k in block order, times inv (one block: o inv). The values' o_k load in batches of 32 blocks, the
// next batch in flight while the current one is folded (the partials come from beyond L2: a batch at a time would
// wait one load latency each), the first batch issued before the coefficients; raw buffer loads over the wave's
// heads' partials (past their last block they read 0, never folded), 8 blocks per scalar offset with the rest
// immediate.
// The quantization groups (32 consecutive values) lie inside a head
#define COMB_T 64
template <int HD, int COMB_B> // (COMB_B: blocks per batch, 32, or 8 for passes of short rows: fewer registers)
__global__ __launch_bounds__(COMB_T) void k_attn_combine_quant(const float *__restrict__ part, int pstride, int nh,
                                                            const int *__restrict__ pos, int8_t *__restrict__ aq,
                                                            float *__restrict__ as, int ldq, float *__restrict__ att_out) {
    constexpr int ST = HD + 2, HPW = HD < COMB_T ? COMB_T / HD : 1;
    extern __shared__ float cl[]; // [HPW][nbm] coefficients, then [HPW][nbm] l
    const int b = blockIdx.x, nb = (pos[b] + 1 + ATT_P - 1) / ATT_P, lane = threadIdx.x, nbm = pstride / ST;
    const int e = blockIdx.y * COMB_T + lane, h0 = blockIdx.y * COMB_T / HD, hl = e / HD - h0, ne = nh * HD;
    float *ll = cl + HPW * nbm;
    const float *pr = part + (size_t)b * nh * pstride;
    // (the descriptor spans the wave's heads up to their last block: the batch's loads past it read 0 and touch no
    // memory; with few blocks (prefill rows: 1 or 2) nearly all of a batch is past it)
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc((void *)(pr + (size_t)h0 * pstride), (short)0,
                                                                        ((HPW - 1) * pstride + nb * ST) * 4, GW_RSRC_DW3);
    const int vo = (hl * pstride + e % HD) * 4; // (this value's o in block 0, bytes from the wave's first head)
    float wa[COMB_B], wb[COMB_B];
    auto ld = [&](float (&w)[COMB_B], int k0) __attribute__((always_inline)) {
        #pragma unroll
        for (int u8 = 0; u8 < COMB_B; u8 += 8) {
            const int so = (k0 + u8) * ST * 4;
            #pragma unroll
            for (int u = 0; u < 8; u++)
                w[u8 + u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rp, vo + u * ST * 4, so, 0));
        }
    };
    if (COMB_B > 8 && nb <= 8) { // (short rows in a pass of long ones: the 8 loads they need)
        #pragma unroll
        for (int u = 0; u < 8; u++)
            wa[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rp, vo + u * ST * 4, 0, 0));
    } else {
        ld(wa, 0);
    }
    // coefficients of the wave's heads
    #pragma unroll
    for (int hh = 0; hh < HPW; hh++) {
        const float *ml = pr + (size_t)(h0 + hh) * pstride + HD;
        float *ch = cl + hh * nbm, *lh = ll + hh * nbm;
        float M = -3.402823466e38f;
        for (int k = lane; k < nb; k += COMB_T) {
            const float mk = ml[(size_t)k * ST];
            ch[k] = mk;
            lh[k] = ml[(size_t)k * ST + 1];
            M = fmaxf(M, mk);
        }
        M = wave_max(M);
        if (nb > 1)
            for (int k = lane; k < nb; k += COMB_T) ch[k] = exp_att(ch[k] - M);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    const float *ch = cl + hl * nbm, *lh = ll + hl * nbm;
    float out;
    if (nb == 1) {
        out = wa[0] * (1.0f / lh[0]);
    } else {
        float L = 0.0f;
        {
            constexpr int LB = COMB_B < 16 ? COMB_B : 16; // (the chain's reads LB ahead)
            int k = 0;
            for (; k + LB <= nb; k += LB) {
                float c16[LB], l16[LB];
                #pragma unroll
                for (int u = 0; u < LB; u++) c16[u] = ch[k + u], l16[u] = lh[k + u];
                #pragma unroll
                for (int u = 0; u < LB; u++) L = __builtin_fmaf(c16[u], l16[u], L);
            }
            for (; k < nb; k++) L = __builtin_fmaf(ch[k], lh[k], L);
        }
        const float inv = 1.0f / L;
        float acc = 0.0f;
        auto fold = [&](const float (&w)[COMB_B], int k0, int m) __attribute__((always_inline)) { // (blocks k0 .. k0 + m - 1)
            #pragma unroll
            for (int u = 0; u < COMB_B; u++)
                if (u < m) acc = __builtin_fmaf(ch[k0 + u], w[u], acc);
        };
        int k = 0; // (wa holds blocks k .. k + COMB_B - 1; the loads of whole pairs of batches unconditional)
        for (; k + 2 * COMB_B <= nb; k += 2 * COMB_B) {
            ld(wb, k + COMB_B);
            fold(wa, k, COMB_B);
            ld(wa, k + 2 * COMB_B);
            fold(wb, k + COMB_B, COMB_B);
        }
        if (k + COMB_B < nb) {
            ld(wb, k + COMB_B);
            fold(wa, k, COMB_B);
            fold(wb, k + COMB_B, nb - k - COMB_B);
        } else {
            fold(wa, k, nb - k);
        }
        out = acc * inv;
    }
    if (att_out) att_out[(size_t)b * ne + e] = out;
    quant_lane32(out, aq + (size_t)b * ldq + e, as + (size_t)b * (ldq / 32) + (e >> 5));
}

// ------------------------------------------------------------------------------------ SwiGLU + quantize

// row blockIdx.x of hb = [h (H) | h2 (H)] (il = 0) or blocks of il h then il h2 (il > 0), values 256 blockIdx.y .. + 255:
// v = swiglu_ref(h, h2) (SwiGLU, forward.c:1953-1958), quantized into hq / hs (one lane per value)
__global__ __launch_bounds__(256) void k_swiglu_quant(const float *__restrict__ hb, int H, int il, int8_t *__restrict__ hq,
                                                      float *__restrict__ hs) {
    int b = blockIdx.x, e = blockIdx.y * 256 + threadIdx.x;
    const float *h1 = hb + (size_t)b * 2 * H;
    int i1 = il ? (e / il) * 2 * il + e % il : e, i2 = il ? i1 + il : H + e;
    float v = swiglu_ref(h1[i1], h1[i2]);
    quant_lane32(v, hq + (size_t)b * H + e, hs + (size_t)b * (H / 32) + (e >> 5));
}

// ---------------------------------------------------------------------------------------- quantize rows

__global__ __launch_bounds__(256) void k_quant_rows(const float *__restrict__ x, int n, int ldxf, int8_t *__restrict__ q,
                                                    float *__restrict__ s, int ldq) {
    int b = blockIdx.x, e = blockIdx.y * 256 + threadIdx.x;
    float v = e < n ? x[(size_t)b * ldxf + e] : 0.0f;
    int8_t qq;
    float ss;
    quant_lane32(v, &qq, &ss);
    if (e < n) {
        q[(size_t)b * ldq + e] = qq;
        if ((e & 31) == 0) s[(size_t)b * (ldq / 32) + (e >> 5)] = ss;
    }
}

// ----------------------------------------------------------------------------------------------- argmax

// per row: the first index holding the maximum (sampler.c:40-60), in two steps: ARGMAX_CH chunks of a row, each its
// (max, first index) into scratch, then one wave per row combines them in chunk order
#define ARGMAX_CH 64
__global__ __launch_bounds__(256) void k_argmax_part(const float *__restrict__ lg, int n, int ld, float2 *__restrict__ scr) {
    __shared__ float smax[4];
    __shared__ int sidx[4];
    int row = blockIdx.x, ch = blockIdx.y, len = (n + ARGMAX_CH - 1) / ARGMAX_CH, i0 = ch * len;
    int i1 = i0 + len < n ? i0 + len : n;
    const float *r = lg + (size_t)row * ld;
    float m = -3.402823466e38f;
    int idx = 0x7fffffff;
    for (int i = i0 + threadIdx.x; i < i1; i += 256) {
        float v = r[i];
        if (v > m) { m = v; idx = i; }
    }
    for (int o = 32; o >= 1; o >>= 1) {
        float m2 = __shfl_xor(m, o);
        int i2 = __shfl_xor(idx, o);
        if (m2 > m || (m2 == m && i2 < idx)) { m = m2; idx = i2; }
    }
    int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { smax[w] = m; sidx[w] = idx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < 4; k++)
            if (smax[k] > m || (smax[k] == m && sidx[k] < idx)) { m = smax[k]; idx = sidx[k]; }
        scr[(size_t)row * ARGMAX_CH + ch] = make_float2(m, __int_as_float(idx));
    }
}

__global__ __launch_bounds__(64) void k_argmax_final(const float2 *__restrict__ scr, int *__restrict__ out) {
    int row = blockIdx.x, l = threadIdx.x;
    float2 p = scr[(size_t)row * ARGMAX_CH + l];
    float m = p.x;
    int idx = __float_as_int(p.y);
    for (int o = 32; o >= 1; o >>= 1) {
        float m2 = __shfl_xor(m, o);
        int i2 = __shfl_xor(idx, o);
        if (m2 > m || (m2 == m && i2 < idx)) { m = m2; idx = i2; }
    }
    if (l == 0) out[row] = idx;
}

// Top-k candidates of each row, in sample_topk's order (sampler.c:186-217): the k largest values, the lower index
// first on ties, larger first. Every element gets a 64-bit key, unique within its row, whose order is that order:
//   (ordered bits of the value: -0 as +0, NaN below -inf) << 32 | (2^32 - 1 - index)
// Step 1, per chunk of TOPK_CH of a row: the chunk's k largest keys by radix select (8-bit digits from the top, a
// 256-bin LDS histogram per digit, stopping at the first digit whose bin holds exactly the keys still needed; at most
// 8 digits, usually 2 or 3), sorted by one wave (a bitonic network over its 64 lanes) into scratch: 64 keys per chunk,
// 0 after the chunk's own. Step 2, per row: the 64 largest of the 64 sorted lists by a merge tree (the larger half of
// two sorted lists: lane l's max of a_l and b_(63 - l), a bitonic sequence, sorted by 6 exchange steps); the first k
// are the row's candidates, their values read back from the row. k <= TOPK_KMAX
#define TOPK_CH 64
#define TOPK_KMAX 64

__device__ __forceinline__ uint64_t tk_key(float v, int i) {
    uint32_t b = __float_as_uint(v), key;
    if ((b & 0x7fffffffu) > 0x7f800000u) key = 0u; // NaN: after every number
    else {
        if (b == 0x80000000u) b = 0u;               // -0 ties +0 (sample_topk compares the values)
        key = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    }
    return ((uint64_t)key << 32) | (uint64_t)(~(uint32_t)i);
}

__device__ __forceinline__ uint64_t tk_shfl(uint64_t x, int src) {
    const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)x, src), hi = (uint32_t)__shfl((int)(uint32_t)(x >> 32), src);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t tk_shfl_xor(uint64_t x, int m) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)x, m), hi = (uint32_t)__shfl_xor((int)(uint32_t)(x >> 32), m);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t tk_bitonic_desc(uint64_t x, int l) {
    // a bitonic sequence over the wave's 64 lanes, sorted descending (lane 0 the largest)
    #pragma unroll
    for (int st = 32; st > 0; st >>= 1) {
        const uint64_t y = tk_shfl_xor(x, st);
        x = ((l & st) == 0) == (x > y) ? x : y;
    }
    return x;
}

__device__ __forceinline__ uint64_t tk_sort_desc(uint64_t x, int l) {
    // any 64 keys over the wave's lanes, sorted descending
    #pragma unroll
    for (int size = 2; size <= 64; size <<= 1)
        #pragma unroll
        for (int st = size >> 1; st > 0; st >>= 1) {
            const uint64_t y = tk_shfl_xor(x, st);
            const bool keep_max = ((l & size) == 0) == ((l & st) == 0);
            x = keep_max == (x > y) ? x : y;
        }
    return x;
}

__device__ __forceinline__ uint64_t tk_max(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t tk_merge(uint64_t a, uint64_t b, int l) {
    // the 64 largest of two descending lists (lane l: a_l, b_l), descending
    return tk_bitonic_desc(tk_max(a, tk_shfl(b, 63 - l)), l);
}

template <int L>
__device__ __forceinline__ void tk_radix(const uint64_t (&c)[L], int need, uint64_t &P, int &shift, int (*hist)[256], int *sh) {
    // the block's `need` largest keys (0: no element; at least `need` others, 256 threads): on return every thread
    // holds P and shift such that exactly the `need` keys c != 0 with (c >> shift) >= P are those. Two histograms in
    // turn: a digit's counts go into one while the next one is cleared
    const int t = threadIdx.x, l = t & 63;
    uint64_t pre = 0;
    int p = 0;
    hist[0][t] = 0;
    __syncthreads();
    for (int sft = 56;; sft -= 8, p ^= 1) {
        #pragma unroll
        for (int u = 0; u < L; u++)
            if (c[u] && (sft == 56 || (c[u] >> (sft + 8)) == pre)) atomicAdd(&hist[p][(int)(c[u] >> sft) & 255], 1);
        hist[p ^ 1][t] = 0;
        __syncthreads();
        if (t < 64) { // lane l: bins 255 - 4 l down to 252 - 4 l; the bin where the count from the top reaches need
            const int *hp = hist[p];
            const int b0 = 255 - 4 * l, h0 = hp[b0], h1 = hp[b0 - 1], h2 = hp[b0 - 2], h3 = hp[b0 - 3];
            const int own = h0 + h1 + h2 + h3;
            int inc = own;
            #pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int y = __shfl_up(inc, o);
                if (l >= o) inc += y;
            }
            const int ex = inc - own;
            if (ex < need && need <= inc) {
                int cum = ex, d = b0, h = h0;
                if (cum + h0 < need) {
                    cum += h0, d = b0 - 1, h = h1;
                    if (cum + h1 < need) {
                        cum += h1, d = b0 - 2, h = h2;
                        if (cum + h2 < need) cum += h2, d = b0 - 3, h = h3;
                    }
                }
                sh[0] = d, sh[1] = need - cum, sh[2] = h;
            }
        }
        __syncthreads();
        const int d = sh[0], h = sh[2];
        need = sh[1];
        pre = (pre << 8) | (uint64_t)d;
        if (h == need || sft == 0) {
            P = pre, shift = sft;
            return;
        }
    }
}

__global__ __launch_bounds__(256) void k_topk_part(const float *__restrict__ lg, int n, int ld, int k, uint64_t *__restrict__ scr) {
    // block (row, chunk): step 1 on the chunk (chunks of ceil(n / TOPK_CH) <= 16 x 256 values): its min(k, its length)
    // largest keys, sorted, then 0 up to 64
    __shared__ int hist[2][256], sh[4];
    __shared__ uint64_t best[TOPK_KMAX];
    const int row = blockIdx.x, ch = blockIdx.y, len = (n + TOPK_CH - 1) / TOPK_CH, i0 = ch * len, t = threadIdx.x;
    const int nv = n - i0 < len ? n - i0 : len, kc = nv < k ? (nv > 0 ? nv : 0) : k;
    const float *r = lg + (size_t)row * ld;
    uint64_t c[16];
    #pragma unroll
    for (int u = 0; u < 16; u++) {
        const int i = i0 + t + 256 * u;
        c[u] = t + 256 * u < nv ? tk_key(r[i], i) : 0;
    }
    if (kc > 0) {
        uint64_t P;
        int shift;
        tk_radix<16>(c, kc, P, shift, hist, sh);
        if (t == 0) sh[3] = 0;
        __syncthreads();
        #pragma unroll
        for (int u = 0; u < 16; u++)
            if (c[u] && (c[u] >> shift) >= P) {
                const int slot = atomicAdd(&sh[3], 1); // (< kc: exactly kc keys pass)
                if (slot < kc) best[slot] = c[u];
            }
        __syncthreads();
    }
    if (t < 64) scr[((size_t)row * TOPK_CH + ch) * TOPK_KMAX + t] = tk_sort_desc(t < kc ? best[t] : 0, t);
}

__global__ __launch_bounds__(256) void k_topk_final(const float *__restrict__ lg, int ld, const uint64_t *__restrict__ scr, int k,
                                                    float *__restrict__ vals, int *__restrict__ idx) {
    // block row: step 2 on the row's TOPK_CH sorted lists: wave w merges lists 16 w .. 16 w + 15 (four levels in
    // registers), then the four waves' lists meet in LDS (two levels); the first k into vals / idx, the values read back
    // from the row (their bits, -0 included)
    __shared__ uint64_t lv[4][64], lv2[2][64];
    const int row = blockIdx.x, t = threadIdx.x, l = t & 63, w = t >> 6;
    const uint64_t *cc = scr + ((size_t)row * TOPK_CH + 16 * w) * TOPK_KMAX;
    uint64_t m[8];
    #pragma unroll
    for (int q = 0; q < 8; q++) // (level 1: lists 16 w + 2 q and 16 w + 2 q + 1, the second read reversed)
        m[q] = tk_bitonic_desc(tk_max(cc[(2 * q) * TOPK_KMAX + l], cc[(2 * q + 1) * TOPK_KMAX + 63 - l]), l);
    #pragma unroll
    for (int q = 0; q < 4; q++) m[q] = tk_merge(m[2 * q], m[2 * q + 1], l);
    #pragma unroll
    for (int q = 0; q < 2; q++) m[q] = tk_merge(m[2 * q], m[2 * q + 1], l);
    lv[w][l] = tk_merge(m[0], m[1], l);
    __syncthreads();
    if (w < 2) lv2[w][l] = tk_bitonic_desc(tk_max(lv[2 * w][l], lv[2 * w + 1][63 - l]), l);
    __syncthreads();
    if (w == 0) {
        const uint64_t x = tk_bitonic_desc(tk_max(lv2[0][l], lv2[1][63 - l]), l);
        if (l < k && x) {
            const int i = (int)~(uint32_t)x;
            vals[(size_t)row * k + l] = lg[(size_t)row * ld + i];
            idx[(size_t)row * k + l] = i;
        }
    }
}

// The no-allocation top-k's scratch (gw_ctx_topk_noalloc): one array per device for the process's lifetime, holding the
// chunk lists of GW_TOPK_NA_ROWS rows (TOPK_CH x TOPK_KMAX keys each) and then the outputs (rows x TOPK_KMAX values, rows
// x TOPK_KMAX indices). Every call on a device uses the same array and leaves its contents there; nothing in it needs
// to start at zero (each call writes every key and output it reads). Calls that overlap on one device race
#define GW_NA_CAND_BYTES ((size_t)GW_TOPK_NA_ROWS * TOPK_CH * TOPK_KMAX * 8)
#define GW_NA_BYTES (GW_NA_CAND_BYTES + (size_t)GW_TOPK_NA_ROWS * TOPK_KMAX * 8)
static __device__ __align__(256) unsigned char scratch[GW_NA_BYTES];

// ------------------------------------------------------------------------------------------ launchers

#include <pthread.h>

extern "C" {

/* the device address of this device's scratch array (the array's name in host code is a host-side stand-in, not a
 * device address): taken once per device with that device current, then kept */
#define GW_NA_MAXDEV 64
static void *na_ptr[GW_NA_MAXDEV];
static pthread_mutex_t na_mu = PTHREAD_MUTEX_INITIALIZER;

int gw_k_topk_noalloc(const float *lg, int n, int ld, int rows, int k, float **vals, int **idx, hipStream_t s) {
    /* gw_k_topk with this device's scratch array as its candidates and outputs (*vals, *idx: where the outputs are,
     * rows x k each, device memory); rows <= GW_TOPK_NA_ROWS. Allocates nothing */
    if (rows < 1 || rows > GW_TOPK_NA_ROWS || !vals || !idx) return (int)hipErrorInvalidValue;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (dev < 0 || dev >= GW_NA_MAXDEV) return (int)hipErrorInvalidDevice;
    pthread_mutex_lock(&na_mu);
    if (!na_ptr[dev]) {
        void *p = NULL;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e == hipSuccess && p) na_ptr[dev] = p;
        else if (e == hipSuccess) e = hipErrorInvalidSymbol;
    }
    unsigned char *base = (unsigned char *)na_ptr[dev];
    pthread_mutex_unlock(&na_mu);
    if (e != hipSuccess) return (int)e;
    *vals = (float *)(base + GW_NA_CAND_BYTES);
    *idx = (int *)(base + GW_NA_CAND_BYTES + (size_t)GW_TOPK_NA_ROWS * TOPK_KMAX * 4);
    return gw_k_topk(lg, n, ld, rows, k, *vals, *idx, base, s);
}

int gw_k_embed_q8(float *x, int dim, const uint8_t *codes, const uint16_t *scales, const int *tok, int n, hipStream_t s) {
    GW_LAUNCH(k_embed_q8, dim3(n, (dim + 255) / 256), dim3(256), 0, s, x, dim, codes, scales, tok);
    return (int)hipGetLastError();
}

int gw_k_rmsnorm_quant(float *x, const float *d, int dim, const float *w, const int *sel, int n, int8_t *xq, float *xs, int ldq,
                       float *hid, hipStream_t s) {
    if (dim % 64 == 0)
        GW_LAUNCH(k_rmsnorm_quant<true>, dim3(n), dim3(NORM_T), (size_t)16 * (4 * rms_nf(dim / 64) + 4) * sizeof(float), s, x, d, dim,
                  w, sel, xq, xs, ldq, hid);
    else
        GW_LAUNCH(k_rmsnorm_quant<false>, dim3(n), dim3(NORM_T), (size_t)dim * sizeof(float), s, x, d, dim, w, sel, xq, xs, ldq, hid);
    return (int)hipGetLastError();
}

int gw_k_set_exact(const float *rsq, int bits, const uint64_t *rcp, const uint8_t *expd) {
    /* this file's copy of the host-measured tables (rsqrt_ref, swiglu_ref) on the current device */
    hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(gw_rsqrt_bits), &bits, sizeof(int));
    if (e == hipSuccess && bits) e = hipMemcpyToSymbol(HIP_SYMBOL(gw_rsqrt_tab), rsq, sizeof(float) << bits);
    if (e == hipSuccess) e = hipMemcpyToSymbol(HIP_SYMBOL(gw_rcp_blk), &rcp, sizeof(rcp));
    if (e == hipSuccess) e = hipMemcpyToSymbol(HIP_SYMBOL(gw_exp_delta), &expd, sizeof(expd));
    return (int)e;
}

int gw_k_qknorm_rope_store(float *qkv, int ldqkv, int n, int nh, int nkv, int hd, const float *qn, const float *kn,
                           const float *rope, const int *pos, uint16_t *const *kc, uint16_t *const *vc, const int *kvt,
                           hipStream_t s) {
    GW_LAUNCH(k_qknorm_rope_store, dim3(n, nh + 2 * nkv), dim3(64), 0, s, qkv, ldqkv, nh, nkv, hd, qn, kn, rope, pos, kc, vc, kvt);
    return (int)hipGetLastError();
}

int gw_k_attn_q(const void *items, int nitems, const float *qkv, int ldqkv, int nh, int nkv, int hd, float scale, const int *pos,
                uint16_t *const *kc, uint16_t *const *vc, const int *kvt, int dot, int nqm, float *part, int pstride,
                hipStream_t s) {
    // (hd a power of two, 32 .. 128; at most nqm query vectors per item: 8 or 16)
    if (hd < 32 || hd > 128 || (hd & (hd - 1)) || (nqm != 8 && nqm != 16)) return (int)hipErrorInvalidValue;
    if (dot && nqm == 8)
        GW_LAUNCH((k_attn_q<true, 8>), dim3(nitems), dim3(AQ_T), 0, s, (const int4 *)items, qkv, ldqkv, nh, nkv, hd, scale, pos,
                  kc, vc, kvt, part, pstride);
    else if (dot)
        GW_LAUNCH((k_attn_q<true, 16>), dim3(nitems), dim3(AQ_T), 0, s, (const int4 *)items, qkv, ldqkv, nh, nkv, hd, scale, pos,
                  kc, vc, kvt, part, pstride);
    else if (nqm == 8)
        GW_LAUNCH((k_attn_q<false, 8>), dim3(nitems), dim3(AQ_T), 0, s, (const int4 *)items, qkv, ldqkv, nh, nkv, hd, scale, pos,
                  kc, vc, kvt, part, pstride);
    else
        GW_LAUNCH((k_attn_q<false, 16>), dim3(nitems), dim3(AQ_T), 0, s, (const int4 *)items, qkv, ldqkv, nh, nkv, hd, scale,
                  pos, kc, vc, kvt, part, pstride);
    return (int)hipGetLastError();
}

int gw_k_fill_synthetic_q(void *kc, void *vc, int kvt, int npos, int nkv, int hd, unsigned long long seed, hipStream_t s) {
    if (hd > 256 || npos < 1) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_fill_synthetic_q, dim3(npos, nkv, 2), dim3(64), 0, s, kc, vc, kvt, nkv, hd, seed);
    return (int)hipGetLastError();
}

int gw_k_unrot_quant(const float *att, int n, int nh, int hd, const int *kvt, int8_t *aq, float *as, int ldq, hipStream_t s) {
    if (hd > 256 || (hd != 32 && hd % 64)) return (int)hipErrorInvalidValue;
    GW_LAUNCH(k_unrot_quant, dim3(n, nh), dim3(64), 0, s, att, nh, hd, kvt, aq, as, ldq);
    return (int)hipGetLastError();
}

int gw_k_attn_part(const void *items, int nitems, int nq_max, const float *qkv, int ldqkv, int nh, int nkv, int hd, float scale,
                   const int *pos, uint16_t *const *kc, uint16_t *const *vc, float *part, int pstride, int kbf, hipStream_t s) {
    int nq = nq_max;
    const int4 *it = (const int4 *)items;
#define ATT_LAUNCH(Q)                                                                                                   \
    do {                                                                                                                \
        if (kbf) GW_LAUNCH((k_attn_part<Q, true>), dim3(nitems), dim3(ATT_TH), 0, s, it, qkv, ldqkv, nh, nkv, hd, scale, pos, kc, vc, part, pstride); \
        else GW_LAUNCH((k_attn_part<Q, false>), dim3(nitems), dim3(ATT_TH), 0, s, it, qkv, ldqkv, nh, nkv, hd, scale, pos, kc, vc, part, pstride); \
    } while (0)
    if (nq <= 1) ATT_LAUNCH(1);
    else if (nq <= 2) ATT_LAUNCH(2);
    else if (nq <= 4) ATT_LAUNCH(4);
    else if (nq <= 8) ATT_LAUNCH(8);
    else ATT_LAUNCH(16);
#undef ATT_LAUNCH
    return (int)hipGetLastError();
}

int gw_k_attn_decode(const float *qkv, int nh, int nkv, int hd, float scale, const float *qn, const float *kn, const float *rope,
                     int pos, uint16_t *kl, uint16_t *vl, float *part, int pstride, int kbf, hipStream_t s) {
    int kvm = nh / nkv, nitems = nkv * (pos / ATT_P + 1);
    dim3 grid(8 * kvm * ((nitems + 7) / 8));
#define ATD_L(H, B) GW_LAUNCH((k_attn_decode<H, B>), grid, dim3(ATD_T), 0, s, qkv, nh, nkv, scale, qn, kn, rope, pos, kl, vl, part, pstride)
    if (hd == 128) { if (kbf) ATD_L(128, true); else ATD_L(128, false); }
    else if (hd == 64) { if (kbf) ATD_L(64, true); else ATD_L(64, false); }
    else if (hd == 32) { if (kbf) ATD_L(32, true); else ATD_L(32, false); }
    else return (int)hipErrorInvalidValue;
#undef ATD_L
    return (int)hipGetLastError();
}

int gw_k_attn_combine_quant(const float *part, int pstride, int nh, int hd, const int *pos, int n, int nbmax, int8_t *aq,
                            float *as, int ldq, float *att_out, hipStream_t s) {
    // (nh hd % 64 == 0, hd in 32, 64, 128); LDS: the coefficients and l of the wave's heads, up to pstride / (hd + 2)
    // blocks
    if ((nh * hd) % COMB_T || (hd != 32 && hd != 64 && hd != 128)) return (int)hipErrorInvalidValue;
    const size_t sh = (size_t)(hd < COMB_T ? COMB_T / hd : 1) * 2 * (pstride / (hd + 2)) * sizeof(float);
    const dim3 grid(n, nh * hd / COMB_T);
#define COMB_L(H, B) GW_LAUNCH((k_attn_combine_quant<H, B>), grid, dim3(COMB_T), sh, s, part, pstride, nh, pos, aq, as, ldq, att_out)
    if (nbmax <= 8) { // (prefill passes: rows of 1 or 2 blocks)
        if (hd == 128) COMB_L(128, 8);
        else if (hd == 64) COMB_L(64, 8);
        else COMB_L(32, 8);
    } else {
        if (hd == 128) COMB_L(128, 32);
        else if (hd == 64) COMB_L(64, 32);
        else COMB_L(32, 32);
    }
#undef COMB_L
    return (int)hipGetLastError();
}

int gw_k_swiglu_quant(const float *hb, int H, int il, int n, int8_t *hq, float *hs, hipStream_t s) {
    GW_LAUNCH(k_swiglu_quant, dim3(n, H / 256), dim3(256), 0, s, hb, H, il, hq, hs);
    return (int)hipGetLastError();
}

int gw_k_quant_rows(const float *x, int n, int ldxf, int rows, int8_t *q, float *sc, int ldq, hipStream_t s) {
    GW_LAUNCH(k_quant_rows, dim3(rows, (n + 255) / 256), dim3(256), 0, s, x, n, ldxf, q, sc, ldq);
    return (int)hipGetLastError();
}

int gw_k_topk(const float *lg, int n, int ld, int rows, int k, float *vals, int *idx, void *scratch, hipStream_t s) {
    /* scratch: rows x TOPK_CH x TOPK_KMAX keys; n <= TOPK_CH x 16 x 256, k <= TOPK_KMAX and < n */
    if (k < 1 || k > TOPK_KMAX || k >= n || n > TOPK_CH * 16 * 256 || ld < n || rows < 1 || !lg || !vals || !idx || !scratch)
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_topk_part, dim3(rows, TOPK_CH), dim3(256), 0, s, lg, n, ld, k, (uint64_t *)scratch);
    hipLaunchKernelGGL(k_topk_final, dim3(rows), dim3(256), 0, s, lg, ld, (const uint64_t *)scratch, k, vals, idx);
    return (int)hipGetLastError();
}

int gw_topk_rows(const float *logits, int n, int ld, int rows, int k, float *vals, int *idx, void *scratch, void *stream) {
    if (k < 1 || k > TOPK_KMAX || k >= n || n > TOPK_CH * 16 * 256 || ld < n || rows < 1 || !logits || !vals || !idx || !scratch)
        return RQ_ERR_ARG;
    return gw_k_topk(logits, n, ld, rows, k, vals, idx, scratch, (hipStream_t)stream) ? RQ_ERR_STATE : RQ_OK;
}

int gw_k_argmax(const float *lg, int n, int ld, int rows, int *out, void *scratch, hipStream_t s) {
    hipEvent_t e0, e1; // (timing: the first kernel's start, the second one's stop)
    gw_take_launch_events(&e0, &e1);
    hipExtLaunchKernelGGL(k_argmax_part, dim3(rows, ARGMAX_CH), dim3(256), 0, s, e0, (hipEvent_t)NULL, 0, lg, n, ld, (float2 *)scratch);
    hipExtLaunchKernelGGL(k_argmax_final, dim3(rows), dim3(64), 0, s, (hipEvent_t)NULL, e1, 0, (const float2 *)scratch, out);
    return (int)hipGetLastError();
}

} // extern "C"
