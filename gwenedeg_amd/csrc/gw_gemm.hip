// The matmul dispatch of the forward passes (gw_k_matmul), the load-time repack, and the isolated Q8_0 / K-quant
// operator of the public ABI (gw_q8_*, gw_kq_matmul, gw_quantize).
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "gw_internal.h"

__device__ __forceinline__ float h2f_g(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// GGUF Q8_0 blocks (fp16 d, 32 int8; 34 bytes) -> codes (32 per block) + fp16 scales: the device layout
__global__ __launch_bounds__(256) void k_q8_unpack(const uint8_t *__restrict__ blk, size_t nblk, int8_t *__restrict__ codes,
                                                   uint16_t *__restrict__ scales, int gpr, int il, int off) {
    // block b of source row i = b / gpr goes to row i (il = 0) or, interleaved, to row (i / il) 2 il + off + i % il
    size_t b = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (b >= nblk) return;
    size_t db = b;
    if (il) {
        size_t i = b / gpr;
        db = ((i / il) * 2 * il + off + i % il) * gpr + b % gpr;
    }
    const uint8_t *p = blk + b * 34;
    scales[db] = (uint16_t)(p[0] | p[1] << 8);
    uint32_t w[8];
    #pragma unroll
    for (int i = 0; i < 8; i++)
        w[i] = (uint32_t)p[2 + 4 * i] | (uint32_t)p[3 + 4 * i] << 8 | (uint32_t)p[4 + 4 * i] << 16 | (uint32_t)p[5 + 4 * i] << 24;
    uint4 *d = (uint4 *)(codes + db * 32);
    d[0] = make_uint4(w[0], w[1], w[2], w[3]);
    d[1] = make_uint4(w[4], w[5], w[6], w[7]);
}

// exact int32 group sums, one thread per (m, n, g)
__global__ __launch_bounds__(256) void k_q8_block_sums(int32_t *__restrict__ isum, const int8_t *__restrict__ W, int N, int K,
                                                       const int8_t *__restrict__ X, int M) {
    size_t G = K / 32, i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)M * N * G) return;
    size_t g = i % G, n = i / G % N, m = i / G / N;
    const int *w = (const int *)(W + n * K + g * 32), *x = (const int *)(X + m * K + g * 32);
    int s = 0;
    #pragma unroll
    for (int k = 0; k < 8; k++) s = __builtin_amdgcn_sdot4(w[k], x[k], s, false);
    isum[i] = s;
}

// pseudo-random f16 K (|K| < 4) and V (|V| < 1) values, for timing runs (rq_seq_fill_synthetic)
__global__ __launch_bounds__(256) void k_fill_synthetic(uint16_t *kc, uint16_t *vc, size_t n, unsigned long long seed) {
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    unsigned long long z = seed + i * 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    z ^= z >> 31;
    float a = (float)(z & 0xffffff) * (1.0f / 16777216.0f), b = (float)((z >> 24) & 0xffffff) * (1.0f / 16777216.0f);
    kc[i] = __half_as_ushort(__float2half((2.0f * a - 1.0f) * 3.9f));
    vc[i] = __half_as_ushort(__float2half((2.0f * b - 1.0f) * 0.99f));
}

// ------------------------------------------------------------------------------------- Q8_0 MFMA GEMM

// out[m * ldo + n] = W row n . X row m for m < M, n < N (prefill / batched rows): per group g of 32 (one K step of
// v_mfma_i32_32x32x32_i8), the exact int32 sums of a 32 x 32 output tile, then per output the reference's fold
// val = val + (ws * xs) * (float) isum, groups in order (forward.c:906-916). A block of 256 threads (4 waves) computes a
// GM x GN tile, GN = 128: GM = 64, wave w takes rows 32 (w / 2) .., columns 64 (w % 2) .. (two MFMA tiles); GM = 32 (for
// matrices whose 64-row tiles leave CUs with one wave per SIMD), wave w takes columns 32 w .. (one MFMA tile). X and W
// are staged in LDS 4 groups (128 bytes of each row) at a time with 16-byte loads, rows padded to 144 bytes.
// MFMA operand layout (32 x 32 x 32, int8): lane l holds A[l % 32][16 (l / 32) .. + 15] and B[16 (l / 32) .. + 15][l % 32];
// result register r of lane l is C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32]
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
#define GN 128
#define GKB 128
#define GROW 144
template <int GM>
__global__ __launch_bounds__(256) void k_gemm_q8(const int8_t *__restrict__ W, const uint16_t *__restrict__ WS, int N, int K,
                                                 const int8_t *__restrict__ X, const float *__restrict__ XS, int ldx, int M,
                                                 float *__restrict__ out, int ldo) {
    constexpr int TJ = GM == 64 ? 2 : 1, XC = GM * 8 / 256; // MFMA tiles per wave, X chunks of 16 B per thread
    __shared__ __align__(16) int8_t xl[GM * GROW];
    __shared__ __align__(16) int8_t wl[GN * GROW];
    __shared__ __align__(16) float xsl[4][GM];
    __shared__ float wsl[GN][4];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int m0 = blockIdx.y * GM, n0 = blockIdx.x * GN, G = K >> 5;
    const int wm = GM == 64 ? (wave >> 1) * 32 : 0, wn = GM == 64 ? (wave & 1) * 64 : wave * 32; // the wave's sub-tile
    float acc[TJ][16];
    #pragma unroll
    for (int j = 0; j < TJ; j++)
        #pragma unroll
        for (int r = 0; r < 16; r++) acc[j][r] = 0.0f;
    for (int k0 = 0; k0 < K; k0 += GKB) {
        const int ng = (K - k0) < GKB ? (K - k0) >> 5 : 4; // groups in this stage
        // stage: X rows m0.. (GM x 128 B: XC chunks of 16 B per thread), W rows n0.. (GN x 128 B: 4 per thread)
        uint4 xr[XC], wr[4];
        #pragma unroll
        for (int k = 0; k < XC; k++) {
            int c = t + 256 * k, row = c >> 3, col = (c & 7) * 16, m = m0 + row < M ? m0 + row : M - 1;
            xr[k] = col < ng * 32 ? *(const uint4 *)(X + (size_t)m * ldx + k0 + col) : make_uint4(0, 0, 0, 0);
        }
        #pragma unroll
        for (int k = 0; k < 4; k++) {
            int c = t + 256 * k, row = c >> 3, col = (c & 7) * 16, n = n0 + row < N ? n0 + row : N - 1;
            wr[k] = col < ng * 32 ? *(const uint4 *)(W + (size_t)n * K + k0 + col) : make_uint4(0, 0, 0, 0);
        }
        float xsv = 0.0f, wsv0 = 0.0f, wsv1 = 0.0f;
        {
            int row = t >> 2, gg = t & 3, m = m0 + row < M ? m0 + row : M - 1;
            if (row < GM && gg < ng) xsv = XS[(size_t)m * (ldx >> 5) + (k0 >> 5) + gg];
            int n = n0 + row < N ? n0 + row : N - 1, n2 = n0 + row + 64 < N ? n0 + row + 64 : N - 1;
            if (gg < ng) {
                wsv0 = h2f_g(WS[(size_t)n * G + (k0 >> 5) + gg]);
                wsv1 = h2f_g(WS[(size_t)n2 * G + (k0 >> 5) + gg]);
            }
        }
        __syncthreads(); // (the previous stage's readers are done)
        #pragma unroll
        for (int k = 0; k < XC; k++) {
            int c = t + 256 * k;
            *(uint4 *)(xl + (c >> 3) * GROW + (c & 7) * 16) = xr[k];
        }
        #pragma unroll
        for (int k = 0; k < 4; k++) {
            int c = t + 256 * k;
            *(uint4 *)(wl + (c >> 3) * GROW + (c & 7) * 16) = wr[k];
        }
        {
            int row = t >> 2, gg = t & 3;
            if (row < GM) xsl[gg][row] = xsv;
            wsl[row][gg] = wsv0;
            wsl[row + 64][gg] = wsv1;
        }
        __syncthreads();
        for (int gg = 0; gg < ng; gg++) {
            i32x4 a = *(const i32x4 *)(xl + (wm + (lane & 31)) * GROW + gg * 32 + 16 * (lane >> 5));
            #pragma unroll
            for (int j = 0; j < TJ; j++) {
                i32x4 b = *(const i32x4 *)(wl + (wn + 32 * j + (lane & 31)) * GROW + gg * 32 + 16 * (lane >> 5));
                i32x16 z = { 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0 };
                i32x16 I = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, z, 0, 0, 0);
                float ws = wsl[wn + 32 * j + (lane & 31)][gg];
                #pragma unroll
                for (int q = 0; q < 4; q++) {
                    float4 xs4 = *(const float4 *)(&xsl[gg][wm + 8 * q + 4 * (lane >> 5)]);
                    float xsq[4] = { xs4.x, xs4.y, xs4.z, xs4.w };
                    #pragma unroll
                    for (int s = 0; s < 4; s++) {
                        float sc = ws * xsq[s];
                        float p = sc * (float)I[4 * q + s];
                        acc[j][4 * q + s] = acc[j][4 * q + s] + p;
                    }
                }
            }
        }
    }
    #pragma unroll
    for (int j = 0; j < TJ; j++) {
        int n = n0 + wn + 32 * j + (lane & 31);
        #pragma unroll
        for (int r = 0; r < 16; r++) {
            int m = m0 + wm + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (m < M && n < N) out[(size_t)m * ldo + n] = acc[j][r];
        }
    }
}

// --------------------------------------------------------------------------------------------- K-quants

// the per-group term of the K-quant fold (kquants.h:86-109) for weight row `row` (its blocks at rb) and group g:
//   Q4_K: a - b, a = (ds * xs) * (float) isum, b = dm * xf, ds = d * sc_j, dm = dmin * m_j (sub-block j = g % 8)
//   Q6_K: (d * xs) * (float) I, I = sc_j0 * t_j0 + sc_j1 * t_j1, t_j = sum q * xq - 32 * sum xq over 16 values
template <int TYPE>
__device__ __forceinline__ float kq_term(const uint8_t *__restrict__ rb, int g, const int8_t *__restrict__ x, float xsg, float xfg) {
    int s = g >> 3, j = g & 7;
    if (TYPE == GW_Q4_K) {
        const uint8_t *b = rb + (size_t)s * 144;
        const uint8_t *sc = b + 4;
        int scj, mj;
        if (j < 4) {
            scj = sc[j] & 63;
            mj = sc[j + 4] & 63;
        } else {
            scj = (sc[j + 4] & 15) | (sc[j - 4] >> 6) << 4;
            mj = (sc[j + 4] >> 4) | (sc[j] >> 6) << 4;
        }
        const uint8_t *qs = b + 16 + 32 * (j >> 1);
        int sh = 4 * (j & 1), isum = 0;
        #pragma unroll
        for (int l = 0; l < 32; l++) isum += ((qs[l] >> sh) & 15) * (int)x[l];
        float d = __half2float(__ushort_as_half((uint16_t)(b[0] | b[1] << 8)));
        float dmin = __half2float(__ushort_as_half((uint16_t)(b[2] | b[3] << 8)));
        float ds = d * (float)scj, dm = dmin * (float)mj;
        float a = (ds * xsg) * (float)isum;
        float bb = dm * xfg;
        return a - bb;
    } else {
        const uint8_t *b = rb + (size_t)s * 210;
        int n = j >> 2, p = j & 3, I = 0;
        #pragma unroll
        for (int h = 0; h < 2; h++) {
            int t = 0, xsum = 0;
            #pragma unroll
            for (int l0 = 0; l0 < 16; l0++) {
                int l = 16 * h + l0;
                int lo = (b[64 * n + 32 * (p & 1) + l] >> (4 * (p >> 1))) & 15;
                int hi = (b[128 + 32 * n + l] >> (2 * p)) & 3;
                t += (lo | hi << 4) * (int)x[l];
                xsum += x[l];
            }
            I += (int)(int8_t)b[192 + 2 * j + h] * (t - 32 * xsum);
        }
        float d = __half2float(__ushort_as_half((uint16_t)(b[208] | b[209] << 8)));
        return (d * xsg) * (float)I;
    }
}

// out[m * ldo + row] = W row . X row m for the K-quant blocks (row-major: K / 256 blocks per row), R rows per block:
// each thread takes groups g = t, t + 256, ... of every row, its term into LDS; one lane per (m, row) folds in order
template <int TYPE, int M, int R>
__global__ __launch_bounds__(256) void k_gemv_kq(const uint8_t *__restrict__ W, int nrows, int K, const int8_t *__restrict__ xq,
                                                 const float *__restrict__ xs, int ldx, float *out, int ldo, int mode) {
    extern __shared__ float P[];
    const int G = K >> 5, PS = G + 1, row0 = blockIdx.x * R, t = threadIdx.x;
    const size_t rowb = (size_t)(K / 256) * (TYPE == GW_Q4_K ? 144 : 210);
    for (int g = t; g < G; g += 256) {
        #pragma unroll
        for (int m = 0; m < M; m++) {
            const int8_t *x = xq + (size_t)m * ldx + 32 * g;
            float xsg = xs[(size_t)m * (ldx >> 5) + g], xfg = 0.0f;
            if (TYPE == GW_Q4_K) {
                int sum = 0;
                #pragma unroll
                for (int l = 0; l < 32; l++) sum += x[l];
                xfg = xsg * (float)sum; // kq_act_prep (kquants.h:392-400)
            }
            #pragma unroll
            for (int r = 0; r < R; r++) {
                int row = row0 + r < nrows ? row0 + r : nrows - 1;
                P[(m * R + r) * PS + g] = kq_term<TYPE>(W + (size_t)row * rowb, g, x, xsg, xfg);
            }
        }
    }
    __syncthreads();
    if (t < M * R) {
        int m = t / R, r = t % R, row = row0 + r;
        if (row < nrows) {
            const float *p = P + t * PS;
            float v = 0.0f;
            for (int g = 0; g < G; g++) v = v + p[g];
            float *o = out + (size_t)m * ldo + row;
            *o = mode == 1 ? *o + v : v;
        }
    }
}

// x[b] = row tok[b] of a K-quant table, dequantized (kq_dequant_row, kquants.h:222-251; every value one rounding
// of an exact expression)
__global__ __launch_bounds__(256) void k_embed_kq(float *__restrict__ x, int dim, int type, const uint8_t *__restrict__ W,
                                                  const int *__restrict__ tok) {
    int bidx = blockIdx.x;
    size_t rowb = (size_t)(dim / 256) * (type == GW_Q4_K ? 144 : 210);
    const uint8_t *rb = W + (size_t)tok[bidx] * rowb;
    for (int i = threadIdx.x; i < dim; i += blockDim.x) {
        int s = i >> 8, k = i & 255;
        float y;
        if (type == GW_Q4_K) {
            const uint8_t *b = rb + (size_t)s * 144, *sc = b + 4;
            int j = k >> 5, scj, mj;
            if (j < 4) { scj = sc[j] & 63; mj = sc[j + 4] & 63; }
            else { scj = (sc[j + 4] & 15) | (sc[j - 4] >> 6) << 4; mj = (sc[j + 4] >> 4) | (sc[j] >> 6) << 4; }
            float d = __half2float(__ushort_as_half((uint16_t)(b[0] | b[1] << 8)));
            float dmin = __half2float(__ushort_as_half((uint16_t)(b[2] | b[3] << 8)));
            int q = (b[16 + 32 * (k / 64) + k % 32] >> (4 * (k / 32 % 2))) & 15;
            float d1 = d * (float)scj, m1 = dmin * (float)mj;
            y = d1 * (float)q - m1;
        } else {
            const uint8_t *b = rb + (size_t)s * 210;
            int n = k / 128, p = k / 32 % 4, l = k % 32;
            int q = ((b[64 * n + 32 * (p & 1) + l] >> (4 * (p >> 1))) & 15) | ((b[128 + 32 * n + l] >> (2 * p)) & 3) << 4;
            float d = __half2float(__ushort_as_half((uint16_t)(b[208] | b[209] << 8)));
            y = (d * (float)(int8_t)b[192 + k / 16]) * (float)(q - 32);
        }
        x[(size_t)bidx * dim + i] = y;
    }
}

template <int TYPE>
static int launch_gemv_kq(const uint8_t *W, int nrows, int K, const int8_t *xq, const float *xs, int ldx, int M, float *out,
                          int ldo, int mode, hipStream_t s) {
    const int R = 4;
    size_t lds = (size_t)4 * R * (K / 32 + 1) * sizeof(float);
    hipEvent_t t0, t1; // (timing: the first launch's start, the last one's stop)
    gw_take_launch_events(&t0, &t1);
    for (int m0 = 0; m0 < M; m0 += 4) {
        int mm = M - m0 < 4 ? M - m0 : 4;
        hipEvent_t e0 = m0 == 0 ? t0 : NULL, e1 = m0 + 4 >= M ? t1 : NULL;
        dim3 grid((nrows + R - 1) / R);
        const int8_t *x = xq + (size_t)m0 * ldx;
        const float *xsc = xs + (size_t)m0 * (ldx / 32);
        float *o = out + (size_t)m0 * ldo;
        switch (mm) {
        case 1: hipExtLaunchKernelGGL((k_gemv_kq<TYPE, 1, R>), grid, dim3(256), lds, s, e0, e1, 0, W, nrows, K, x, xsc, ldx, o, ldo, mode); break;
        case 2: hipExtLaunchKernelGGL((k_gemv_kq<TYPE, 2, R>), grid, dim3(256), lds, s, e0, e1, 0, W, nrows, K, x, xsc, ldx, o, ldo, mode); break;
        case 3: hipExtLaunchKernelGGL((k_gemv_kq<TYPE, 3, R>), grid, dim3(256), lds, s, e0, e1, 0, W, nrows, K, x, xsc, ldx, o, ldo, mode); break;
        default: hipExtLaunchKernelGGL((k_gemv_kq<TYPE, 4, R>), grid, dim3(256), lds, s, e0, e1, 0, W, nrows, K, x, xsc, ldx, o, ldo, mode); break;
        }
    }
    return (int)hipGetLastError();
}

extern "C" {

int gw_k_embed_kq(float *x, int dim, int type, const uint8_t *blocks, const int *tok, int n, hipStream_t s) {
    hipEvent_t e0, e1;
    gw_take_launch_events(&e0, &e1);
    hipExtLaunchKernelGGL(k_embed_kq, dim3(n), dim3(256), 0, s, e0, e1, 0, x, dim, type, blocks, tok);
    return (int)hipGetLastError();
}

int gw_k_q8_unpack(const uint8_t *blocks, size_t nblk, int8_t *codes, uint16_t *scales, int gpr, int il, int off, hipStream_t s) {
    if (!nblk) return 0;
    hipLaunchKernelGGL(k_q8_unpack, dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0, s, blocks, nblk, codes, scales, gpr, il, off);
    return (int)hipGetLastError();
}

int gw_k_fill_synthetic(uint16_t *kc, uint16_t *vc, size_t n, unsigned long long seed, hipStream_t s) {
    if (!n) return 0;
    hipLaunchKernelGGL(k_fill_synthetic, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, kc, vc, n, seed);
    return (int)hipGetLastError();
}

static hipEvent_t tev0, tev1; // the pending timing pair of the next matmul launch (calls are single-threaded)

void gw_time_next_launch(hipEvent_t a, hipEvent_t b) {
    tev0 = a;
    tev1 = b;
}

void gw_take_launch_events(hipEvent_t *a, hipEvent_t *b) {
    *a = tev0;
    *b = tev1;
    tev0 = tev1 = NULL;
}

int gw_k_matmul(const GwMat *w, const int8_t *xq, const float *xs, int ldx, int M, float *out, int ldo, int mode, hipStream_t s) {
    if (w->type == GW_Q8_0 && M > GW_GEMV_MAX_ROWS && mode == 0) {
        hipEvent_t e0, e1;
        gw_take_launch_events(&e0, &e1);
        static int cus = 0;
        if (!cus) {
            int dev = 0;
            if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
                cus = 256;
        }
        int nt = (w->rows + GN - 1) / GN;
        if ((size_t)nt * ((M + 63) / 64) >= (size_t)4 * cus) // enough 64-row tiles for several waves per SIMD
            hipExtLaunchKernelGGL(k_gemm_q8<64>, dim3(nt, (M + 63) / 64), dim3(256), 0, s, e0, e1, 0, (const int8_t *)w->codes,
                                  (const uint16_t *)w->scales, w->rows, w->cols, xq, xs, ldx, M, out, ldo);
        else
            hipExtLaunchKernelGGL(k_gemm_q8<32>, dim3(nt, (M + 31) / 32), dim3(256), 0, s, e0, e1, 0, (const int8_t *)w->codes,
                                  (const uint16_t *)w->scales, w->rows, w->cols, xq, xs, ldx, M, out, ldo);
        return (int)hipGetLastError();
    }
    if (w->type == GW_Q8_0)
        return gw_k_gemv_q8(w->codes, w->scales, w->rows, w->cols, xq, xs, ldx, M, out, ldo, mode, s);
    if (w->type == GW_Q4_K)
        return launch_gemv_kq<GW_Q4_K>(w->blocks, w->rows, w->cols, xq, xs, ldx, M, out, ldo, mode, s);
    if (w->type == GW_Q6_K)
        return launch_gemv_kq<GW_Q6_K>(w->blocks, w->rows, w->cols, xq, xs, ldx, M, out, ldo, mode, s);
    return (int)hipErrorInvalidValue;
}

int gw_q8_pack(const void *blocks, int N, int K, int8_t *codes, uint16_t *scales, void *stream) {
    if (N <= 0 || K <= 0 || K % 32 || !blocks || !codes || !scales) return RQ_ERR_ARG;
    return gw_k_q8_unpack((const uint8_t *)blocks, (size_t)N * (K / 32), codes, scales, K / 32, 0, 0, (hipStream_t)stream) ? RQ_ERR_STATE : RQ_OK;
}

int gw_quantize(const float *x, int M, int K, int8_t *xq, float *xs, void *stream) {
    if (M <= 0 || K <= 0 || K % 32 || !x || !xq || !xs) return RQ_ERR_ARG;
    return gw_k_quant_rows(x, K, K, M, xq, xs, K, (hipStream_t)stream) ? RQ_ERR_STATE : RQ_OK;
}

int gw_q8_matmul(float *out, const int8_t *codes, const uint16_t *scales, int N, int K, const int8_t *xq, const float *xs,
                 int M, void *stream) {
    if (N <= 0 || K <= 0 || M <= 0 || N % 16 || K % 32 || !out || !codes || !scales || !xq || !xs) return RQ_ERR_ARG;
    GwMat w = { GW_Q8_0, N, K, (int8_t *)codes, (uint16_t *)scales, NULL };
    return gw_k_matmul(&w, xq, xs, K, M, out, N, 0, (hipStream_t)stream) ? RQ_ERR_STATE : RQ_OK;
}

int gw_q8_block_sums(int32_t *isum, const int8_t *codes, int N, int K, const int8_t *xq, int M, void *stream) {
    if (N <= 0 || K <= 0 || M <= 0 || K % 32 || !isum || !codes || !xq) return RQ_ERR_ARG;
    size_t tot = (size_t)M * N * (K / 32);
    hipLaunchKernelGGL(k_q8_block_sums, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, (hipStream_t)stream, isum, codes, N,
                       K, xq, M);
    return hipGetLastError() ? RQ_ERR_STATE : RQ_OK;
}

int gw_kq_matmul(float *out, int type, const void *blocks, int N, int K, const int8_t *xq, const float *xs, int M, void *stream) {
    if (N <= 0 || K <= 0 || M <= 0 || K % 256 || (type != GW_Q4_K && type != GW_Q6_K) || !out || !blocks || !xq || !xs)
        return RQ_ERR_ARG;
    GwMat w = { type, N, K, NULL, NULL, (uint8_t *)blocks };
    return gw_k_matmul(&w, xq, xs, K, M, out, N, 0, (hipStream_t)stream) ? RQ_ERR_STATE : RQ_OK;
}

} // extern "C"
