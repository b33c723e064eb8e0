// The matmul dispatch of the forward passes (gw_k_matmul), the load-time repack, and the isolated Q8_0 / K-quant
// operator of the public ABI (gw_q8_*, gw_kq_matmul, gw_quantize).
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <type_traits>

#include "gw_internal.h"
#include "gw_device.h"
#include "gw_iq.h"

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

// pseudo-random 16-bit K (|K| < 4) and V (|V| < 1) values, for timing runs (rq_seq_fill_synthetic): f16, or bf16 (bf:
// the bf16 and bf16-dot caches; every element drawn alike, so any tile layout holds the same distribution)
__global__ __launch_bounds__(256) void k_fill_synthetic(uint16_t *kc, uint16_t *vc, size_t n, unsigned long long seed, int bf) {
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    unsigned long long z = seed + i * 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    z ^= z >> 31;
    float a = (float)(z & 0xffffff) * (1.0f / 16777216.0f), b = (float)((z >> 24) & 0xffffff) * (1.0f / 16777216.0f);
    const float k = (2.0f * a - 1.0f) * 3.9f, v = (2.0f * b - 1.0f) * 0.99f;
    kc[i] = bf ? f2bf_ref(k) : __half_as_ushort(__float2half(k));
    vc[i] = bf ? f2bf_ref(v) : __half_as_ushort(__float2half(v));
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
typedef float f32x32 __attribute__((ext_vector_type(32)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
#define GN 128
#define GKB 128
#define GROW 144
template <int GM>
__global__ __launch_bounds__(256) void k_gemm_q8(const int8_t *__restrict__ W, const uint16_t *__restrict__ WS, int N, int K,
                                                 const int8_t *__restrict__ X, const float *__restrict__ XS, int ldx, int M,
                                                 float *__restrict__ out, int ldo) {
    // software-pipelined: the stage after the current one is loaded into registers while the current one is computed
    // from LDS (two LDS buffers), then stored into the other buffer; one barrier per stage and one loop exit (a loop
    // that can leave after each step makes the compiler wait for every load in flight at its top)
    constexpr int TJ = GM == 64 ? 2 : 1, XC = GM * 8 / 256; // MFMA tiles per wave, X chunks of 16 B per thread
    __shared__ __align__(16) int8_t xl[2][GM * GROW];
    __shared__ __align__(16) int8_t wl[2][GN * GROW];
    __shared__ __align__(16) float xsl[2][4][GM];
    __shared__ float wsl[2][GN][4];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int m0 = blockIdx.y * GM, n0 = blockIdx.x * GN, G = K >> 5, NS = (K + GKB - 1) / GKB;
    const int wm = GM == 64 ? (wave >> 1) * 32 : 0, wn = GM == 64 ? (wave & 1) * 64 : wave * 32; // the wave's sub-tile
    float acc[TJ][16];
    #pragma unroll
    for (int j = 0; j < TJ; j++)
        #pragma unroll
        for (int r = 0; r < 16; r++) acc[j][r] = 0.0f;
    // a stage in registers: X rows m0.. (GM x 128 B: XC chunks of 16 B per thread), W rows n0.. (GN x 128 B: 4 per
    // thread), this thread's activation scale and two weight scales (every load unconditional: past K or the last
    // row, clamped addresses; the values past K are zeroed when stored, not here, where it would wait for the loads)
    const int srow = t >> 2, sgg = t & 3;
    const int sm = m0 + srow < M ? m0 + srow : M - 1;
    const int sn = n0 + srow < N ? n0 + srow : N - 1, sn2 = n0 + srow + 64 < N ? n0 + srow + 64 : N - 1;
    struct St { // (named fields, passed by value: arrays captured by the lambdas were placed in scratch memory)
        uint4 x0, x1, w0, w1, w2, w3;
        float xs, ws0, ws1;
    };
    auto xptr = [&](int k, int k0, int ng) __attribute__((always_inline)) -> const uint4 * {
        const int c = t + 256 * k, row = c >> 3, col = (c & 7) * 16, m = m0 + row < M ? m0 + row : M - 1;
        return (const uint4 *)(X + (size_t)m * ldx + k0 + (col < ng * 32 ? col : 0));
    };
    auto wptr = [&](int k, int k0, int ng) __attribute__((always_inline)) -> const uint4 * {
        const int c = t + 256 * k, row = c >> 3, col = (c & 7) * 16, n = n0 + row < N ? n0 + row : N - 1;
        return (const uint4 *)(W + (size_t)n * K + k0 + (col < ng * 32 ? col : 0));
    };
    auto load = [&](int st) __attribute__((always_inline)) -> St {
        st = st < NS ? st : NS - 1;
        const int k0 = st * GKB, ng = (K - k0) < GKB ? (K - k0) >> 5 : 4, gq = sgg < ng ? sgg : 0;
        St o;
        o.x0 = *xptr(0, k0, ng);
        o.x1 = XC > 1 ? *xptr(1, k0, ng) : o.x0;
        o.w0 = *wptr(0, k0, ng);
        o.w1 = *wptr(1, k0, ng);
        o.w2 = *wptr(2, k0, ng);
        o.w3 = *wptr(3, k0, ng);
        o.xs = XS[(size_t)sm * (ldx >> 5) + (k0 >> 5) + gq];
        o.ws0 = h2f_g(WS[(size_t)sn * G + (k0 >> 5) + gq]);
        o.ws1 = h2f_g(WS[(size_t)sn2 * G + (k0 >> 5) + gq]);
        return o;
    };
    auto store = [&](const St o, int buf, int st) __attribute__((always_inline)) {
        // stage st's registers into buffer buf (codes past K and scales of missing groups: 0)
        const int ng = (K - st * GKB) < GKB ? (K - st * GKB) >> 5 : 4;
        const bool in = (t & 7) * 16 < ng * 32; // (c & 7 is t & 7 for every chunk c = t + 256 k)
        // (the select per component: a ?: between two uint4 values went through scratch memory)
        auto sel = [&](const uint4 v) __attribute__((always_inline)) -> uint4 {
            return make_uint4(in ? v.x : 0u, in ? v.y : 0u, in ? v.z : 0u, in ? v.w : 0u);
        };
        const int r0 = (t >> 3) * GROW + (t & 7) * 16; // (chunk t + 256 k: row (t >> 3) + 32 k, the same column)
        *(uint4 *)(&xl[buf][r0]) = sel(o.x0);
        if (XC > 1) *(uint4 *)(&xl[buf][r0 + 32 * GROW]) = sel(o.x1);
        *(uint4 *)(&wl[buf][r0]) = sel(o.w0);
        *(uint4 *)(&wl[buf][r0 + 32 * GROW]) = sel(o.w1);
        *(uint4 *)(&wl[buf][r0 + 64 * GROW]) = sel(o.w2);
        *(uint4 *)(&wl[buf][r0 + 96 * GROW]) = sel(o.w3);
        if (srow < GM) xsl[buf][sgg][srow] = sgg < ng ? o.xs : 0.0f;
        wsl[buf][srow][sgg] = sgg < ng ? o.ws0 : 0.0f;
        wsl[buf][srow + 64][sgg] = sgg < ng ? o.ws1 : 0.0f;
    };
    store(load(0), 0, 0);
    __syncthreads();
    for (int st = 0; st < NS; st++) {
        const int buf = st & 1, k0 = st * GKB, ng = (K - k0) < GKB ? (K - k0) >> 5 : 4; // groups in this stage
        const St nx = load(st + 1); // (past the last stage: the last again, never stored)
        for (int gg = 0; gg < ng; gg++) {
            i32x4 a = *(const i32x4 *)(&xl[buf][(wm + (lane & 31)) * GROW + gg * 32 + 16 * (lane >> 5)]);
            #pragma unroll
            for (int j = 0; j < TJ; j++) {
                i32x4 b = *(const i32x4 *)(&wl[buf][(wn + 32 * j + (lane & 31)) * GROW + gg * 32 + 16 * (lane >> 5)]);
                i32x16 z = { 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0 };
                i32x16 I = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, z, 0, 0, 0);
                float ws = wsl[buf][wn + 32 * j + (lane & 31)][gg];
                #pragma unroll
                for (int q = 0; q < 4; q++) {
                    float4 xs4 = *(const float4 *)(&xsl[buf][gg][wm + 8 * q + 4 * (lane >> 5)]);
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
        if (st + 1 < NS) store(nx, buf ^ 1, st + 1); // (the other buffer's readers, stage st - 1, are past the last barrier)
        __syncthreads();
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

// k_gemm_q8 for K % GKB == 0 (every stage full: the model's widths): the same tiles, pipeline and fold, with fewer
// instructions around the fold (which needs 4 VALU instructions per output and group: the bound of this GEMM). Loads
// through buffer descriptors over the block's own rows: rows past M or N read as 0 (the descriptor's range), so no
// clamped addresses and no selects; each thread's offsets are fixed and a stage moves the scalar offset only.
template <int GM>
__global__ __launch_bounds__(256) void k_gemm_q8f(const int8_t *__restrict__ W, const uint16_t *__restrict__ WS, int N, int K,
                                                  const int8_t *__restrict__ X, const float *__restrict__ XS, int ldx, int M,
                                                  float *__restrict__ out, int ldo) {
    constexpr int TJ = GM == 64 ? 2 : 1, XC = GM * 8 / 256;
    __shared__ __align__(16) int8_t xl[2][GM * GROW];
    __shared__ __align__(16) int8_t wl[2][GN * GROW];
    __shared__ __align__(16) float xsl[2][4][GM];
    __shared__ float wsl[2][GN][4];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int m0 = blockIdx.y * GM, n0 = blockIdx.x * GN, G = K >> 5, NS = K / GKB, gx = ldx >> 5;
    const int wm = GM == 64 ? (wave >> 1) * 32 : 0, wn = GM == 64 ? (wave & 1) * 64 : wave * 32;
    const int mr = M - m0 < GM ? M - m0 : GM, nr = N - n0 < GN ? N - n0 : GN; // (the block's rows)
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void *)(X + (size_t)m0 * ldx), (short)0, mr * ldx, GW_RSRC_DW3);
    const __amdgpu_buffer_rsrc_t rxs = __builtin_amdgcn_make_buffer_rsrc((void *)(XS + (size_t)m0 * gx), (short)0, mr * gx * 4, GW_RSRC_DW3);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void *)(W + (size_t)n0 * K), (short)0, nr * K, GW_RSRC_DW3);
    const __amdgpu_buffer_rsrc_t rws = __builtin_amdgcn_make_buffer_rsrc((void *)(WS + (size_t)n0 * G), (short)0, nr * G * 2, GW_RSRC_DW3);
    float acc[TJ][16];
    #pragma unroll
    for (int j = 0; j < TJ; j++)
        #pragma unroll
        for (int r = 0; r < 16; r++) acc[j][r] = 0.0f;
    // this thread's chunks (16 B: chunk c = t + 256 k is row c / 8, bytes 16 (c % 8) .. of the stage's 128) and scales
    // (row t / 4, group t % 4 of the stage; W rows t / 4 and t / 4 + 64)
    const int crow = t >> 3, ccol = (t & 7) * 16, srow = t >> 2, sgg = t & 3;
    const int xo = crow * ldx + ccol, wo = crow * K + ccol, xso = (srow * gx + sgg) * 4, wso = (srow * G + sgg) * 2;
    struct St {
        uint4 x0, x1, w0, w1, w2, w3;
        float xs, ws0, ws1;
    };
    auto ld16 = [&](__amdgpu_buffer_rsrc_t r, int vo, int so) __attribute__((always_inline)) -> uint4 {
        return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, 0));
    };
    auto load = [&](int st) __attribute__((always_inline)) -> St {
        const int k0 = st * GKB; // (st = NS: past the last stage, inside the buffers or read as 0; never stored)
        St o;
        o.x0 = ld16(rx, xo, k0);
        o.x1 = XC > 1 ? ld16(rx, xo + 32 * ldx, k0) : o.x0;
        o.w0 = ld16(rw, wo, k0);
        o.w1 = ld16(rw, wo + 32 * K, k0);
        o.w2 = ld16(rw, wo + 64 * K, k0);
        o.w3 = ld16(rw, wo + 96 * K, k0);
        o.xs = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rxs, xso, st * 16, 0));
        o.ws0 = h2f_g(__builtin_amdgcn_raw_buffer_load_b16(rws, wso, st * 8, 0));
        o.ws1 = h2f_g(__builtin_amdgcn_raw_buffer_load_b16(rws, wso + 64 * G * 2, st * 8, 0));
        return o;
    };
    auto store = [&](const St o, int buf) __attribute__((always_inline)) {
        const int r0 = crow * GROW + ccol;
        *(uint4 *)(&xl[buf][r0]) = o.x0;
        if (XC > 1) *(uint4 *)(&xl[buf][r0 + 32 * GROW]) = o.x1;
        *(uint4 *)(&wl[buf][r0]) = o.w0;
        *(uint4 *)(&wl[buf][r0 + 32 * GROW]) = o.w1;
        *(uint4 *)(&wl[buf][r0 + 64 * GROW]) = o.w2;
        *(uint4 *)(&wl[buf][r0 + 96 * GROW]) = o.w3;
        if (srow < GM) xsl[buf][sgg][srow] = o.xs;
        wsl[buf][srow][sgg] = o.ws0;
        wsl[buf][srow + 64][sgg] = o.ws1;
    };
    const int xa = (wm + (lane & 31)) * GROW + 16 * (lane >> 5), wa = (wn + (lane & 31)) * GROW + 16 * (lane >> 5);
    auto compute = [&](int buf) __attribute__((always_inline)) {
        // the stage's groups in pairs (g0, g0 + 1): per 32 x 32 tile the two exact sums (int8 MFMA) and the two groups'
        // scale products ws * xs as one outer-product MFMA (v_mfma_f32_32x32x1f32, two blocks: lane i gives group
        // g0 + i / 32's xs of row i % 32 and ws of column i % 32; each result one fp32 product rounded once, as the
        // VALU's multiply), so the VALU's fold is 3 instructions per output and group: (float) isum, the multiply by
        // the product, the add. (rolled: unrolled, the compiler keeps every MFMA result live at once; an explicit
        // software pipeline, the next tile's MFMAs issued before this tile's fold and pinned there, measured 17 % slower)
        #pragma unroll 1
        for (int g0 = 0; g0 < 4; g0 += 2) {
            const i32x4 a0 = *(const i32x4 *)(&xl[buf][xa + g0 * 32]), a1 = *(const i32x4 *)(&xl[buf][xa + g0 * 32 + 32]);
            const float xsa = xsl[buf][g0 + (lane >> 5)][wm + (lane & 31)];
            #pragma unroll
            for (int j = 0; j < TJ; j++) {
                const i32x4 b0 = *(const i32x4 *)(&wl[buf][wa + 32 * j * GROW + g0 * 32]);
                const i32x4 b1 = *(const i32x4 *)(&wl[buf][wa + 32 * j * GROW + g0 * 32 + 32]);
                const i32x16 z = { 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0 };
                const f32x32 zf = {};
                const i32x16 I0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b0, z, 0, 0, 0);
                const i32x16 I1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b1, z, 0, 0, 0);
                const float wsb = wsl[buf][wn + 32 * j + (lane & 31)][g0 + (lane >> 5)];
                const f32x32 C = __builtin_amdgcn_mfma_f32_32x32x1f32(xsa, wsb, zf, 0, 0, 0);
                #pragma unroll
                for (int r = 0; r < 16; r++) acc[j][r] = acc[j][r] + C[r] * (float)I0[r];
                #pragma unroll
                for (int r = 0; r < 16; r++) acc[j][r] = acc[j][r] + C[16 + r] * (float)I1[r];
            }
        }
    };
    // two stages' loads in flight: register sets sa and sb take turns (stage st + 1 in sa, st + 2 loaded into sb while
    // stage st is computed, and so on; a copy from one set into the other would wait for its loads), the stages in LDS
    // buffers 0 / 1 by parity; each buffer is rewritten only after the barrier that follows its readers
    St sa = load(1);
    store(load(0), 0);
    __syncthreads();
    int st = 0;
    for (; st + 1 < NS; st += 2) {
        const St sb = load(st + 2); // (past the last stage: inside the buffers or read as 0; never stored)
        compute(0);
        store(sa, 1);
        __syncthreads();
        sa = load(st + 3);
        compute(1);
        if (st + 2 < NS) store(sb, 0);
        __syncthreads();
    }
    if (st < NS) compute(0); // (an odd stage count: the last stage, in buffer 0)
    #pragma unroll
    for (int j = 0; j < TJ; j++) {
        const int n = n0 + wn + 32 * j + (lane & 31);
        #pragma unroll
        for (int r = 0; r < 16; r++) {
            const int m = m0 + wm + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (m < M && n < N) out[(size_t)m * ldo + n] = acc[j][r];
        }
    }
}

// Q8_0 GEMM whose stages reach LDS by the buffer unit's direct copies (buffer_load_dwordx4 ... lds): no staging
// registers and no LDS writes by the waves, a ring of LQ_S stages so that two are in flight while one is computed.
// Blocks of 64 rows x TN columns (TN = 128: 8 waves, two blocks per CU; TN = 64: 4 waves, three per CU): wave w takes
// the 32 x 32 tile of rows 32 (w / NC), columns 32 (w % NC), NC = TN / 32.
// A copy writes a wave's 64 lanes to 1 KB of consecutive LDS, so stage rows (128 bytes = 4 groups) cannot be padded
// apart; chunk c (16 bytes) of row r is stored at chunk c ^ ((r / 2) % 8), which puts the MFMA operand reads of 16
// consecutive rows (a 16-byte read serves 16 lanes per cycle from the 64 banks) on distinct banks (c ^ (r % 8) had
// rows r and r + 8 on one bank: 3 conflict cycles per LDS-active cycle). Per stage, wave w copies 8 / NW of the 8
// X pieces and W pieces 2 w, 2 w + 1
// (1 KB = 8 rows each), wave 0 the stage's xs (a lane per row), waves 1 .. NC the ws (fp16, a dword = 2 groups of one
// row per lane). Per pair of groups the fold of k_gemm_q8f: two int8 MFMAs for the exact sums, the outer-product MFMA
// of the scale products, then val = val + (ws xs) (float) isum per output in group order (forward.c:906-916). Blocks:
// XCD b % 8 takes column tiles 8 q + b % 8 with their row tiles in a row (the W tile read once into that XCD's L2).
// mode 0 (out = val), K % 128 == 0; rows past M / N read as 0 (the descriptors' ranges) and are not stored. (The w1 / w3
// SwiGLU with its quantization in this kernel's epilogue, the row maxima of a quantization group's two halves exchanged
// between waves in LDS, was measured against its own kernel after the GEMM: 8B prefill 22.7 k against 23.2 k tok/s,
// the epilogue's table reads waiting at the end of each block)
#define LQ_S 3
#define LQ_X 0
#define LQ_W 8192
#define LQ_XS(TN) (8192 + 128 * (TN))
#define LQ_WS(TN) (8192 + 128 * (TN) + 1024)
#define LQ_STAGE(TN) (8192 + 136 * (TN) + 1024)
#define LQ_AS3 __attribute__((address_space(3)))
template <int C, int LMAX, int L = 0>
__device__ __forceinline__ void lq_vmwait(int n) {
    // s_waitcnt vmcnt(C n) for a wave-uniform n in 0 .. LMAX (the count is an immediate)
    if constexpr (L < LMAX) {
        if (n == L) {
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(C * L) : "memory");
            return;
        }
        lq_vmwait<C, LMAX, L + 1>(n);
    } else {
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(C * L) : "memory");
    }
}
__device__ __forceinline__ void lq_copy(__amdgpu_buffer_rsrc_t r, uint8_t *lds, int voff, int bytes) {
    // (the offset in the per-lane operand, so the descriptor's range check sees all of it)
    if (bytes == 16) __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LQ_AS3 void *)lds, 16, voff, 0, 0, 0);
    else __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LQ_AS3 void *)lds, 4, voff, 0, 0, 0);
}
template <int TN>
__global__ __launch_bounds__(TN * 4, TN == 128 ? 2 : 3) void k_gemm_q8l(const int8_t *__restrict__ W,
                                                                       const uint16_t *__restrict__ WS, int N, int K,
                                                                       const int8_t *__restrict__ X,
                                                                       const float *__restrict__ XS, int ldx, int M,
                                                                       float *__restrict__ out, int ldo, int MT) {
    constexpr int NC = TN / 32, NW = 2 * NC, XP = 8 / NW; // (waves per row of tiles, waves, X pieces per wave)
    __shared__ __align__(16) uint8_t sl[LQ_S * LQ_STAGE(TN)];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, hi = lane >> 5, r32 = lane & 31;
    const int b = blockIdx.x, j = b >> 3, nt = (N + TN - 1) / TN;
    const int ntile = (j / MT) * 8 + (b & 7), m0 = (j % MT) * 64, n0 = ntile * TN;
    if (ntile >= nt) return; // (the grid's padding to 8 column tiles per XCD)
    const int G = K >> 5, gx = ldx >> 5, NS = K >> 7;
    const int mr = M - m0 < 64 ? M - m0 : 64, nr = N - n0 < TN ? N - n0 : TN;
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void *)(X + (size_t)m0 * ldx), (short)0, mr * ldx, GW_RSRC_DW3);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void *)(W + (size_t)n0 * K), (short)0, nr * K, GW_RSRC_DW3);
    const __amdgpu_buffer_rsrc_t rxs = __builtin_amdgcn_make_buffer_rsrc((void *)(XS + (size_t)m0 * gx), (short)0, mr * gx * 4, GW_RSRC_DW3);
    const __amdgpu_buffer_rsrc_t rws = __builtin_amdgcn_make_buffer_rsrc((void *)(WS + (size_t)n0 * G), (short)0, nr * G * 2, GW_RSRC_DW3);
    // this lane's copies: row 8 p + lane / 8 of its 1 KB piece p, logical chunk (lane % 8) ^ ((row / 2) % 8), which is
    // (lane % 8) ^ (lane / 16) in an even piece, (lane % 8) ^ (4 + lane / 16) in an odd one
    const int pr = lane >> 3, pce = (lane & 7) ^ (pr >> 1), pco = (lane & 7) ^ (4 + (pr >> 1));
    const int xo = (8 * XP * wave + pr) * ldx, wo = (16 * wave + pr) * K + 16 * pce, wo1 = (16 * wave + 8 + pr) * K + 16 * pco;
    const int so = wave == 0 ? lane * gx * 4 : ((32 * (wave - 1) + (lane >> 1)) * G + 2 * (lane & 1)) * 2;
    auto issue = [&](int st, int slot) __attribute__((always_inline)) { // (slot: st % LQ_S)
        uint8_t *bs = sl + slot * LQ_STAGE(TN);
        const int k0 = st * 128;
        #pragma unroll
        for (int p = 0; p < XP; p++) // (piece XP wave + p: odd where XP == 1 and the wave is odd, or p is)
            lq_copy(rx, bs + LQ_X + 1024 * (XP * wave + p), xo + 8 * p * ldx + 16 * (((XP * wave + p) & 1) ? pco : pce) + k0, 16);
        lq_copy(rw, bs + LQ_W + 2048 * wave, wo + k0, 16);
        lq_copy(rw, bs + LQ_W + 2048 * wave + 1024, wo1 + k0, 16);
        if (wave == 0) lq_copy(rxs, bs + LQ_XS(TN), so + 16 * st, 16);
        else if (wave <= NC) lq_copy(rws, bs + LQ_WS(TN) + 256 * (wave - 1), so + 8 * st, 4);
    };
    const int wm = (wave / NC) * 32, wn = (wave % NC) * 32;
    float acc[16];
    #pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.0f;
    const int xa = LQ_X + (wm + r32) * 128, wa = LQ_W + (wn + r32) * 128, sw = (r32 >> 1) & 7;
    const int xsa_o = LQ_XS(TN) + (wm + r32) * 16 + 4 * hi, wsb_o = LQ_WS(TN) + (wn + r32) * 8 + 2 * hi;
    // the operands' offsets in a stage (the same every stage): group 2 p + u's 16 bytes of this lane, chunk 4 p + 2 u + hi
    int oa[4], ob[4];
    #pragma unroll
    for (int q = 0; q < 4; q++) {
        const int c = 16 * ((2 * q + hi) ^ sw);
        oa[q] = xa + c;
        ob[q] = wa + c;
    }
    issue(0, 0);
    if (NS > 1) issue(1, 1);
    for (int st = 0; st < NS; st++) {
        // stage st landed (this wave's copies: only stage st + 1's XP + 3 or XP + 2 outstanding), then every wave's
        if (st + 1 < NS) {
            if (wave <= NC) {
                if (XP == 1) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
                else asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
            } else {
                if (XP == 1) asm volatile("s_waitcnt vmcnt(3)" ::: "memory");
                else asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
            }
        } else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (st + 2 < NS) issue(st + 2, (st + 2) % LQ_S); // (into the slot of stage st - 1, whose readers are past the barrier)
        const uint8_t *bs = sl + (st % LQ_S) * LQ_STAGE(TN);
        // both pairs' operands first: the second pair's LDS reads complete under the first pair's MFMAs and fold
        i32x4 A[4], B[4];
        float XA[2], WB[2];
        #pragma unroll
        for (int p = 0; p < 2; p++) {
            A[2 * p] = *(const i32x4 *)(bs + oa[2 * p]);
            A[2 * p + 1] = *(const i32x4 *)(bs + oa[2 * p + 1]);
            B[2 * p] = *(const i32x4 *)(bs + ob[2 * p]);
            B[2 * p + 1] = *(const i32x4 *)(bs + ob[2 * p + 1]);
            XA[p] = *(const float *)(bs + xsa_o + 8 * p);
            WB[p] = h2f_g(*(const uint16_t *)(bs + wsb_o + 4 * p));
        }
        #pragma unroll
        for (int p = 0; p < 2; p++) {
            const i32x16 z = { 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0 };
            const f32x32 zf = {};
            const i32x16 I0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[2 * p], B[2 * p], z, 0, 0, 0);
            const i32x16 I1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[2 * p + 1], B[2 * p + 1], z, 0, 0, 0);
            const f32x32 C = __builtin_amdgcn_mfma_f32_32x32x1f32(XA[p], WB[p], zf, 0, 0, 0);
            #pragma unroll
            for (int r = 0; r < 16; r++) acc[r] = acc[r] + C[r] * (float)I0[r];
            #pragma unroll
            for (int r = 0; r < 16; r++) acc[r] = acc[r] + C[16 + r] * (float)I1[r];
            if (p == 0) __builtin_amdgcn_sched_barrier(0); // (the second pair's MFMAs after the first pair's fold)
        }
    }
    const int n = n0 + wn + r32;
    #pragma unroll
    for (int r = 0; r < 16; r++) {
        const int m = m0 + wm + 8 * (r >> 2) + 4 * hi + (r & 3);
        if (m < M && n < N) out[(size_t)m * ldo + n] = acc[r];
    }
}

// k_gemm_q8l's 64 x 64 stages (the same LDS copies, ring, swizzle and block order) with 16 waves of 16 x 16 tiles
// (v_mfma_i32_16x16x32_i8: one group per instruction; the 4 groups' scale products ws xs from one
// v_mfma_f32_16x16x1f32 of 4 blocks, each product one fp32 rounding as the VALU's multiply): a wave's fold is 4
// outputs per lane, a quarter of a 32 x 32 tile's, so a block's 64 x 64 outputs are folded by 16 waves in parallel.
// For few rows (one or two row tiles) the 32 x 32 waves sit one per SIMD with 16 outputs each, and their fold's
// dependent chain of latencies sets the time. Copies per stage: wave w < 8 X piece w, wave 8 + p W piece p, wave 0 the
// xs, waves 1 and 2 the ws. mode 0, K % 128 == 0
template <int TM, int TN, int S, int Q>
__global__ __launch_bounds__(TM * TN / 4, TM * TN >= 4096 ? 1 : 2) void k_gemm_q8t(const int8_t *__restrict__ W,
                                                                               const uint16_t *__restrict__ WS, int N, int K,
                                                                               const int8_t *__restrict__ X,
                                                                               const float *__restrict__ XS, int ldx, int M,
                                                                               float *__restrict__ out, int ldo, int MT) {
    // blocks of TM x TN outputs (16 x 16 per wave, NW = TM TN / 256 waves); S stages in the ring, each of GK = 128 Q
    // bytes of K (GP = 4 Q groups): X TM x GK, W TN x GK, xs TM x GP floats, ws TN x GP halves. A stage's copies are
    // pieces of 1 KB (RPP = 1024 / GK rows) of X, then of W, then the xs pieces (1 KB: 1024 / (4 GP) rows) and the ws
    // pieces (dwords, 256 bytes: 128 / GP rows), piece p copied by wave p % NW
    constexpr int NW = TM * TN / 256, GK = 128 * Q, GP = 4 * Q, CH = GK / 16, RPP = 1024 / GK;
    constexpr int PX = TM * GK / 1024, PW = TN * GK / 1024, PXS = (TM * GP * 4 + 1023) / 1024, PWS = TN * GP * 2 / 256;
    constexpr int PT = PX + PW + PXS + PWS, PPW = (PT + NW - 1) / NW; // (pieces, per wave at most)
    constexpr int OX = 0, OW = TM * GK, OXS = (TM + TN) * GK, OWS = OXS + PXS * 1024, STG = OWS + TN * GP * 2;
    static_assert(PT <= 63 && TM % 16 == 0 && TN % 16 == 0 && PWS * 256 == TN * GP * 2, "tile shape");
    __shared__ __align__(16) uint8_t sl[S * STG];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, l16 = lane & 15, q4 = lane >> 4;
    const int b = blockIdx.x, j = b >> 3, nt = (N + TN - 1) / TN;
    const int ntile = (j / MT) * 8 + (b & 7), m0 = (j % MT) * TM, n0 = ntile * TN;
    if (ntile >= nt) return; // (the grid's padding to 8 column tiles per XCD)
    const int G = K >> 5, gx = ldx >> 5, NS = K / GK;
    const int mr = M - m0 < TM ? M - m0 : TM, nr = N - n0 < TN ? N - n0 : TN;
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc((void *)(X + (size_t)m0 * ldx), (short)0, mr * ldx, GW_RSRC_DW3);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void *)(W + (size_t)n0 * K), (short)0, nr * K, GW_RSRC_DW3);
    const __amdgpu_buffer_rsrc_t rxs = __builtin_amdgcn_make_buffer_rsrc((void *)(XS + (size_t)m0 * gx), (short)0, mr * gx * 4, GW_RSRC_DW3);
    const __amdgpu_buffer_rsrc_t rws = __builtin_amdgcn_make_buffer_rsrc((void *)(WS + (size_t)n0 * G), (short)0, nr * G * 2, GW_RSRC_DW3);
    // the swizzle: chunk c of row r at c ^ sw(r), so that 16 consecutive rows' reads of one chunk fall on distinct banks
    auto swz = [](int r) -> int { return Q == 1 ? (r >> 1) & 7 : r & 15; };
    // piece p's LDS offset in a stage, its buffer and its per-lane byte offset at K = 0 (stage st adds GK st, or 4 GP st
    // for xs, 2 GP st for ws)
    auto piece = [&](int p, int &lo, int &vo, int &kind) __attribute__((always_inline)) {
        if (p < PX + PW) { // X or W: row RPP q + lane / CH, physical chunk lane % CH
            const bool w = p >= PX;
            const int q = w ? p - PX : p, row = RPP * q + lane / CH, lc = (lane % CH) ^ swz(row);
            lo = (w ? OW : OX) + 1024 * q;
            vo = row * (w ? K : ldx) + 16 * lc;
            kind = w ? 1 : 0;
        } else if (p < PX + PW + PXS) { // xs: 16 bytes per lane, GP / 4 lanes per row
            const int q = p - PX - PW, row = (1024 / (4 * GP)) * q + lane / (GP / 4), h = lane % (GP / 4);
            lo = OXS + 1024 * q;
            vo = (row * gx + 4 * h) * 4;
            kind = 2;
        } else { // ws: a dword (2 groups) per lane, GP / 2 lanes per row
            const int q = p - PX - PW - PXS, row = (128 / GP) * q + lane / (GP / 2), h = lane % (GP / 2);
            lo = OWS + 256 * q;
            vo = (row * G + 2 * h) * 2;
            kind = 3;
        }
    };
    int plo[PPW], pvo[PPW], pk[PPW];
    #pragma unroll
    for (int i = 0; i < PPW; i++) piece(wave + NW * i < PT ? wave + NW * i : 0, plo[i], pvo[i], pk[i]);
    const int cnt = (PT - wave + NW - 1) / NW; // (this wave's pieces per stage)
    auto issue = [&](int st) __attribute__((always_inline)) {
        uint8_t *bs = sl + (st % S) * STG;
        #pragma unroll
        for (int i = 0; i < PPW; i++) {
            if (i < cnt) {
                if (pk[i] == 0) lq_copy(rx, bs + plo[i], pvo[i] + GK * st, 16);
                else if (pk[i] == 1) lq_copy(rw, bs + plo[i], pvo[i] + GK * st, 16);
                else if (pk[i] == 2) lq_copy(rxs, bs + plo[i], pvo[i] + 4 * GP * st, 16);
                else lq_copy(rws, bs + plo[i], pvo[i] + 2 * GP * st, 4);
            }
        }
    };
    const int wm = (wave / (TN / 16)) * 16, wn = (wave % (TN / 16)) * 16; // (this wave's 16 x 16 tile)
    float acc[4] = { 0.0f, 0.0f, 0.0f, 0.0f };
    // operands: A row wm + l16 (X), B row wn + l16 (W), bytes 32 g + 8 q4 .. + 7 of the stage row: logical chunk
    // 2 g + q4 / 2, its half q4 % 2
    const int xr = wm + l16, wr = wn + l16;
    const int xa = OX + xr * GK + 8 * (q4 & 1), wa = OW + wr * GK + 8 * (q4 & 1);
    const int xsw = swz(xr), wsw = swz(wr);
    const int xsa_o = OXS + xr * GP * 4 + 4 * q4, wsb_o = OWS + wr * GP * 2 + 2 * q4;
    // S - 1 stages in flight: the ring holds S; stage st's slot is refilled with stage st + S after the barrier of
    // stage st + 1 (its readers are past it)
    for (int p = 0; p < S - 1 && p < NS; p++) issue(p);
    for (int st = 0; st < NS; st++) {
        // stage st landed: this wave's copies of the later stages issued (L stages of cnt copies) may be outstanding
        const int L = NS - 1 - st < S - 2 ? NS - 1 - st : S - 2;
        if (cnt == PPW) lq_vmwait<PPW, S - 2>(L);
        else if (PPW > 1 && cnt == PPW - 1) lq_vmwait<(PPW > 1 ? PPW - 1 : 1), S - 2>(L);
        else lq_vmwait<(PPW > 2 ? PPW - 2 : 1), S - 2>(L);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (st + S - 1 < NS) issue(st + S - 1); // (into the slot of stage st - 1, whose readers are past the barrier)
        const uint8_t *bs = sl + (st % S) * STG;
        #pragma unroll
        for (int q = 0; q < Q; q++) {
            // groups 4 q .. 4 q + 3: their scale products (block g: xs of row 4 (lane / 16) + r, ws of column lane % 16)
            const float xsa = *(const float *)(bs + xsa_o + 16 * q), wsb = h2f_g(*(const uint16_t *)(bs + wsb_o + 8 * q));
            const f32x16 zf = {};
            const f32x16 C = __builtin_amdgcn_mfma_f32_16x16x1f32(xsa, wsb, zf, 0, 0, 0);
            i32x4 I[4];
            #pragma unroll
            for (int g = 0; g < 4; g++) {
                const int c = 2 * (4 * q + g) + (q4 >> 1);
                const long a = *(const long *)(bs + xa + 16 * (c ^ xsw)), bb = *(const long *)(bs + wa + 16 * (c ^ wsw));
                const i32x4 z = { 0, 0, 0, 0 };
                I[g] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bb, z, 0, 0, 0);
            }
            #pragma unroll
            for (int g = 0; g < 4; g++)
                #pragma unroll
                for (int r = 0; r < 4; r++) acc[r] = acc[r] + C[4 * g + r] * (float)I[g][r];
        }
    }
    const int n = n0 + wn + l16;
    #pragma unroll
    for (int r = 0; r < 4; r++) {
        const int m = m0 + wm + 4 * q4 + r;
        if (m < M && n < N) out[(size_t)m * ldo + n] = acc[r];
    }
}

typedef long i64;

// ------------------------------------------------------------------------------------- K-quant MFMA GEMM

// out[m * ldo + n] (+)= W row n . X row m for m < M, n < N, W in the file's Q4_K / Q6_K super-blocks (batched rows,
// prefill): the tiling of k_gemm_q8 (GM x 128 outputs per block of 4 waves, stages of 128 values = 4 groups of 32 = half
// a super-block), each stage's weights unpacked into int8 rows in LDS, then per group the reference's term and fold
// (kquants.h:86-109, :410-554):
//   Q4_K: codes 0 .. 15; I = the exact sum q x (v_mfma_i32_32x32x32_i8), S = the exact sum of x (the same MFMA with
//     B = 1); term = ((d sc_j) xs) I - (dmin m_j) (xs S)
//   Q6_K: codes q - 32 (-32 .. 31, exact in int8; q 6-bit from ql / qh); per half-group of 16 the exact sum
//     (v_mfma_i32_32x32x16_i8), I = sc_0 I_0 + sc_1 I_1 (exact int); term = (d xs) I
//   the i-quants (IQ4_XS and the codebook types: each unit's 16 v and its S decoded by gw_iq.h when staged, D per
//   super-block): Q6_K's term with v and S                                                            (iquants.h:49-55)
//   Q2_K (96 bytes: the file's 84 and padding; q 0 .. 3): Q6_K's term with the 4-bit scales sc, minus the mins' term
//     (dmin xs) M, M = m_0 X_0 + m_1 X_1 from the sums of x of each half (the same MFMA with B = 1)   (iquants.h:56-57)
// then val = val + term in group order. mode 1: out = out + val. K % 256 == 0.
template <int TYPE, int GM>
__global__ __launch_bounds__(256) void k_gemm_kq(const uint8_t *__restrict__ W, int bstride, int N, int K,
                                                 const int8_t *__restrict__ X, const float *__restrict__ XS, int ldx, int M,
                                                 float *out, int ldo, int mode) {
    constexpr int TJ = GM == 64 ? 2 : 1, XC = GM * 8 / 256;
    __shared__ __align__(16) int8_t xl[GM * GROW];
    __shared__ __align__(16) int8_t wl[GN * GROW];
    __shared__ __align__(16) float xsl[4][GM];
    __shared__ float f0l[GN][5], f1l[GN][5]; // Q4_K, Q5_K: d sc_j, dmin m_j of the stage's groups; Q6_K, Q3_K: f0l[n][0] = d
    __shared__ int scl[GN][9];               // Q6_K, Q3_K: the stage's 8 half-group scales (Q3_K: sc - 32)
    constexpr bool Q45 = TYPE == GW_Q4_K || TYPE == GW_Q5_K; // (else Q6_K, Q3_K: half-groups of 16)
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int m0 = blockIdx.y * GM, n0 = blockIdx.x * GN;
    const int wm = GM == 64 ? (wave >> 1) * 32 : 0, wn = GM == 64 ? (wave & 1) * 64 : wave * 32;
    const size_t rowb = (size_t)(K >> 8) * bstride;
    float acc[TJ][16];
    #pragma unroll
    for (int j = 0; j < TJ; j++)
        #pragma unroll
        for (int r = 0; r < 16; r++) acc[j][r] = 0.0f;
    // stage k0's loads into registers (the next stage's issued before this stage's MFMAs): X as in k_gemm_q8; W: Q4_K
    // 2 x 16 bytes of the stage's 64 bytes of nibbles per thread, Q6_K 4 units (row, group p, half h) of 16 bytes of
    // ql and 16 of qh; the headers (threads < 128: one row each). (xr0 / xr1 named: an array here was placed in
    // scratch memory)
    constexpr int NW = Q45 ? 2 : 4;
    uint4 xr0, xr1, wa[NW], wb[NW], hd0, hd1;
    IqRaw iqr[IqCb<TYPE>::iform ? NW : 1]; // (the i-quants: each unit's loads, decoded when staged)
    float xsv;
    auto load = [&](int k0) {
        const int hs = (k0 >> 7) & 1; // (the stage's half of super-block k0 / 256)
        const uint8_t *sbk = W + (size_t)(k0 >> 8) * bstride;
        auto xload = [&](int k) -> uint4 {
            int c = t + 256 * k, row = c >> 3, col = (c & 7) * 16, m = m0 + row < M ? m0 + row : M - 1;
            return *(const uint4 *)(X + (size_t)m * ldx + k0 + col);
        };
        xr0 = xload(0);
        xr1 = XC > 1 ? xload(1) : xr0;
        #pragma unroll
        for (int k = 0; k < NW; k++) {
            int c = t + 256 * k;
            if (TYPE == GW_Q4_K) {
                int row = c >> 2, q = c & 3, n = n0 + row < N ? n0 + row : N - 1;
                wa[k] = *(const uint4 *)(sbk + (size_t)n * rowb + 16 + 64 * hs + 16 * q);
            } else if (TYPE == GW_Q5_K) { // (the nibbles at +48; the 16 qh bytes of the piece's positions)
                int row = c >> 2, q = c & 3, n = n0 + row < N ? n0 + row : N - 1;
                wa[k] = *(const uint4 *)(sbk + (size_t)n * rowb + 48 + 64 * hs + 16 * q);
                wb[k] = *(const uint4 *)(sbk + (size_t)n * rowb + 16 + 16 * (q & 1));
            } else if (TYPE == GW_Q3_K) { // (unit (row, group p, half h): 16 bytes of qs and of hmask)
                int row = c >> 3, u = c & 7, h = u & 1, n = n0 + row < N ? n0 + row : N - 1;
                const uint8_t *b = sbk + (size_t)n * rowb;
                wa[k] = *(const uint4 *)(b + 32 + 32 * hs + 16 * h);
                wb[k] = *(const uint4 *)(b + 16 * h);
            } else if constexpr (IqCb<TYPE>::iform) { // (unit (row, group p, half h): its half-group's loads)
                int row = c >> 3, u = c & 7, p = u >> 1, h = u & 1, n = n0 + row < N ? n0 + row : N - 1;
                iqr[k] = iq_raw<TYPE>(sbk + (size_t)n * rowb, 8 * hs + 2 * p + h);
            } else if (TYPE == GW_Q2_K) { // (unit (row, group p, half h): sub-block 8 hs + 2 p + h, 16 bytes of qs)
                int row = c >> 3, u = c & 7, h = u & 1, n = n0 + row < N ? n0 + row : N - 1;
                wa[k] = *(const uint4 *)(sbk + (size_t)n * rowb + 16 + 32 * hs + 16 * h);
            } else {
                int row = c >> 3, u = c & 7, p = u >> 1, h = u & 1, n = n0 + row < N ? n0 + row : N - 1;
                const uint8_t *b = sbk + (size_t)n * rowb;
                wa[k] = *(const uint4 *)(b + 64 * hs + 32 * (p & 1) + 16 * h);
                wb[k] = *(const uint4 *)(b + 128 + 32 * hs + 16 * h);
            }
        }
        hd0 = make_uint4(0, 0, 0, 0), hd1 = make_uint4(0, 0, 0, 0);
        if (t < GN) {
            int n = n0 + t < N ? n0 + t : N - 1;
            const uint8_t *b = sbk + (size_t)n * rowb;
            if (Q45) {
                hd0 = *(const uint4 *)b; // d, dmin, then scale bytes 0 .. 11 in words y, z, w
            } else if (TYPE == GW_Q3_K) {
                hd0 = *(const uint4 *)(b + 96); // the 12 scale bytes, then d
            } else if constexpr (IqCb<TYPE>::iform) { // (the dwords of d)
                hd0.x = *(const uint32_t *)(b + iq_d_off<TYPE>());
                if (TYPE == GW_IQ1_M) hd0.y = *(const uint32_t *)(b + iq_d_off<TYPE>() + 4);
            } else if (TYPE == GW_Q2_K) {
                hd0 = *(const uint4 *)b;        // the 16 scale bytes (sc | m << 4)
                hd1 = *(const uint4 *)(b + 80); // d, dmin
            } else {
                hd0 = *(const uint4 *)(b + 192); // the 16 int8 scales
                hd1 = *(const uint4 *)(b + 208); // d
            }
        }
        xsv = 0.0f;
        int row = t >> 2, gg = t & 3, m = m0 + row < M ? m0 + row : M - 1;
        if (row < GM) xsv = XS[(size_t)m * (ldx >> 5) + (k0 >> 5) + gg];
    };
    load(0);
    for (int k0 = 0; k0 < K; k0 += GKB) {
        const int hs = (k0 >> 7) & 1;
        __syncthreads(); // (the previous stage's readers are done)
        *(uint4 *)(xl + (t >> 3) * GROW + (t & 7) * 16) = xr0;
        if (XC > 1) *(uint4 *)(xl + ((t + 256) >> 3) * GROW + ((t + 256) & 7) * 16) = xr1;
        #pragma unroll
        for (int k = 0; k < NW; k++) {
            int c = t + 256 * k;
            if (TYPE == GW_Q4_K) {
                // piece q: run i = q / 2 (32 bytes: low nibbles = group 2 i, high = group 2 i + 1), positions 16 (q % 2) ..
                int row = c >> 2, q = c & 3, i = q >> 1, o = 16 * (q & 1);
                uint4 lo = make_uint4(wa[k].x & 0x0F0F0F0Fu, wa[k].y & 0x0F0F0F0Fu, wa[k].z & 0x0F0F0F0Fu, wa[k].w & 0x0F0F0F0Fu);
                uint4 hi = make_uint4((wa[k].x >> 4) & 0x0F0F0F0Fu, (wa[k].y >> 4) & 0x0F0F0F0Fu, (wa[k].z >> 4) & 0x0F0F0F0Fu,
                                      (wa[k].w >> 4) & 0x0F0F0F0Fu);
                *(uint4 *)(wl + row * GROW + 32 * (2 * i) + o) = lo;
                *(uint4 *)(wl + row * GROW + 32 * (2 * i + 1) + o) = hi;
            } else if (TYPE == GW_Q5_K) { // (Q4_K's pieces with bit 4 of each code from qh: bit j of qh[l], j the sub-block)
                int row = c >> 2, q = c & 3, i = q >> 1, o = 16 * (q & 1), jl = 4 * hs + 2 * i;
                uint32_t a4[4] = { wa[k].x, wa[k].y, wa[k].z, wa[k].w }, b4[4] = { wb[k].x, wb[k].y, wb[k].z, wb[k].w }, lo[4], hi[4];
                #pragma unroll
                for (int e = 0; e < 4; e++) {
                    lo[e] = (a4[e] & 0x0F0F0F0Fu) | ((b4[e] >> jl) & 0x01010101u) << 4;
                    hi[e] = ((a4[e] >> 4) & 0x0F0F0F0Fu) | ((b4[e] >> (jl + 1)) & 0x01010101u) << 4;
                }
                *(uint4 *)(wl + row * GROW + 32 * (2 * i) + o) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
                *(uint4 *)(wl + row * GROW + 32 * (2 * i + 1) + o) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
            } else if (TYPE == GW_Q3_K) {
                // q' = ((qs >> 2 p) & 3) | (hmask bit 4 hs + p) << 2; q = q' - 4 as int8: q' with bit 2 flipped, sign-extended
                int row = c >> 3, u = c & 7, p = u >> 1, h = u & 1, hb = 4 * hs + p;
                uint32_t a4[4] = { wa[k].x, wa[k].y, wa[k].z, wa[k].w }, b4[4] = { wb[k].x, wb[k].y, wb[k].z, wb[k].w }, o4[4];
                #pragma unroll
                for (int e = 0; e < 4; e++) {
                    uint32_t q = ((a4[e] >> (2 * p)) & 0x03030303u) | ((b4[e] >> hb) & 0x01010101u) << 2;
                    uint32_t f = q ^ 0x04040404u, sg = f & 0x04040404u;
                    o4[e] = f | sg * 62u; // (bits 3 .. 7 of each byte whose bit 2 is set)
                }
                *(uint4 *)(wl + row * GROW + 32 * p + 16 * h) = make_uint4(o4[0], o4[1], o4[2], o4[3]);
            } else if constexpr (IqCb<TYPE>::iform) { // (the 16 values v as int8; the half-group's S)
                int row = c >> 3, u = c & 7, p = u >> 1, h = u & 1;
                int4 v;
                int S;
                iq_dec<TYPE>(iqr[k], 8 * hs + 2 * p + h, v, S);
                *(int4 *)(wl + row * GROW + 32 * p + 16 * h) = v;
                scl[row][2 * p + h] = S;
            } else if (TYPE == GW_Q2_K) { // q = 2 bits 2 p of each byte (0 .. 3)
                int row = c >> 3, u = c & 7, p = u >> 1, h = u & 1, sl = 2 * p;
                *(uint4 *)(wl + row * GROW + 32 * p + 16 * h) =
                    make_uint4((wa[k].x >> sl) & 0x03030303u, (wa[k].y >> sl) & 0x03030303u, (wa[k].z >> sl) & 0x03030303u,
                               (wa[k].w >> sl) & 0x03030303u);
            } else {
                // q = ((ql >> 4 (p / 2)) & 15) | ((qh >> 2 p) & 3) << 4; q - 32 as int8: the 6-bit value with bit 5
                // flipped, sign-extended
                int row = c >> 3, u = c & 7, p = u >> 1, h = u & 1, sl = 4 * (p >> 1), sh = 2 * p;
                uint32_t a4[4] = { wa[k].x, wa[k].y, wa[k].z, wa[k].w }, b4[4] = { wb[k].x, wb[k].y, wb[k].z, wb[k].w }, o4[4];
                #pragma unroll
                for (int e = 0; e < 4; e++) {
                    uint32_t q = ((a4[e] >> sl) & 0x0F0F0F0Fu) | (((b4[e] >> sh) & 0x03030303u) << 4);
                    uint32_t f = q ^ 0x20202020u, sg = f & 0x20202020u;
                    o4[e] = f | (sg << 1) | (sg << 2);
                }
                *(uint4 *)(wl + row * GROW + 32 * p + 16 * h) = make_uint4(o4[0], o4[1], o4[2], o4[3]);
            }
        }
        if (t < GN) {
            if (Q45) {
                auto scb = [&](int k) -> int { // (k < 12)
                    uint32_t w = k < 4 ? hd0.y : k < 8 ? hd0.z : hd0.w;
                    return (int)((w >> (8 * (k & 3))) & 0xffu);
                };
                const float d = h2f_g((uint16_t)(hd0.x & 0xffffu)), dmin = h2f_g((uint16_t)(hd0.x >> 16));
                #pragma unroll
                for (int gg = 0; gg < 4; gg++) {
                    const int sb = 4 * hs + gg;
                    int scj, mj;
                    if (sb < 4) {
                        scj = scb(sb) & 63;
                        mj = scb(sb + 4) & 63;
                    } else {
                        scj = (scb(sb + 4) & 15) | (scb(sb - 4) >> 6) << 4;
                        mj = (scb(sb + 4) >> 4) | (scb(sb) >> 6) << 4;
                    }
                    f0l[t][gg] = d * (float)scj;
                    f1l[t][gg] = dmin * (float)mj;
                }
            } else if (TYPE == GW_Q3_K) {
                // 6-bit sc_j = (s[j % 8] >> 4 (j / 8)) & 15 | ((s[8 + j % 4] >> 2 (j / 4)) & 3) << 4, j = 8 hs + k
                uint32_t sw[3] = { hd0.x, hd0.y, hd0.z };
                auto sbyte = [&](int i) -> uint32_t { return (sw[i >> 2] >> (8 * (i & 3))) & 0xffu; };
                #pragma unroll
                for (int k = 0; k < 8; k++) {
                    const int j = 8 * hs + k;
                    const uint32_t lo = (sbyte(j & 7) >> (4 * (j >> 3))) & 15u, hi = (sbyte(8 + (j & 3)) >> (2 * (j >> 2))) & 3u;
                    scl[t][k] = (int)(lo | hi << 4) - 32;
                }
                f0l[t][0] = h2f_g((uint16_t)(hd0.w & 0xffffu));
            } else if constexpr (IqCb<TYPE>::iform) { // (the S came with the units)
                f0l[t][0] = iq_d_raw<TYPE>(hd0.x, hd0.y);
            } else {
                uint32_t sw[4] = { hd0.x, hd0.y, hd0.z, hd0.w };
                #pragma unroll
                for (int k = 0; k < 8; k++) { // (half-group k of the stage: the super-block's scale 8 hs + k)
                    const int ks = 8 * hs + k;
                    scl[t][k] = (int)(int8_t)((sw[ks >> 2] >> (8 * (ks & 3))) & 0xffu);
                }
                f0l[t][0] = h2f_g((uint16_t)(hd1.x & 0xffffu));
                if (TYPE == GW_Q2_K) { // (scl: the raw byte sc | m << 4; f1l: dmin)
                    #pragma unroll
                    for (int k = 0; k < 8; k++) scl[t][k] = (int)(uint8_t)(sw[(8 * hs + k) >> 2] >> (8 * ((8 * hs + k) & 3)));
                    f1l[t][0] = h2f_g((uint16_t)(hd1.x >> 16));
                }
            }
        }
        {
            int row = t >> 2, gg = t & 3;
            if (row < GM) xsl[gg][row] = xsv;
        }
        __syncthreads();
        if (k0 + GKB < K) load(k0 + GKB);
        #pragma unroll
        for (int gg = 0; gg < 4; gg++) {
            const int8_t *xa = xl + (wm + (lane & 31)) * GROW + gg * 32;
            i32x16 S;
            i32x4 a;
            i64 a0, a1;
            const i32x16 z = { 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0 };
            if (Q45) {
                a = *(const i32x4 *)(xa + 16 * (lane >> 5));
                const i32x4 ones = { 0x01010101, 0x01010101, 0x01010101, 0x01010101 };
                S = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, ones, z, 0, 0, 0);
            } else {
                a0 = *(const i64 *)(xa + 8 * (lane >> 5));
                a1 = *(const i64 *)(xa + 16 + 8 * (lane >> 5));
            }
            i32x16 X0, X1; // Q2_K: the sums of x of the group's two halves (the same MFMA with B = 1)
            if (TYPE == GW_Q2_K) {
                const i64 ones = 0x0101010101010101l;
                X0 = __builtin_amdgcn_mfma_i32_32x32x16_i8(a0, ones, z, 0, 0, 0);
                X1 = __builtin_amdgcn_mfma_i32_32x32x16_i8(a1, ones, z, 0, 0, 0);
            }
            #pragma unroll
            for (int j = 0; j < TJ; j++) {
                const int nl = wn + 32 * j + (lane & 31);
                const int8_t *wbp = wl + nl * GROW + gg * 32;
                if (Q45) {
                    i32x4 b = *(const i32x4 *)(wbp + 16 * (lane >> 5));
                    i32x16 I = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, z, 0, 0, 0);
                    const float f0 = f0l[nl][gg], f1 = f1l[nl][gg];
                    #pragma unroll
                    for (int q = 0; q < 4; q++) {
                        float4 xs4 = *(const float4 *)(&xsl[gg][wm + 8 * q + 4 * (lane >> 5)]);
                        float xsq[4] = { xs4.x, xs4.y, xs4.z, xs4.w };
                        #pragma unroll
                        for (int e = 0; e < 4; e++) {
                            float pa = (f0 * xsq[e]) * (float)I[4 * q + e];
                            float pb = f1 * (xsq[e] * (float)S[4 * q + e]);
                            acc[j][4 * q + e] = acc[j][4 * q + e] + (pa - pb);
                        }
                    }
                } else {
                    i64 b0 = *(const i64 *)(wbp + 8 * (lane >> 5)), b1 = *(const i64 *)(wbp + 16 + 8 * (lane >> 5));
                    i32x16 I0 = __builtin_amdgcn_mfma_i32_32x32x16_i8(a0, b0, z, 0, 0, 0);
                    i32x16 I1 = __builtin_amdgcn_mfma_i32_32x32x16_i8(a1, b1, z, 0, 0, 0);
                    const int s0 = scl[nl][2 * gg], s1 = scl[nl][2 * gg + 1];
                    const float d = f0l[nl][0];
                    #pragma unroll
                    for (int q = 0; q < 4; q++) {
                        float4 xs4 = *(const float4 *)(&xsl[gg][wm + 8 * q + 4 * (lane >> 5)]);
                        float xsq[4] = { xs4.x, xs4.y, xs4.z, xs4.w };
                        #pragma unroll
                        for (int e = 0; e < 4; e++) {
                            if (TYPE == GW_Q2_K) { // (iquants.h:56-57: the mins' term beside the scales')
                                const int I = (s0 & 15) * I0[4 * q + e] + (s1 & 15) * I1[4 * q + e];
                                const int Mi = (s0 >> 4) * X0[4 * q + e] + (s1 >> 4) * X1[4 * q + e];
                                const float dm = f1l[nl][0];
                                acc[j][4 * q + e] = acc[j][4 * q + e] + ((d * xsq[e]) * (float)I - (dm * xsq[e]) * (float)Mi);
                            } else {
                                int I = s0 * I0[4 * q + e] + s1 * I1[4 * q + e];
                                acc[j][4 * q + e] = acc[j][4 * q + e] + (d * xsq[e]) * (float)I;
                            }
                        }
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
            if (m < M && n < N) {
                float *o = out + (size_t)m * ldo + n;
                *o = mode == 1 ? *o + acc[j][r] : acc[j][r];
            }
        }
    }
}

// K-quant GEMM for 9 .. 32 activation rows (batched decode): one block of 512 threads per 32 weight rows, the 8 waves
// taking the 8 groups of each super-block (wave w: group w), each wave's VALU work one group in eight. Per super-block s,
// the block stages the 32 rows' super-blocks and the activation rows' 256 codes and 8 scales in LDS (double-buffered),
// loaded with coalesced 16-byte loads (consecutive threads: consecutive 16 bytes of one row) SK_P super-blocks ahead;
// each wave reads its MFMA operands (X row l % 32, W row l % 32: k_gemm_kq's layouts) from LDS: the exact int32 sums
// (MFMA), the wave's terms (k_gemm_kq's expressions) into LDS, a barrier, then each thread adds the 8 terms of its 2
// outputs in group order (val = val + term, kquants.h:86-109, :410-554). A tile's 32 activation rows are 4 quads of
// 8 (the MFMA result's registers 4 q .. 4 q + 3 of every lane): a block takes NQR of them, the tile's 4 / NQR blocks
// on one XCD (blocks b and b + 8 k share b % 8), each staging the whole tile (the second reads hit that XCD's L2) and
// computing the terms and folds of its own quads only: a matrix of few rows fills the device with 4 / NQR times the
// blocks, each with 1 / (4 / NQR) of the VALU work. The terms go through one LDS buffer (a barrier before they are
// written, one after), so with 128 registers two blocks share a CU (double-buffered terms: 95 KB of LDS, one block per
// CU, 15 % slower). Two matrices of one type and width may share a launch (blocks below nb1 take the first, the
// others the second; each writes at its own column offset of out). M <= 32, K % 256 == 0, mode 1: out = out + val
#define SK_T 512
#define SK_P 4                      // super-blocks whose loads are in flight beyond the one computed
#define SK_XR 272                   // LDS bytes per activation row (256 codes + 16: rows 4 banks apart)
template <int TYPE>
struct SkStage { // one thread's share of a super-block's staging: a 16-byte piece of W and of X, an activation scale
    uint4 w, x;
    float xs;
};
struct SkMats { // the launch's matrices: blocks [0, nb1) the first, [nb1, grid) the second
    const uint8_t *W[2];
    int N[2], col[2], nb1;
};
template <int TYPE, int Q, typename CT>
__device__ __forceinline__ void kq32_terms(const i32x16 &I, const i32x16 &I1, const CT &C, int s0, int s1, int lane,
                                           float *Tq) {
    // quad Q's 4 terms of this lane (registers 4 Q + e: activation rows 8 Q + 4 hi + e) into Tq[e * 64 + lane]. C: the
    // outer-product MFMA's result, the same (row, column) per register as I: C[r] = f0 xs (the scale product of the
    // first term), Q4_K: C[16 + r] = f1 xf (the mins' term, xf = xs (float) sum x as kq_act_prep's, kquants.h:392-400)
    #pragma unroll
    for (int e = 0; e < 4; e++) {
        const int r = 4 * Q + e;
        float term;
        if constexpr (TYPE == GW_Q4_K) {
            float pa = C[r] * (float)I[r];
            term = pa - C[16 + r];
        } else { // (|s| <= 127, |I_h| < 2^17: the 24-bit multiplies are exact)
            int Ii = __mul24(s0, I[r]) + __mul24(s1, I1[r]);
            term = C[r] * (float)Ii;
        }
        Tq[e * 64 + lane] = term;
    }
}
template <int TYPE, int NQR, int SB>
__global__ __launch_bounds__(SK_T * SB, SB == 1 ? 2 : 1) void k_gemm_kq32(SkMats mats, int bstride, int K,
                                                                          const int8_t *__restrict__ X,
                                                                          const float *__restrict__ XS, int ldx, int M,
                                                                          float *out, int ldo, int mode) {
    constexpr int WST = TYPE == GW_Q4_K ? 160 : 240;            // LDS bytes per weight row (bstride + 16)
    constexpr int PW = TYPE == GW_Q4_K ? GW_Q4K_BYTES / 16 : GW_Q6K_DEV / 16; // 16-byte pieces per weight row
    constexpr int PARTS = 4 / NQR, NO = NQR * 256, NT = SK_T * SB; // blocks per tile, outputs per block, threads
    __shared__ __align__(16) float Tl[8 * SB][NO];              // term of group g of super-block b (row 8 b + g)
    __shared__ __align__(16) uint8_t Ws[2][SB][32 * WST];
    __shared__ __align__(16) uint8_t Xs[2][SB][32 * SK_XR];
    __shared__ __align__(16) float xsl[2][SB][8][32];           // [super-block][group][m]
    // wave wv: group w = wv % 8 of super-block sb = wv / 8 of the step; thread t stages super-block ts = t / SK_T
    const int t = threadIdx.x, lane = t & 63, wv = t >> 6, w = wv & 7, sb = wv >> 3, hi = lane >> 5, r32 = lane & 31;
    const int tt = t & (SK_T - 1), ts = t / SK_T;
    const int mi = blockIdx.x >= mats.nb1;
    // block b of its matrix: XCD b % 8, then (b / 8) % PARTS its quads, tile 8 (b / 8 / PARTS) + b % 8
    const int bl = blockIdx.x - (mi ? mats.nb1 : 0), part = (bl >> 3) % PARTS, q0 = part * NQR;
    const int n0 = (((bl >> 3) / PARTS) * 8 + (bl & 7)) * 32, N = mats.N[mi], S = K >> 8;
    if (n0 >= N || 8 * q0 >= M) return; // (the grid's padding to 8 tiles; quads past the last activation row)
    const int S2 = (S + SB - 1) / SB; // (steps of SB super-blocks)
    const size_t rowb = (size_t)S * bstride;
    out += mats.col[mi];
    // this thread's staging pieces of super-block ts of a step: W row tt / PW piece tt % PW (tt < 32 PW), X row tt / 16
    // piece tt % 16, XS (tt < 256); every thread loads (the others a piece of row 31 again, never staged), so no load
    // sits under a branch
    const int wr = tt / PW < 32 ? tt / PW : 31, wp = tt % PW, wn = n0 + wr < N ? n0 + wr : N - 1;
    const uint8_t *wsrc = mats.W[mi] + (size_t)wn * rowb + 16 * wp;
    const int xr = tt >> 4, xm = xr < M ? xr : M - 1;
    const int8_t *xsrc = X + (size_t)xm * ldx + 16 * (tt & 15);
    const int sm = (tt >> 3) < M ? (tt >> 3) : M - 1;
    const float *xssrc = XS + (size_t)sm * (ldx >> 5) + (tt & 7);
    auto load = [&](int s) __attribute__((always_inline)) -> SkStage<TYPE> {
        int b = s * SB + ts;
        b = b < S ? b : S - 1; // (past the last super-block: the last again)
        SkStage<TYPE> o; // (32-bit offsets: a 64-bit multiply per load was a quarter-rate v_mad_u64_u32)
        o.w = *(const uint4 *)(wsrc + (uint32_t)(b * bstride));
        o.x = *(const uint4 *)(xsrc + (uint32_t)(256 * b));
        o.xs = xssrc[(uint32_t)(8 * b)];
        return o;
    };
    auto stage = [&](const SkStage<TYPE> &o, int buf) __attribute__((always_inline)) {
        if (tt < 32 * PW) *(uint4 *)(&Ws[buf][ts][wr * WST + 16 * wp]) = o.w;
        *(uint4 *)(&Xs[buf][ts][xr * SK_XR + 16 * (tt & 15)]) = o.x;
        if (tt < 256) xsl[buf][ts][tt & 7][tt >> 3] = o.xs;
    };
    float acc0 = 0.0f, acc1 = 0.0f; // outputs t and t + NT
    const i32x16 z = { 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0 };
    const uint8_t *wrow_l = &Ws[0][sb][r32 * WST], *xrow_l = &Xs[0][sb][r32 * SK_XR + 32 * w];
    auto step = [&](const SkStage<TYPE> nx, int s) __attribute__((always_inline)) -> SkStage<TYPE> {
        // step s (super-blocks SB s ..): nx holds step s + 1's pieces: staged into the other buffer (its readers, step
        // s - 1, are past the barriers of step s - 1); returned: the set reloaded with step s + 1 + SK_P (values, not
        // references: a set passed by reference was placed in memory)
        const int buf = s & 1;
        if (s + 1 < S2) stage(nx, buf ^ 1);
        const SkStage<TYPE> nl = load(s + 1 + SK_P);
        if (s >= S2) return nl; // (the last group of four steps past the end: its loads only, uniform)
        const uint8_t *wb = wrow_l + buf * (SB * 32 * WST), *xb = xrow_l + buf * (SB * 32 * SK_XR);
        float f0, f1 = 0.0f;
        int s0 = 0, s1 = 0, sxs = 0;
        i32x16 I, I1 = z;
        if constexpr (TYPE == GW_Q4_K) {
            const uint4 xq = *(const uint4 *)(xb + 16 * hi);
            const uint4 q = *(const uint4 *)(wb + 16 + 32 * (w >> 1) + 16 * hi);
            const uint4 hd = *(const uint4 *)wb;
            const int sh = 4 * (w & 1);
            const i32x4 bq = { (int)((q.x >> sh) & 0x0F0F0F0Fu), (int)((q.y >> sh) & 0x0F0F0F0Fu),
                               (int)((q.z >> sh) & 0x0F0F0F0Fu), (int)((q.w >> sh) & 0x0F0F0F0Fu) };
            const i32x4 a = { (int)xq.x, (int)xq.y, (int)xq.z, (int)xq.w };
            I = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, bq, z, 0, 0, 0);
            // the sum of x of activation row r32 (its two halves of 16 in lanes l and l ^ 32)
            int sx = __builtin_amdgcn_sdot4((int)xq.x, 0x01010101, 0, false);
            sx = __builtin_amdgcn_sdot4((int)xq.y, 0x01010101, sx, false);
            sx = __builtin_amdgcn_sdot4((int)xq.z, 0x01010101, sx, false);
            sx = __builtin_amdgcn_sdot4((int)xq.w, 0x01010101, sx, false);
            sxs = sx + __shfl_xor(sx, 32);
            // the scale bytes k = w, w + 4 and w - 4 (the 12 bytes in words y, z, w of the header)
            const int bs = 8 * (w & 3);
            const int bw = (int)(((w < 4 ? hd.y : hd.z) >> bs) & 0xffu), bw4 = (int)(((w < 4 ? hd.z : hd.w) >> bs) & 0xffu);
            const int bm4 = (int)((hd.y >> bs) & 0xffu);
            int scj, mj;
            if (w < 4) {
                scj = bw & 63;
                mj = bw4 & 63;
            } else {
                scj = (bw4 & 15) | (bm4 >> 6) << 4;
                mj = (bw4 >> 4) | (bw >> 6) << 4;
            }
            f0 = h2f_g((uint16_t)(hd.x & 0xffffu)) * (float)scj;
            f1 = h2f_g((uint16_t)(hd.x >> 16)) * (float)mj;
        } else {
            const int nn = w >> 2, p = w & 3, sl = 4 * (p >> 1), sh = 2 * p;
            const uint2 x0 = *(const uint2 *)(xb + 8 * hi), x1 = *(const uint2 *)(xb + 16 + 8 * hi);
            const uint2 l0 = *(const uint2 *)(wb + 64 * nn + 32 * (p & 1) + 8 * hi);
            const uint2 l1 = *(const uint2 *)(wb + 64 * nn + 32 * (p & 1) + 16 + 8 * hi);
            const uint2 h0 = *(const uint2 *)(wb + 128 + 32 * nn + 8 * hi), h1 = *(const uint2 *)(wb + 128 + 32 * nn + 16 + 8 * hi);
            const uint32_t sc = *(const uint32_t *)(wb + 192 + 4 * (w >> 1)), dw = *(const uint32_t *)(wb + 208);
            auto code = [&](uint32_t lo, uint32_t hq) -> int { // 4 codes q - 32 (q = lo nibble | 2 bits of qh << 4)
                uint32_t q = ((lo >> sl) & 0x0F0F0F0Fu) | (((hq >> sh) & 0x03030303u) << 4);
                uint32_t f = q ^ 0x20202020u, sg = f & 0x20202020u;
                return (int)(f | (sg << 1) | (sg << 2));
            };
            const i64 b0 = (i64)(uint32_t)code(l0.x, h0.x) | (i64)(uint32_t)code(l0.y, h0.y) << 32;
            const i64 b1 = (i64)(uint32_t)code(l1.x, h1.x) | (i64)(uint32_t)code(l1.y, h1.y) << 32;
            const i64 a0 = (i64)x0.x | (i64)x0.y << 32, a1 = (i64)x1.x | (i64)x1.y << 32;
            I = __builtin_amdgcn_mfma_i32_32x32x16_i8(a0, b0, z, 0, 0, 0);
            I1 = __builtin_amdgcn_mfma_i32_32x32x16_i8(a1, b1, z, 0, 0, 0);
            const uint32_t sc2 = sc >> (16 * (w & 1)); // (scales 2 w, 2 w + 1)
            s0 = (int)(int8_t)(sc2 & 0xffu);
            s1 = (int)(int8_t)((sc2 >> 8) & 0xffu);
            f0 = h2f_g((uint16_t)(dw & 0xffffu));
        }
        // the scale products as an outer-product MFMA (each product one fp32 rounding, as the VALU's multiply): lanes
        // 0 .. 31 xs of activation row r32 and f0 of weight row r32; Q4_K: two blocks, lanes 32 .. 63 the row's
        // xf = xs (float) sum x and f1; Q6_K: one block of K = 2, lanes 32 .. 63 (k = 1) zero (x y + 0 0 = x y)
        const float xsr = xsl[buf][sb][w][r32];
        const float ca = hi ? (TYPE == GW_Q4_K ? xsr * (float)sxs : 0.0f) : xsr, cb = hi ? (TYPE == GW_Q4_K ? f1 : 0.0f) : f0;
        using CT = typename std::conditional<TYPE == GW_Q4_K, f32x32, f32x16>::type;
        CT C;
        if constexpr (TYPE == GW_Q4_K) {
            const f32x32 zf = {};
            C = __builtin_amdgcn_mfma_f32_32x32x1f32(ca, cb, zf, 0, 0, 0);
        } else {
            const f32x16 zf = {};
            C = __builtin_amdgcn_mfma_f32_32x32x2f32(ca, cb, zf, 0, 0, 0);
        }
        // this block's quads (uniform branches: a register index must be a constant)
        float *Tw = &Tl[wv][0];
        __syncthreads(); // (every wave's fold of the previous step has read the terms)
        if (NQR == 4) {
            kq32_terms<TYPE, 0, CT>(I, I1, C, s0, s1, lane, Tw);
            kq32_terms<TYPE, 1, CT>(I, I1, C, s0, s1, lane, Tw + 256);
            kq32_terms<TYPE, 2, CT>(I, I1, C, s0, s1, lane, Tw + 512);
            kq32_terms<TYPE, 3, CT>(I, I1, C, s0, s1, lane, Tw + 768);
        } else if (NQR == 2) {
            if (q0 == 0) {
                kq32_terms<TYPE, 0, CT>(I, I1, C, s0, s1, lane, Tw);
                kq32_terms<TYPE, 1, CT>(I, I1, C, s0, s1, lane, Tw + 256);
            } else {
                kq32_terms<TYPE, 2, CT>(I, I1, C, s0, s1, lane, Tw);
                kq32_terms<TYPE, 3, CT>(I, I1, C, s0, s1, lane, Tw + 256);
            }
        } else {
            if (q0 == 0) kq32_terms<TYPE, 0, CT>(I, I1, C, s0, s1, lane, Tw);
            else if (q0 == 1) kq32_terms<TYPE, 1, CT>(I, I1, C, s0, s1, lane, Tw);
            else if (q0 == 2) kq32_terms<TYPE, 2, CT>(I, I1, C, s0, s1, lane, Tw);
            else kq32_terms<TYPE, 3, CT>(I, I1, C, s0, s1, lane, Tw);
        }
        __syncthreads(); // (the terms of step s written; step s + 1 staged)
        const int ng = 8 * (S - s * SB < SB ? S - s * SB : SB); // (a last step past K: its terms not added)
        if (t < NO) {
            #pragma unroll
            for (int g = 0; g < 8 * SB; g++)
                if (g < ng) acc0 = acc0 + Tl[g][t];
        }
        if (NO > NT) {
            #pragma unroll
            for (int g = 0; g < 8 * SB; g++)
                if (g < ng) acc1 = acc1 + Tl[g][t + NT];
        }
        return nl;
    };
    // four register sets take turns (super-block s + 1 + k in set (s + 1 + k) % 4; named: an array of them was placed
    // in scratch memory): super-block 0 staged, set 0 reloaded with 4, then step s stages s + 1 and reloads with s + 5
    static_assert(SK_P == 4, "four register sets");
    SkStage<TYPE> o0 = load(0), o1 = load(1), o2 = load(2), o3 = load(3);
    stage(o0, 0);
    o0 = load(4);
    __syncthreads();
    // (one exit, at the end of each group of four: a break after each step made the compiler wait for every load in
    // flight at the top of the loop)
    for (int s0 = 0; s0 < S2; s0 += 4) {
        o1 = step(o1, s0);
        o2 = step(o2, s0 + 1);
        o3 = step(o3, s0 + 2);
        o0 = step(o0, s0 + 3);
    }
    #pragma unroll
    for (int k = 0; k < (NO + NT - 1) / NT; k++) {
        const int o = t + NT * k, r = (o >> 6) + 4 * q0, ln = o & 63;
        const int m = 8 * (r >> 2) + 4 * (ln >> 5) + (r & 3), n = n0 + (ln & 31);
        if (o < NO && m < M && n < N) {
            float *po = out + (size_t)m * ldo + n;
            const float v = k ? acc1 : acc0;
            *po = mode == 1 ? *po + v : v;
        }
    }
}

// --------------------------------------------------------------------------------------------- K-quants

// The batched GEMV of every weight format: out[m * ldo + row] (+)= W row . X row m for M <= 8 activation rows, R weight
// rows per block. Each thread takes half-groups (16 weights) j = t, t + 256, ..., U per pass (the launcher uses U = 1),
// with every load of the pass issued before the first dot; the 16 weights become 16 int8 codes in four 32-bit words, the exact int32 sums by
// 4 v_dot4 per (row, activation row), and the group's term (the even lane of the pair) goes into LDS:
//   Q8_0 (codes row-major, fp16 scales): (ws * xs) * (float) isum                                   (forward.c:906-916)
//   Q4_K (144-byte super-blocks of 256: d, dmin, 12 bytes of 6-bit scales / mins, 128 of nibbles):
//     a - b, a = ((d * sc_j) * xs) * (float) isum, b = (dmin * m_j) * (xs * (float) sum x)            (kquants.h:86-109)
//   Q6_K (224-byte super-blocks: the file's 210 bytes, 16-byte aligned: ql 128, qh 64, 16 int8 scales, fp16 d):
//     (d * xs) * (float) (sc_0 (sum q x - 32 sum x) + sc_1 (...)), over the group's two halves of 16
//   Q5_K (176 bytes: Q4_K's header, qh 32, nibbles 128): Q4_K's term with q 0 .. 31 (bit 4 from qh)
//   Q3_K (112 bytes: hmask 32, qs 64, 12 bytes of 6-bit scales, fp16 d, 2 of padding): Q6_K's term with q' 0 .. 7
//     (2 bits from qs, bit 2 from hmask), - 4 sum x and the scales sc - 32
//   the i-quants (IQ4_XS and the codebook types, their integer form w = D S v read by gw_iq.h: a half-group's 16 v and
//     its S decoded from the super-block, D): (D * xs) * (float) (S_0 sum v x + S_1 (...)) over the group's two halves
//     of 16                                                                                            (iquants.h:49-55)
//   Q2_K (96 bytes: 16 scale bytes sc | m << 4, qs 64, fp16 d, dmin, padding; q 0 .. 3): (d * xs) * (float) (sc_0 sum q x
//     + sc_1 (...)) - (dmin * xs) * (float) (m_0 sum x + m_1 (...))                                  (iquants.h:49-57)
// then one lane per (activation row, weight row) folds the groups in order: val = val + term. mode 1: out = out + val.
// K % 32 == 0 (Q8_0), % 256 (K-quants); the K-quants' q are 0 .. 63, so v_dot4 with signed codes is exact
template <int TYPE, int M, int R, int U, bool PF>
__global__ __launch_bounds__(256) void k_gemv_mr(const uint8_t *__restrict__ W, const uint16_t *__restrict__ WS, int nrows,
                                                 int K, int bstride, const int8_t *__restrict__ xq, const float *__restrict__ xs,
                                                 int ldx, float *out, int ldo, int mode) {
    extern __shared__ float P[];
    // (P: the terms of the row, or with PF of one pass (128 U groups), folded after each pass with the running value
    // in the fold lane: rows of several passes (K = 12288) no longer held to three blocks per CU by a whole row's
    // terms. A separate instance: the fold inside the pass loop keeps 106 registers, the row's fold after it 70, and
    // the one-pass matrices run seven blocks per CU on 70; rows 16-byte aligned)
    constexpr int GPASS = PF ? 128 * U : 1 << 30;
    const int G = K >> 5, H = K >> 4, PS = ((G < GPASS ? G : GPASS) + 7) & ~3;
    const int row0 = blockIdx.x * R, t = threadIdx.x;
    float vf = 0.0f; // (fold lane t < M R: the value of activation row t / R, weight row t % R so far)
    // v + the terms p[0 .. ng - 1] in order (sets of 32 terms' LDS reads alternating)
    auto fold_terms = [&](const float *p, int ng, float v) __attribute__((always_inline)) -> float {
        int g = 0;
        if (ng >= 32) {
            float4 a[8], b[8];
            #pragma unroll
            for (int u = 0; u < 8; u++) a[u] = *(const float4 *)(p + 4 * u);
            for (g = 32; g + 64 <= ng; g += 64) {
                #pragma unroll
                for (int u = 0; u < 8; u++) b[u] = *(const float4 *)(p + g + 4 * u);
                #pragma unroll
                for (int u = 0; u < 8; u++) {
                    v = v + a[u].x;
                    v = v + a[u].y;
                    v = v + a[u].z;
                    v = v + a[u].w;
                }
                #pragma unroll
                for (int u = 0; u < 8; u++) a[u] = *(const float4 *)(p + g + 32 + 4 * u);
                #pragma unroll
                for (int u = 0; u < 8; u++) {
                    v = v + b[u].x;
                    v = v + b[u].y;
                    v = v + b[u].z;
                    v = v + b[u].w;
                }
            }
            // (a holds groups g - 32 .. g - 1)
            #pragma unroll
            for (int u = 0; u < 8; u++) {
                v = v + a[u].x;
                v = v + a[u].y;
                v = v + a[u].z;
                v = v + a[u].w;
            }
        }
        for (; g < ng; g++) v = v + p[g];
        return v;
    };
    const size_t rowb = TYPE == GW_Q8_0 ? (size_t)K : (size_t)(K >> 8) * bstride;
    for (int j0 = 0; j0 < H; j0 += 256 * U) {
        // the pass's loads (past the row's end: its last half-group again, unconditionally; only the stores below are
        // predicated, so no load waits for a branch)
        int4 wv[U][R];
        float f0[U][R], f1[U][R]; // Q8_0: ws; Q4_K, Q5_K: d sc_j, dmin m_j; Q6_K, Q3_K: d
        int isc[U][R];            // Q6_K: the half-group's int8 scale; Q3_K: its scale - 32
        #pragma unroll
        for (int u = 0; u < U; u++) {
            const int j = j0 + 256 * u + t < H ? j0 + 256 * u + t : H - 1;
            #pragma unroll
            for (int r = 0; r < R; r++) {
                const int row = row0 + r < nrows ? row0 + r : nrows - 1;
                const uint8_t *rb = W + (size_t)row * rowb;
                if (TYPE == GW_Q8_0) {
                    wv[u][r] = *(const int4 *)(rb + 16 * j);
                } else {
                    const int sblk = j >> 4, sb = (j >> 1) & 7, h = j & 1;
                    const uint8_t *b = rb + (size_t)sblk * bstride;
                    if (TYPE == GW_Q4_K) { // (sub-block sb: the low nibbles of its byte pair's run for even sb, high for odd)
                        const int4 q = *(const int4 *)(b + 16 + 32 * (sb >> 1) + 16 * h);
                        const int sl = 4 * (sb & 1);
                        wv[u][r].x = (int)(((uint32_t)q.x >> sl) & 0x0F0F0F0Fu);
                        wv[u][r].y = (int)(((uint32_t)q.y >> sl) & 0x0F0F0F0Fu);
                        wv[u][r].z = (int)(((uint32_t)q.z >> sl) & 0x0F0F0F0Fu);
                        wv[u][r].w = (int)(((uint32_t)q.w >> sl) & 0x0F0F0F0Fu);
                    } else if (TYPE == GW_Q5_K) { // (Q4_K's nibbles at +48, and bit sb of qh[l] as bit 4)
                        const int4 q = *(const int4 *)(b + 48 + 32 * (sb >> 1) + 16 * h);
                        const int4 qh = *(const int4 *)(b + 16 + 16 * h);
                        const int sl = 4 * (sb & 1);
                        wv[u][r].x = (int)((((uint32_t)q.x >> sl) & 0x0F0F0F0Fu) | ((((uint32_t)qh.x >> sb) & 0x01010101u) << 4));
                        wv[u][r].y = (int)((((uint32_t)q.y >> sl) & 0x0F0F0F0Fu) | ((((uint32_t)qh.y >> sb) & 0x01010101u) << 4));
                        wv[u][r].z = (int)((((uint32_t)q.z >> sl) & 0x0F0F0F0Fu) | ((((uint32_t)qh.z >> sb) & 0x01010101u) << 4));
                        wv[u][r].w = (int)((((uint32_t)q.w >> sl) & 0x0F0F0F0Fu) | ((((uint32_t)qh.w >> sb) & 0x01010101u) << 4));
                    } else if (TYPE == GW_Q3_K) { // (values 32 sb + 16 h ..: 2 bits 2 (sb % 4) of qs[32 (sb / 4) + l], hmask bit sb)
                        const int4 q = *(const int4 *)(b + 32 + 32 * (sb >> 2) + 16 * h);
                        const int4 hm = *(const int4 *)(b + 16 * h);
                        const int sl = 2 * (sb & 3);
                        wv[u][r].x = (int)((((uint32_t)q.x >> sl) & 0x03030303u) | ((((uint32_t)hm.x >> sb) & 0x01010101u) << 2));
                        wv[u][r].y = (int)((((uint32_t)q.y >> sl) & 0x03030303u) | ((((uint32_t)hm.y >> sb) & 0x01010101u) << 2));
                        wv[u][r].z = (int)((((uint32_t)q.z >> sl) & 0x03030303u) | ((((uint32_t)hm.z >> sb) & 0x01010101u) << 2));
                        wv[u][r].w = (int)((((uint32_t)q.w >> sl) & 0x03030303u) | ((((uint32_t)hm.w >> sb) & 0x01010101u) << 2));
                    } else if constexpr (IqCb<TYPE>::iform) { // (the i-quants: the half-group's 16 values v, its S)
                        iq_half<TYPE>(b, j & 15, wv[u][r], isc[u][r]);
                    } else if (TYPE == GW_Q2_K) { // (sub-block k = j % 16: 16 bytes of qs at 32 (k / 8) + 16 (k % 2), 2 bits 2 ((k / 2) % 4))
                        const int k = j & 15, sl = 2 * ((k >> 1) & 3);
                        const int4 q = *(const int4 *)(b + 16 + 32 * (k >> 3) + 16 * (k & 1));
                        wv[u][r].x = (int)(((uint32_t)q.x >> sl) & 0x03030303u);
                        wv[u][r].y = (int)(((uint32_t)q.y >> sl) & 0x03030303u);
                        wv[u][r].z = (int)(((uint32_t)q.z >> sl) & 0x03030303u);
                        wv[u][r].w = (int)(((uint32_t)q.w >> sl) & 0x03030303u);
                    } else {
                        const int n = sb >> 2, p = sb & 3;
                        int4 lo = *(const int4 *)(b + 64 * n + 32 * (p & 1) + 16 * h);
                        int4 hi = *(const int4 *)(b + 128 + 32 * n + 16 * h);
                        const int sl = 4 * (p >> 1), sh = 2 * p;
                        wv[u][r].x = (int)((((uint32_t)lo.x >> sl) & 0x0F0F0F0Fu) | ((((uint32_t)hi.x >> sh) & 0x03030303u) << 4));
                        wv[u][r].y = (int)((((uint32_t)lo.y >> sl) & 0x0F0F0F0Fu) | ((((uint32_t)hi.y >> sh) & 0x03030303u) << 4));
                        wv[u][r].z = (int)((((uint32_t)lo.z >> sl) & 0x0F0F0F0Fu) | ((((uint32_t)hi.z >> sh) & 0x03030303u) << 4));
                        wv[u][r].w = (int)((((uint32_t)lo.w >> sl) & 0x0F0F0F0Fu) | ((((uint32_t)hi.w >> sh) & 0x03030303u) << 4));
                    }
                }
            }
        }
        #pragma unroll
        for (int u = 0; u < U; u++) {
            const int j = j0 + 256 * u + t < H ? j0 + 256 * u + t : H - 1;
            #pragma unroll
            for (int r = 0; r < R; r++) {
                const int row = row0 + r < nrows ? row0 + r : nrows - 1;
                const uint8_t *rb = W + (size_t)row * rowb;
                if (TYPE == GW_Q8_0) {
                    f0[u][r] = h2f_g(WS[(size_t)row * G + (j >> 1)]);
                    f1[u][r] = 0.0f;
                    isc[u][r] = 0;
                } else if (TYPE == GW_Q4_K || TYPE == GW_Q5_K) {
                    const int sblk = j >> 4, sb = (j >> 1) & 7;
                    const uint8_t *b = rb + (size_t)sblk * bstride;
                    const uint4 hd = *(const uint4 *)b; // d, dmin, then scale bytes 0 .. 11 in words y, z, w
                    auto scb = [&](int k) -> int { // (k < 12)
                        uint32_t w = k < 4 ? hd.y : k < 8 ? hd.z : hd.w;
                        return (int)((w >> (8 * (k & 3))) & 0xffu);
                    };
                    int scj, mj;
                    if (sb < 4) {
                        scj = scb(sb) & 63;
                        mj = scb(sb + 4) & 63;
                    } else {
                        scj = (scb(sb + 4) & 15) | (scb(sb - 4) >> 6) << 4;
                        mj = (scb(sb + 4) >> 4) | (scb(sb) >> 6) << 4;
                    }
                    f0[u][r] = h2f_g((uint16_t)(hd.x & 0xffffu)) * (float)scj;
                    f1[u][r] = h2f_g((uint16_t)(hd.x >> 16)) * (float)mj;
                    isc[u][r] = 0;
                } else if (TYPE == GW_Q2_K) { // (isc: the raw scale byte sc | m << 4; f0 d, f1 dmin)
                    const int sblk = j >> 4, k = j & 15;
                    const uint8_t *b = rb + (size_t)sblk * bstride;
                    const uint4 sw = *(const uint4 *)b;
                    uint32_t w = k < 4 ? sw.x : k < 8 ? sw.y : k < 12 ? sw.z : sw.w;
                    isc[u][r] = (int)((w >> (8 * (k & 3))) & 0xffu);
                    const uint32_t dw = (*(const uint4 *)(b + 80)).x;
                    f0[u][r] = h2f_g((uint16_t)(dw & 0xffffu));
                    f1[u][r] = h2f_g((uint16_t)(dw >> 16));
                } else if constexpr (IqCb<TYPE>::iform) { // (S came with the values; D of the super-block)
                    f0[u][r] = iq_d<TYPE>(rb + (size_t)(j >> 4) * bstride);
                    f1[u][r] = 0.0f;
                } else if (TYPE == GW_Q6_K) {
                    const int sblk = j >> 4, k = j & 15;
                    const uint8_t *b = rb + (size_t)sblk * bstride;
                    const uint4 sw = *(const uint4 *)(b + 192); // the 16 int8 scales
                    uint32_t w = k < 4 ? sw.x : k < 8 ? sw.y : k < 12 ? sw.z : sw.w;
                    isc[u][r] = (int)(int8_t)((w >> (8 * (k & 3))) & 0xffu);
                    const uint32_t dw = (*(const uint4 *)(b + 208)).x;
                    f0[u][r] = h2f_g((uint16_t)dw);
                    f1[u][r] = 0.0f;
                } else { // Q3_K (the 12 scale bytes s and d: 6-bit sc_k = low 4 bits of s[k % 8] (k / 8: high nibble) |
                         // bits 2 (k / 4) of s[8 + k % 4] << 4)
                    const int sblk = j >> 4, k = j & 15;
                    const uint8_t *b = rb + (size_t)sblk * bstride;
                    const uint4 sw = *(const uint4 *)(b + 96);
                    auto sbyte = [&](int i) -> uint32_t { // (i < 12)
                        uint32_t w = i < 4 ? sw.x : i < 8 ? sw.y : sw.z;
                        return (w >> (8 * (i & 3))) & 0xffu;
                    };
                    const uint32_t lo = (sbyte(k & 7) >> (4 * (k >> 3))) & 15u, hi = (sbyte(8 + (k & 3)) >> (2 * (k >> 2))) & 3u;
                    isc[u][r] = (int)(lo | hi << 4) - 32;
                    f0[u][r] = h2f_g((uint16_t)(sw.w & 0xffffu));
                    f1[u][r] = 0.0f;
                }
            }
        }
        int4 xv[U][M];
        float xsg[U][M];
        #pragma unroll
        for (int u = 0; u < U; u++) {
            const int j = j0 + 256 * u + t < H ? j0 + 256 * u + t : H - 1;
            #pragma unroll
            for (int m = 0; m < M; m++) {
                xv[u][m] = *(const int4 *)(xq + (size_t)m * ldx + 16 * j);
                xsg[u][m] = xs[(size_t)m * (ldx >> 5) + (j >> 1)];
            }
        }
        #pragma unroll
        for (int u = 0; u < U; u++) {
            const int j = j0 + 256 * u + t;
            if (j < H) { // (whole lane pairs: H is even)
                #pragma unroll
                for (int m = 0; m < M; m++) {
                    int xsum = 0; // K-quants: the sum of the half-group's activation codes
                    if (TYPE != GW_Q8_0 && !IqCb<TYPE>::iform) {
                        xsum = __builtin_amdgcn_sdot4(xv[u][m].x, 0x01010101, 0, false);
                        xsum = __builtin_amdgcn_sdot4(xv[u][m].y, 0x01010101, xsum, false);
                        xsum = __builtin_amdgcn_sdot4(xv[u][m].z, 0x01010101, xsum, false);
                        xsum = __builtin_amdgcn_sdot4(xv[u][m].w, 0x01010101, xsum, false);
                    }
                    const int xsum2 = TYPE == GW_Q4_K || TYPE == GW_Q5_K ? xsum + __shfl_xor(xsum, 1) : 0;
                    #pragma unroll
                    for (int r = 0; r < R; r++) {
                        int sd = __builtin_amdgcn_sdot4(wv[u][r].x, xv[u][m].x, 0, false);
                        sd = __builtin_amdgcn_sdot4(wv[u][r].y, xv[u][m].y, sd, false);
                        sd = __builtin_amdgcn_sdot4(wv[u][r].z, xv[u][m].z, sd, false);
                        sd = __builtin_amdgcn_sdot4(wv[u][r].w, xv[u][m].w, sd, false);
                        float term;
                        if (TYPE == GW_Q8_0) {
                            int is = sd + __shfl_xor(sd, 1);
                            float sc = f0[u][r] * xsg[u][m];
                            term = sc * (float)is;
                        } else if (TYPE == GW_Q4_K || TYPE == GW_Q5_K) {
                            int is = sd + __shfl_xor(sd, 1);
                            float a = (f0[u][r] * xsg[u][m]) * (float)is;
                            float bb = f1[u][r] * (xsg[u][m] * (float)xsum2);
                            term = a - bb;
                        } else if (TYPE == GW_Q3_K) {
                            int I = isc[u][r] * (sd - 4 * xsum);
                            I = I + __shfl_xor(I, 1);
                            term = (f0[u][r] * xsg[u][m]) * (float)I;
                        } else if (TYPE == GW_Q2_K) { // (I = sc_0 T_0 + sc_1 T_1, M = m_0 X_0 + m_1 X_1, iquants.h:49-57)
                            int I = (isc[u][r] & 15) * sd, Mi = (isc[u][r] >> 4) * xsum;
                            I = I + __shfl_xor(I, 1);
                            Mi = Mi + __shfl_xor(Mi, 1);
                            term = (f0[u][r] * xsg[u][m]) * (float)I - (f1[u][r] * xsg[u][m]) * (float)Mi;
                        } else if (IqCb<TYPE>::iform) { // (I = S_0 T_0 + S_1 T_1, iquants.h:49-55)
                            int I = isc[u][r] * sd;
                            I = I + __shfl_xor(I, 1);
                            term = (f0[u][r] * xsg[u][m]) * (float)I;
                        } else {
                            int I = isc[u][r] * (sd - 32 * xsum);
                            I = I + __shfl_xor(I, 1);
                            term = (f0[u][r] * xsg[u][m]) * (float)I;
                        }
                        if (!(j & 1)) P[(m * R + r) * PS + ((j - (PF ? j0 : 0)) >> 1)] = term;
                    }
                }
            }
        }
        if constexpr (PF) { // this pass's groups j0 / 2 .. into the fold lanes' values
            __syncthreads();
            if (t < M * R) vf = fold_terms(P + t * PS, G - (j0 >> 1) < GPASS ? G - (j0 >> 1) : GPASS, vf);
            __syncthreads();
        }
    }
    if constexpr (!PF) { // the row's groups
        __syncthreads();
        if (t < M * R) vf = fold_terms(P + t * PS, G, 0.0f);
    }
    if (t < M * R) {
        const int m = t / R, r = t % R, row = row0 + r;
        if (row < nrows) {
            float *o = out + (size_t)m * ldo + row;
            *o = mode == 1 ? *o + vf : vf;
        }
    }
}

// an i-quant row's values (D S) v, one half-group per thread and step: exact in fp32 (iquants.h:211-216), so equal to
// the reference's dequantization expressions (iq_dequant_row, iquants.h:217)
template <int TYPE>
__device__ __forceinline__ void embed_iq(float *__restrict__ y, int dim, const uint8_t *__restrict__ rb, int bstride) {
    for (int j = threadIdx.x; j < dim / 16; j += blockDim.x) {
        const uint8_t *b = rb + (size_t)(j >> 4) * bstride;
        int4 v;
        int S;
        iq_half<TYPE>(b, j & 15, v, S);
        const float ds = iq_d<TYPE>(b) * (float)S;
        const uint32_t w[4] = { (uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w };
        float o[16];
        #pragma unroll
        for (int e = 0; e < 16; e++) o[e] = ds * (float)(int8_t)(w[e >> 2] >> (8 * (e & 3)));
        #pragma unroll
        for (int e = 0; e < 16; e += 4) *(float4 *)(y + 16 * j + e) = make_float4(o[e], o[e + 1], o[e + 2], o[e + 3]);
    }
}

// x[b] = row tok[b] of a K-quant table (Q2_K .. Q6_K) or an i-quant one, dequantized (kq_dequant_row, kquants.h:222-251;
// iq_dequant_row, iquants.h:217; every value one rounding of an exact expression)
__global__ __launch_bounds__(256) void k_embed_kq(float *__restrict__ x, int dim, int type, const uint8_t *__restrict__ W,
                                                  int bstride, const int *__restrict__ tok) {
    int bidx = blockIdx.x;
    size_t rowb = (size_t)(dim / 256) * bstride;
    const uint8_t *rb = W + (size_t)tok[bidx] * rowb;
    float *xo = x + (size_t)bidx * dim;
    switch (type) { // (the i-quants: whole half-groups)
    case GW_IQ4_XS: embed_iq<GW_IQ4_XS>(xo, dim, rb, bstride); return;
    case GW_IQ2_XXS: embed_iq<GW_IQ2_XXS>(xo, dim, rb, bstride); return;
    case GW_IQ2_XS: embed_iq<GW_IQ2_XS>(xo, dim, rb, bstride); return;
    case GW_IQ2_S: embed_iq<GW_IQ2_S>(xo, dim, rb, bstride); return;
    case GW_IQ3_XXS: embed_iq<GW_IQ3_XXS>(xo, dim, rb, bstride); return;
    case GW_IQ3_S: embed_iq<GW_IQ3_S>(xo, dim, rb, bstride); return;
    case GW_IQ1_S: embed_iq<GW_IQ1_S>(xo, dim, rb, bstride); return;
    case GW_IQ1_M: embed_iq<GW_IQ1_M>(xo, dim, rb, bstride); return;
    case GW_IQ3_XXS_R: embed_iq<GW_IQ3_XXS_R>(xo, dim, rb, bstride); return;
    case GW_IQ3_S_R: embed_iq<GW_IQ3_S_R>(xo, dim, rb, bstride); return;
    }
    for (int i = threadIdx.x; i < dim; i += blockDim.x) {
        int s = i >> 8, k = i & 255;
        float y;
        if (type == GW_Q4_K || type == GW_Q5_K) {
            const uint8_t *b = rb + (size_t)s * bstride, *sc = b + 4;
            int j = k >> 5, scj, mj;
            if (j < 4) { scj = sc[j] & 63; mj = sc[j + 4] & 63; }
            else { scj = (sc[j + 4] & 15) | (sc[j - 4] >> 6) << 4; mj = (sc[j + 4] >> 4) | (sc[j] >> 6) << 4; }
            float d = __half2float(__ushort_as_half((uint16_t)(b[0] | b[1] << 8)));
            float dmin = __half2float(__ushort_as_half((uint16_t)(b[2] | b[3] << 8)));
            int q = type == GW_Q4_K ? (b[16 + 32 * (k / 64) + k % 32] >> (4 * (k / 32 % 2))) & 15
                                    : ((b[48 + 32 * (j / 2) + k % 32] >> (4 * (j % 2))) & 15) | ((b[16 + k % 32] >> j) & 1) << 4;
            float d1 = d * (float)scj, m1 = dmin * (float)mj;
            y = d1 * (float)q - m1;
        } else if (type == GW_Q3_K) { // (d (sc_j - 32)) (q' - 4), sub-blocks j of 16
            const uint8_t *b = rb + (size_t)s * bstride;
            int j = k >> 4, n = k / 128, p = k / 32 % 4, l = k % 32;
            int scj = (j < 8 ? b[96 + j] & 15 : b[96 + j - 8] >> 4) | ((b[104 + j % 4] >> (2 * (j / 4))) & 3) << 4;
            int q = ((b[32 + 32 * n + l] >> (2 * p)) & 3) | ((b[l] >> (k / 32)) & 1) << 2;
            float d = __half2float(__ushort_as_half((uint16_t)(b[108] | b[109] << 8)));
            y = (d * (float)(scj - 32)) * (float)(q - 4);
        } else if (type == GW_Q2_K) { // (d sc) q - dmin m, sub-blocks of 16 (iquants.h:224-231)
            const uint8_t *b = rb + (size_t)s * bstride;
            const int sc = b[k >> 4], q = (b[16 + 32 * (k / 128) + k % 32] >> (2 * (k / 32 % 4))) & 3;
            const float d = __half2float(__ushort_as_half((uint16_t)(b[80] | b[81] << 8)));
            const float dmin = __half2float(__ushort_as_half((uint16_t)(b[82] | b[83] << 8)));
            const float dl = d * (float)(sc & 15), ml = dmin * (float)(sc >> 4);
            y = dl * (float)q - ml;
        } else {
            const uint8_t *b = rb + (size_t)s * bstride;
            int n = k / 128, p = k / 32 % 4, l = k % 32;
            int q = ((b[64 * n + 32 * (p & 1) + l] >> (4 * (p >> 1))) & 15) | ((b[128 + 32 * n + l] >> (2 * p)) & 3) << 4;
            float d = __half2float(__ushort_as_half((uint16_t)(b[208] | b[209] << 8)));
            y = (d * (float)(int8_t)b[192 + k / 16]) * (float)(q - 32);
        }
        x[(size_t)bidx * dim + i] = y;
    }
}

template <int TYPE>
static int launch_gemv_mr(const uint8_t *W, const uint16_t *WS, int nrows, int K, int bstride, const int8_t *xq, const float *xs,
                          int ldx, int M, float *out, int ldo, int mode, hipStream_t s) {
    // launches of up to 8 activation rows, one half-group per thread and pass (a row of K > 4096 in several passes: a
    // pass holding a longer row's loads needed every register, one wave per SIMD, and ran the K = 12288 matrix at half
    // the speed)
    const int R = 4;
    hipEvent_t t0, t1; // (timing: the first launch's start, the last one's stop)
    gw_take_launch_events(&t0, &t1);
    dim3 grid((nrows + R - 1) / R);
    for (int m0 = 0; m0 < M; m0 += 8) {
        const int mm = M - m0 < 8 ? M - m0 : 8;
        hipEvent_t e0 = m0 == 0 ? t0 : NULL, e1 = m0 + 8 >= M ? t1 : NULL;
        const bool pf = K > 4096; // (several passes: the terms folded per pass)
        const uint32_t lds = (uint32_t)((size_t)mm * R * (((pf ? 128 : K / 32) + 7) & ~3) * sizeof(float));
        const int8_t *x = xq + (size_t)m0 * ldx;
        const float *xsc = xs + (size_t)m0 * (ldx / 32);
        float *o = out + (size_t)m0 * ldo;
#define MR_L(MM)                                                                                                        \
    do {                                                                                                                \
        if (pf) hipExtLaunchKernelGGL((k_gemv_mr<TYPE, MM, R, 1, true>), grid, dim3(256), lds, s, e0, e1, 0, W, WS, nrows, K, bstride, x, xsc, ldx, o, ldo, mode); \
        else hipExtLaunchKernelGGL((k_gemv_mr<TYPE, MM, R, 1, false>), grid, dim3(256), lds, s, e0, e1, 0, W, WS, nrows, K, bstride, x, xsc, ldx, o, ldo, mode); \
    } while (0)
        switch (mm) {
        case 1: MR_L(1); break;
        case 2: MR_L(2); break;
        case 3: MR_L(3); break;
        case 4: MR_L(4); break;
        case 5: MR_L(5); break;
        case 6: MR_L(6); break;
        case 7: MR_L(7); break;
        default: MR_L(8); break;
        }
#undef MR_L
    }
    return (int)hipGetLastError();
}

// the device layout's byte k (gw_iq.h) of an i-quant super-block: its byte in the file's block, or -1 for padding;
// IQ4_XS's S and D bytes (k 128 .. 139) are computed by k_iq_to_dev
__device__ __forceinline__ int iq_src_byte(int type, int k) {
    switch (type) {
    case GW_IQ2_XXS: return k < 64 ? k + 2 : k < 66 ? k - 64 : -1;
    case GW_IQ2_XS: return k < 72 ? k + 2 : k < 74 ? k - 72 : -1;
    case GW_IQ2_S: return k < 80 ? k + 2 : k < 82 ? k - 80 : -1;
    case GW_IQ3_XXS: return k < 96 ? k + 2 : k < 98 ? k - 96 : -1;
    case GW_IQ3_S: return k < 64 ? k + 2 : k < 96 ? k + 10 : k < 104 ? k - 30 : k < 108 ? k + 2 : k < 110 ? k - 108 : -1;
    case GW_IQ1_S: return k < 48 ? k + 2 : k < 50 ? k - 48 : -1;
    case GW_IQ1_M: return k < 56 ? k : -1;
    case GW_IQ4_XS: return k < 128 ? k + 8 : -1;
    }
    return -1;
}

// an i-quant tensor's super-blocks (sb bytes each in the file) -> the device layout (db bytes), one thread per byte;
// IQ4_XS: S = ls - 32 of group k - 128 (iquants.h:28-29) as int8, then D = d as fp32
__global__ __launch_bounds__(256) void k_iq_to_dev(const uint8_t *__restrict__ src, size_t nblk, int type, int sb, int db,
                                                   uint8_t *__restrict__ dst) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x, b = i / (size_t)db;
    const int k = (int)(i % (size_t)db);
    if (b >= nblk) return;
    const uint8_t *f = src + b * (size_t)sb;
    int v = 0;
    const int o = iq_src_byte(type, k);
    if (o >= 0) v = f[o];
    else if (type == GW_IQ4_XS && k < 136) {
        const int ib = k - 128, sh = f[2] | f[3] << 8;
        v = (uint8_t)(int8_t)((((f[4 + ib / 2] >> (4 * (ib % 2))) & 15) | ((sh >> (2 * ib)) & 3) << 4) - 32);
    } else if (type == GW_IQ4_XS && k < 140) {
        const float D = __half2float(__ushort_as_half((uint16_t)(f[0] | f[1] << 8)));
        v = (__float_as_uint(D) >> (8 * (k - 136))) & 255u;
    }
    dst[i] = (uint8_t)v;
}

// the IQ3 repack (RqModelOpts.repack): IQ3_XXS / IQ3_S super-blocks (the file's, sb bytes) -> 4-bit codes (GW_IQ3R_DEV
// bytes, gw_iq.h). A block of 256 threads takes 32 super-blocks: their device layouts assembled in LDS, then thread
// (super-block, group) decodes its group's 32 values and S (the kernels' own decode, iq_half), writes the codes
// n = e | (v < 0) << 3 in IQ4_XS's nibble order and S; group 0 also D (fp32) and the padding. The same v, S and D, so
// every result is the same bits
template <int BASE>
__global__ __launch_bounds__(256) void k_iq3r_to_dev(const uint8_t *__restrict__ src, size_t nblk, int sb,
                                                     uint8_t *__restrict__ dst) {
    constexpr int DB = BASE == GW_IQ3_XXS ? GW_IQ3XXS_DEV : GW_IQ3S_DEV;
    __shared__ __align__(16) uint8_t lb[32 * DB];
    const size_t b0 = (size_t)blockIdx.x * 32;
    for (int i = threadIdx.x; i < 32 * DB; i += 256) {
        const size_t b = b0 + i / DB;
        const int k = i % DB, o = iq_src_byte(BASE, k);
        lb[i] = b < nblk && o >= 0 ? src[b * (size_t)sb + o] : 0;
    }
    __syncthreads();
    const int lbk = threadIdx.x >> 3, ib = threadIdx.x & 7;
    const size_t b = b0 + lbk;
    if (b >= nblk) return;
    const uint8_t *blk = lb + lbk * DB;
    int4 v0, v1;
    int S0, S1;
    iq_half<BASE>(blk, 2 * ib, v0, S0);
    iq_half<BASE>(blk, 2 * ib + 1, v1, S1);
    auto code = [](int v) -> uint32_t {
        const int a = v < 0 ? -v : v;
        const int e = BASE == GW_IQ3_S ? (a - 1) >> 1 : a == 62 ? 7 : (a - 4) >> 3;
        return (uint32_t)e | (v < 0 ? 8u : 0u);
    };
    const uint32_t w0[4] = { (uint32_t)v0.x, (uint32_t)v0.y, (uint32_t)v0.z, (uint32_t)v0.w };
    const uint32_t w1[4] = { (uint32_t)v1.x, (uint32_t)v1.y, (uint32_t)v1.z, (uint32_t)v1.w };
    uint32_t q[4] = { 0, 0, 0, 0 };
    #pragma unroll
    for (int j = 0; j < 16; j++) {
        const int lo = (int)(int8_t)(w0[j >> 2] >> (8 * (j & 3))), hi = (int)(int8_t)(w1[j >> 2] >> (8 * (j & 3)));
        q[j >> 2] |= (code(lo) | code(hi) << 4) << (8 * (j & 3));
    }
    uint8_t *d = dst + b * GW_IQ3R_DEV;
    *(uint4 *)(d + 16 * ib) = make_uint4(q[0], q[1], q[2], q[3]);
    d[128 + ib] = (uint8_t)(int8_t)S0; // (S0 == S1: one scale per group, iquants.h:18-21)
    if (ib == 0) *(uint2 *)(d + 136) = make_uint2(__float_as_uint(iq_d<BASE>(blk)), 0u);
}

// dst super-block i (db bytes) = src super-block i (sb bytes) and zero padding
__global__ __launch_bounds__(256) void k_kq_pad(const uint8_t *__restrict__ src, size_t nblk, int sb, int db, uint8_t *__restrict__ dst) {
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x, b = i / (size_t)db, k = i % (size_t)db;
    if (b < nblk) dst[i] = k < (size_t)sb ? src[b * sb + k] : 0;
}

// K-quant GEMM for 9 .. 32 activation rows: k_gemm_kq32's tiles (32 weight rows x 32 activation rows per block) and
// staging (per super-block, the 32 rows' blocks and the activation rows' codes and scales loaded with coalesced 16-byte
// loads into double-buffered LDS, four register sets ahead), but 4 waves, each on 16 weight rows x 16 activation rows
// over all 8 groups: per group one v_mfma_i32_16x16x32_i8 (lane l: A = X row l % 16, B = W row l % 16, bytes
// 8 (l / 16) .. + 7 of the group; result register r: activation row 4 (l / 16) + r, weight row l % 16), so each lane's
// weight row is its own and the fold (val = val + term, groups in order) stays in registers: no exchange of terms, one
// barrier per super-block. Q4_K: a second MFMA against ones gives the sums of x; Q6_K: one MFMA per half-group of 16
// (the other half's codes zero: its scale differs), I = sc_0 I_0 + sc_1 I_1. Terms as k_gemm_kq32's (kquants.h:86-109,
// :410-554). Blocks: k_gemm_kq32's (tiles padded to 8 per XCD). M <= 32, K % 256 == 0, mode 1: out = out + val.
// Measured against k_gemm_kq32 at the 4B widths (32 rows): slower on every matrix (4.8 against 3.9 ms of matmuls per
// step; half the waves per CU, each with a chain of 8 groups per super-block; with one wave per tile and no staging,
// scattered 8-byte loads, 6.6 ms; at three blocks per CU it spills), so k_gemm_kq32 is the default
#define KQ16_T 256
template <int TYPE>
struct K16Stage { // one thread's share of a super-block's staging (two 16-byte pieces of W and of X, one scale)
    uint4 w0, w1, x0, x1;
    float xs;
};
template <int TYPE>
__global__ __launch_bounds__(KQ16_T, 2) void k_gemm_kq16(SkMats mats, int bstride, int K, const int8_t *__restrict__ X,
                                                         const float *__restrict__ XS, int ldx, int M, float *out, int ldo,
                                                         int mode) {
    typedef int i32x4v __attribute__((ext_vector_type(4)));
    constexpr int WST = TYPE == GW_Q4_K ? 160 : 240;            // LDS bytes per weight row (bstride + 16)
    constexpr int PW = TYPE == GW_Q4_K ? GW_Q4K_BYTES / 16 : GW_Q6K_DEV / 16; // 16-byte pieces per weight row
    __shared__ __align__(16) uint8_t Ws[2][32 * WST];
    __shared__ __align__(16) uint8_t Xs[2][32 * SK_XR];
    __shared__ __align__(16) float xsl[2][8][32];               // [group][activation row]
    const int t = threadIdx.x, lane = t & 63, w = t >> 6, c = lane >> 4, rr = lane & 15;
    const int wn = 16 * (w & 1), wm = 16 * (w >> 1);            // the wave's weight rows and activation rows in the tile
    const int mi = blockIdx.x >= mats.nb1, bl = blockIdx.x - (mi ? mats.nb1 : 0);
    const int n0 = 32 * ((bl >> 3) * 8 + (bl & 7)), N = mats.N[mi], S = K >> 8;
    if (n0 >= N) return; // (tiles padded to 8 per XCD)
    const size_t rowb = (size_t)S * bstride;
    out += mats.col[mi];
    // staging pieces: W piece t and t + 256 of the tile's 32 PW (row p / PW, piece p % PW; pieces past 32 PW: row 31's
    // again, never staged), X piece t and t + 256 (row p / 16, piece p % 16), XS t (row t / 8, group t % 8)
    const int p1 = t + KQ16_T;
    const int wr0 = t / PW, wr1 = p1 / PW < 32 ? p1 / PW : 31, wp0 = t % PW, wp1 = p1 % PW;
    const uint8_t *ws0 = mats.W[mi] + (size_t)(n0 + wr0 < N ? n0 + wr0 : N - 1) * rowb + 16 * wp0;
    const uint8_t *ws1 = mats.W[mi] + (size_t)(n0 + wr1 < N ? n0 + wr1 : N - 1) * rowb + 16 * wp1;
    const int xr0 = t >> 4, xr1 = xr0 + 16;
    const int8_t *xs0 = X + (size_t)(xr0 < M ? xr0 : M - 1) * ldx + 16 * (t & 15);
    const int8_t *xs1 = X + (size_t)(xr1 < M ? xr1 : M - 1) * ldx + 16 * (t & 15);
    const int sm = (t >> 3) < M ? (t >> 3) : M - 1;
    const float *xssrc = XS + (size_t)sm * (ldx >> 5) + (t & 7);
    auto load = [&](int s) __attribute__((always_inline)) -> K16Stage<TYPE> {
        s = s < S ? s : S - 1; // (past the last super-block: the last again)
        K16Stage<TYPE> o;
        o.w0 = *(const uint4 *)(ws0 + (size_t)s * bstride);
        o.w1 = *(const uint4 *)(ws1 + (size_t)s * bstride);
        o.x0 = *(const uint4 *)(xs0 + 256 * s);
        o.x1 = *(const uint4 *)(xs1 + 256 * s);
        o.xs = xssrc[8 * s];
        return o;
    };
    auto stage = [&](const K16Stage<TYPE> &o, int buf) __attribute__((always_inline)) {
        *(uint4 *)(&Ws[buf][wr0 * WST + 16 * wp0]) = o.w0;
        if (p1 < 32 * PW) *(uint4 *)(&Ws[buf][wr1 * WST + 16 * wp1]) = o.w1;
        *(uint4 *)(&Xs[buf][xr0 * SK_XR + 16 * (t & 15)]) = o.x0;
        *(uint4 *)(&Xs[buf][xr1 * SK_XR + 16 * (t & 15)]) = o.x1;
        xsl[buf][t & 7][t >> 3] = o.xs;
    };
    float acc0 = 0.0f, acc1 = 0.0f, acc2 = 0.0f, acc3 = 0.0f; // activation rows wm + 4 c + r, weight row n0 + wn + rr
    const i32x4v z = { 0, 0, 0, 0 };
    const uint8_t *wrow_l = &Ws[0][(wn + rr) * WST];
    const uint8_t *xrow_l = &Xs[0][(wm + rr) * SK_XR + 8 * c];
    auto step = [&](const K16Stage<TYPE> nx, int s) __attribute__((always_inline)) -> K16Stage<TYPE> {
        // nx holds super-block s + 1: staged into the other buffer (its readers, step s - 1, are past the barrier of
        // step s - 1); returned: the set reloaded with super-block s + 1 + SK_P
        const int buf = s & 1;
        if (s + 1 < S) stage(nx, buf ^ 1);
        const K16Stage<TYPE> nl = load(s + 1 + SK_P);
        if (s >= S) return nl; // (the last group of four steps past the end: its loads only, uniform)
        const uint8_t *wb = wrow_l + buf * (32 * WST), *xb = xrow_l + buf * (32 * SK_XR);
        const float *xsb = &xsl[buf][0][wm + 4 * c];
        if constexpr (TYPE == GW_Q4_K) {
            const uint4 hd = *(const uint4 *)wb;
            const float d = h2f_g((uint16_t)(hd.x & 0xffffu)), dm = h2f_g((uint16_t)(hd.x >> 16));
            #pragma unroll
            for (int g = 0; g < 8; g++) {
                const uint2 xg = *(const uint2 *)(xb + 32 * g);
                const uint2 qq = *(const uint2 *)(wb + 16 + 32 * (g >> 1) + 8 * c);
                const int sh = 4 * (g & 1);
                const i64 a = (i64)xg.x | (i64)xg.y << 32;
                const i64 b = (i64)((qq.x >> sh) & 0x0F0F0F0Fu) | (i64)((qq.y >> sh) & 0x0F0F0F0Fu) << 32;
                const i32x4v I = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
                const i32x4v I1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, (i64)0x0101010101010101ll, z, 0, 0, 0);
                const int bs = 8 * (g & 3);
                const int bw = (int)(((g < 4 ? hd.y : hd.z) >> bs) & 0xffu), bw4 = (int)(((g < 4 ? hd.z : hd.w) >> bs) & 0xffu);
                const int bm4 = (int)((hd.y >> bs) & 0xffu);
                const int scj = g < 4 ? bw & 63 : (bw4 & 15) | (bm4 >> 6) << 4;
                const int mj = g < 4 ? bw4 & 63 : (bw4 >> 4) | (bw >> 6) << 4;
                const float f0 = d * (float)scj, f1 = dm * (float)mj;
                const float4 x4 = *(const float4 *)(xsb + 32 * g);
                acc0 = acc0 + ((f0 * x4.x) * (float)I[0] - f1 * (x4.x * (float)I1[0]));
                acc1 = acc1 + ((f0 * x4.y) * (float)I[1] - f1 * (x4.y * (float)I1[1]));
                acc2 = acc2 + ((f0 * x4.z) * (float)I[2] - f1 * (x4.z * (float)I1[2]));
                acc3 = acc3 + ((f0 * x4.w) * (float)I[3] - f1 * (x4.w * (float)I1[3]));
            }
        } else {
            const uint4 scv = *(const uint4 *)(wb + 192);
            const float d = h2f_g((uint16_t)(*(const uint32_t *)(wb + 208) & 0xffffu));
            #pragma unroll
            for (int g = 0; g < 8; g++) {
                const int nn = g >> 2, p = g & 3, sl = 4 * (p >> 1), shh = 2 * p;
                const uint2 xg = *(const uint2 *)(xb + 32 * g);
                const uint2 lo = *(const uint2 *)(wb + 64 * nn + 32 * (p & 1) + 8 * c);
                const uint2 hq = *(const uint2 *)(wb + 128 + 32 * nn + 8 * c);
                auto code = [&](uint32_t lw, uint32_t hw) -> uint32_t { // 4 codes q - 32 (q = nibble | 2 bits of qh << 4)
                    uint32_t q = ((lw >> sl) & 0x0F0F0F0Fu) | (((hw >> shh) & 0x03030303u) << 4);
                    uint32_t f = q ^ 0x20202020u, sg = f & 0x20202020u;
                    return f | (sg << 1) | (sg << 2);
                };
                const i64 a = (i64)xg.x | (i64)xg.y << 32;
                const i64 b = (i64)code(lo.x, hq.x) | (i64)code(lo.y, hq.y) << 32;
                const i64 b0 = c < 2 ? b : 0, b1 = c < 2 ? 0 : b; // (half-group 0: bytes 0 .. 15 of the group)
                const i32x4v I0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b0, z, 0, 0, 0);
                const i32x4v I1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b1, z, 0, 0, 0);
                const uint32_t scw = (g >> 1) == 0 ? scv.x : (g >> 1) == 1 ? scv.y : (g >> 1) == 2 ? scv.z : scv.w;
                const int sb = 16 * (g & 1);
                const int s0 = (int)(int8_t)((scw >> sb) & 0xffu), s1 = (int)(int8_t)((scw >> (sb + 8)) & 0xffu);
                const float4 x4 = *(const float4 *)(xsb + 32 * g);
                acc0 = acc0 + (d * x4.x) * (float)(s0 * I0[0] + s1 * I1[0]);
                acc1 = acc1 + (d * x4.y) * (float)(s0 * I0[1] + s1 * I1[1]);
                acc2 = acc2 + (d * x4.z) * (float)(s0 * I0[2] + s1 * I1[2]);
                acc3 = acc3 + (d * x4.w) * (float)(s0 * I0[3] + s1 * I1[3]);
            }
        }
        __syncthreads(); // (super-block s + 1 staged; this buffer's readers done)
        return nl;
    };
    static_assert(SK_P == 4, "four register sets");
    K16Stage<TYPE> o0 = load(0), o1 = load(1), o2 = load(2), o3 = load(3);
    stage(o0, 0);
    o0 = load(4);
    __syncthreads();
    for (int s0 = 0; s0 < S; s0 += 4) { // (one exit per group of four steps)
        o1 = step(o1, s0);
        o2 = step(o2, s0 + 1);
        o3 = step(o3, s0 + 2);
        o0 = step(o0, s0 + 3);
    }
    const int n = n0 + wn + rr;
    const float accs[4] = { acc0, acc1, acc2, acc3 };
    #pragma unroll
    for (int r = 0; r < 4; r++) {
        const int m = wm + 4 * c + r;
        if (m < M && n < N) {
            float *po = out + (size_t)m * ldo + n;
            *po = mode == 1 ? *po + accs[r] : accs[r];
        }
    }
}

extern "C" {

int gw_k_kq_to_dev(const uint8_t *src, size_t nblk, int type, uint8_t *dst, hipStream_t s) {
    const int sbytes = gw_kq_file_bytes(type), dbytes = gw_kq_dev_bytes(type);
    if (sbytes < 1 || dbytes < sbytes) return (int)hipErrorInvalidValue;
    if (type == GW_IQ3_XXS_R || type == GW_IQ3_S_R) { // (the file's IQ3 blocks -> the repacked codes)
        const dim3 g((unsigned)((nblk + 31) / 32));
        if (type == GW_IQ3_XXS_R) hipLaunchKernelGGL(k_iq3r_to_dev<GW_IQ3_XXS>, g, dim3(256), 0, s, src, nblk, sbytes, dst);
        else hipLaunchKernelGGL(k_iq3r_to_dev<GW_IQ3_S>, g, dim3(256), 0, s, src, nblk, sbytes, dst);
        return (int)hipGetLastError();
    }
    if (type == GW_IQ4_XS || GW_IS_CB(type)) {
        const size_t n = nblk * (size_t)dbytes;
        hipLaunchKernelGGL(k_iq_to_dev, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src, nblk, type, sbytes, dbytes, dst);
        return (int)hipGetLastError();
    }
    size_t n = nblk * (size_t)dbytes;
    hipLaunchKernelGGL(k_kq_pad, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src, nblk, sbytes, dbytes, dst);
    return (int)hipGetLastError();
}

int gw_k_embed_kq(float *x, int dim, int type, const uint8_t *blocks, int bstride, const int *tok, int n, hipStream_t s) {
    hipEvent_t e0, e1;
    gw_take_launch_events(&e0, &e1);
    hipExtLaunchKernelGGL(k_embed_kq, dim3(n), dim3(256), 0, s, e0, e1, 0, x, dim, type, blocks, bstride, tok);
    return (int)hipGetLastError();
}

int gw_k_q8_unpack(const uint8_t *blocks, size_t nblk, int8_t *codes, uint16_t *scales, int gpr, int il, int off, hipStream_t s) {
    if (!nblk) return 0;
    hipLaunchKernelGGL(k_q8_unpack, dim3((unsigned)((nblk + 255) / 256)), dim3(256), 0, s, blocks, nblk, codes, scales, gpr, il, off);
    return (int)hipGetLastError();
}

int gw_k_fill_synthetic(uint16_t *kc, uint16_t *vc, size_t n, unsigned long long seed, int bf, hipStream_t s) {
    if (!n) return 0;
    hipLaunchKernelGGL(k_fill_synthetic, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, kc, vc, n, seed, bf);
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

static int g_tile_rows = 0; // gw_matmul_tile_rows

static int gemm_cus(void) { // the device's compute units
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            cus = 256;
    }
    return cus;
}

static int g_kq32_nqr; // (0: chosen per launch; 1, 2 or 4: forced, gw_kq32_quads)
static int g_kq32_sb;  // (0: chosen per launch; 1 or 2 super-blocks per step: forced, gw_kq32_step)
static int g_kq16;     // (9 .. 32 K-quant rows: 0 k_gemm_kq32, 1 k_gemm_kq16; gw_kq_small_kernel)
static int g_q8_batch;  // (Q8_0 at 2 .. 32 rows: 0 chosen per launch, 1 the batched GEMV, 2 the MFMA GEMM; gw_q8_batch_kernel)
static int g_q8_lds;    // (the Q8_0 GEMM: 0 chosen per launch, 1 k_gemm_q8f / k_gemm_q8, 2 / 3 k_gemm_q8l of 128 / 64 columns; gw_q8_gemm_kernel)

static bool q8_gemm_rows(const GwMat *w, int M) {
    // a Q8_0 matmul of M activation rows takes the MFMA GEMM (else the batched GEMV in passes of 8 rows): above 16 rows;
    // above 8 for matrices of 8,192 rows or more, above 12 for 6,144 or more at K <= 4,096; where the GEMM takes 512-byte
    // stages (K % 512 == 0), above 8 for 6,144 rows or more and above 12 for 4,096 or more at K <= 4,096 (9 rows 6,144 x
    // 4,096 17.4 / 16.4 us; 16 rows 4,096 x 4,096 17.8 / 16.3 us; 4,096 x 12,288 stays on the GEMV up to 16 rows,
    // 39.3 / 43.5 us). The GEMM's time hardly
    // depends on M or the width (18-23 us at K = 4,096, 50 at 12,288, k_gemm_q8t), the GEMV's grows with both (per 8
    // rows a pass over the weights). Measured at the 8B widths, us (GEMV / GEMM): 9 rows 24,576 x 4,096 48.5 / 32.8,
    // 12,288 x 4,096 28.8 / 21.7, 6,144 x 4,096 17.4 / 18.4, 4,096 x 4,096 14.7 / 18.4, 4,096 x 12,288 34.0 / 49.4;
    // 16 rows 6,144 x 4,096 21.8 / 18.3, 4,096 x 4,096 17.8 / 18.4, 4,096 x 12,288 39.3 / 49.3; 24 rows 4,096 x 4,096
    // 25.7 / 18.4, 4,096 x 12,288 57.9 / 49.4
    const bool s512 = w->cols % 512 == 0 && w->cols <= 4096;
    return M > 16 || (M > 8 && w->rows >= 8192) || (M > 12 && w->rows >= 6144 && w->cols <= 4096) ||
           (s512 && ((M > 8 && w->rows >= 6144) || (M > 12 && w->rows >= 4096)));
}

static int q8l_width(int N, int M, int K) {
    // the Q8_0 GEMM's kernel for N columns and M rows (K % 128 == 0): k_gemm_q8l with 128-column tiles (returns 128),
    // with 64-column tiles (64), k_gemm_q8t of 64 x 64 tiles (16; 17: its 128-byte stages), of 32 x 32 (18; 20: its
    // 512-byte stages) or 32 x 16 (19), or 0: k_gemm_q8f. Forced by gw_q8_gemm_kernel (1 .. 8), else: k_gemm_q8t of
    // 32 x 32 tiles with 512-byte stages where those tiles are at most one per CU and K % 512 == 0 (one block per CU
    // by its LDS; 32 rows 4,096 x 4,096 18.3 -> 16.4, 6,144 x 4,096 18.3 -> 16.7, 4,096 x 12,288 49.9 -> 43.6 us), with
    // 256-byte stages where they are at most 1.5 per CU, of 64 x 64 where those are at most one per CU; else up to 32
    // rows k_gemm_q8f's 32-row tiles, 128
    // columns where those tiles give three blocks per CU or more, else 64. Measured at the 8B widths, us per launch:
    //   k_gemm_q8t 32 x 32 / 64 x 64 / k_gemm_q8f: 32 rows 12,288 x 4,096 22.9 / 25.0 / 31.9; 6,144 x 4,096 18.8 / 23.9 /
    //   31.4; 4,096 x 12,288 49.7 / 63.4 / 87.5; 24,576 x 4,096 38.4 / 47.6 / 34.1; 64 rows 12,288 x 4,096 38.4 / 25.6 /
    //   33.0; 6,144 x 4,096 22.1 / 24.2 / 31.8; 4,096 x 4,096 18.8 / 24.1 / 31.4
    // and (k_gemm_q8f / k_gemm_q8l 128 / 64 columns):
    //   512 rows: 24,576 x 4,096 208 / 188 / 201; 12,288 x 4,096 116 / 101 / 102; 6,144 x 4,096 63.1 / 65.3 / 58.6;
    //             4,096 x 4,096 48.8 / 44.1 / 42.5; 4,096 x 12,288 133 / 122 / 119
    //   256 rows: 24,576 x 4,096 123 / 109 / 109; 12,288 x 4,096 62.9 / 66.2 / 55.1; 4,096 x 12,288 91.2 / 122 / 88.8
    if (g_q8_lds) return g_q8_lds == 2 ? 128 : g_q8_lds == 3 ? 64 : g_q8_lds >= 4 ? 12 + g_q8_lds : 0;
    const size_t cus = (size_t)gemm_cus(), mt = (size_t)((M + 63) / 64);
    const size_t t32 = (size_t)((N + 31) / 32) * ((M + 31) / 32);
    if (t32 <= cus && K % 512 == 0) return 20;
    if (t32 * 2 <= 3 * cus) return 18;
    if ((size_t)((N + 63) / 64) * mt <= cus) return 16;
    if (M <= 32) return 0;
    return (size_t)((N + 127) / 128) * mt >= 3 * cus ? 128 : 64;
}

static bool kq32_takes(const GwMat *w, int M) {
    // K-quants, 9 .. 32 rows: the 32-row GEMM with the groups spread over a block's waves (a matrix of 32768 rows or
    // more, the classifier: the 128-column MFMA GEMM, a block for every compute unit)
    return (w->type == GW_Q4_K || w->type == GW_Q6_K) && M > 8 && M <= 32 && !g_tile_rows && w->rows < 32768;
}

static int launch_kq32(const GwMat *a, const GwMat *b, int col_b, const int8_t *xq, const float *xs, int ldx, int M,
                       float *out, int ldo, int mode, hipStream_t s) {
    // a, and b (NULL: none; same type and width as a) written from column col_b of out
    hipEvent_t e0, e1;
    gw_take_launch_events(&e0, &e1);
    if (g_kq16) { // 16 x 16 sub-tiles per wave, the fold in registers
        SkMats m16;
        m16.W[0] = a->blocks;
        m16.N[0] = a->rows;
        m16.col[0] = 0;
        m16.nb1 = ((a->rows + 255) / 256) * 8; // (32-row tiles padded to 8, one per XCD)
        m16.W[1] = b ? b->blocks : a->blocks;
        m16.N[1] = b ? b->rows : a->rows;
        m16.col[1] = b ? col_b : 0;
        const dim3 g16(m16.nb1 + (b ? ((b->rows + 255) / 256) * 8 : 0));
        if (a->type == GW_Q4_K)
            hipExtLaunchKernelGGL(k_gemm_kq16<GW_Q4_K>, g16, dim3(KQ16_T), 0, s, e0, e1, 0, m16, a->bstride, a->cols, xq, xs, ldx,
                                  M, out, ldo, mode);
        else
            hipExtLaunchKernelGGL(k_gemm_kq16<GW_Q6_K>, g16, dim3(KQ16_T), 0, s, e0, e1, 0, m16, a->bstride, a->cols, xq, xs, ldx,
                                  M, out, ldo, mode);
        return (int)hipGetLastError();
    }
    // quads per block: the whole tile (splitting a tile's activation rows over 2 or 4 blocks, each staging the whole
    // tile, measured slower at the 4B widths even where the tiles alone leave CUs idle: with one block per CU 4.3 ->
    // 4.8 ms of matmuls per 32-row step, with two (2 quads for matrices of fewer tiles than CUs) 3.9 -> 4.1 ms; kept as
    // a forced setting)
    const int nqr = g_kq32_nqr ? g_kq32_nqr : 4, parts = 4 / nqr;
    SkMats mt;
    mt.W[0] = a->blocks;
    mt.N[0] = a->rows;
    mt.col[0] = 0;
    mt.nb1 = ((a->rows + 255) / 256) * 8 * parts; // (tiles padded to 8: one per XCD)
    mt.W[1] = b ? b->blocks : a->blocks;
    mt.N[1] = b ? b->rows : a->rows;
    mt.col[1] = b ? col_b : 0;
    const dim3 grid(mt.nb1 + (b ? ((b->rows + 255) / 256) * 8 * parts : 0));
    // (two super-blocks per step, 16 waves: half the steps, each twice as long: measured slower on every 4B matrix,
    // 3.9 -> 4.7 ms of matmuls per 32-row step; kept as a forced setting)
    const int sbs = g_kq32_sb ? g_kq32_sb : 1;
#define SK_L(TT, NQ, SS) hipExtLaunchKernelGGL((k_gemm_kq32<TT, NQ, SS>), grid, dim3(SK_T * SS), 0, s, e0, e1, 0, mt, a->bstride, \
                                               a->cols, xq, xs, ldx, M, out, ldo, mode)
#define SK_N(TT, SS)                \
    if (nqr == 4) SK_L(TT, 4, SS);  \
    else if (nqr == 2) SK_L(TT, 2, SS); \
    else SK_L(TT, 1, SS);
    if (a->type == GW_Q4_K) {
        if (sbs == 2) { SK_N(GW_Q4_K, 2) } else { SK_N(GW_Q4_K, 1) }
    } else {
        if (sbs == 2) { SK_N(GW_Q6_K, 2) } else { SK_N(GW_Q6_K, 1) }
    }
#undef SK_N
#undef SK_L
    return (int)hipGetLastError();
}

int gw_k_matmul2(const GwMat *a, const GwMat *b, int col_b, const int8_t *xq, const float *xs, int ldx, int M, float *out,
                 int ldo, int mode, hipStream_t s) {
    /* a and b (b from column col_b of out) in one launch where the 9 .. 32-row K-quant GEMM takes both with one type
     * and width; else -1 and nothing launched (the caller launches them one by one) */
    if (kq32_takes(a, M) && kq32_takes(b, M) && a->type == b->type && a->cols == b->cols && a->bstride == b->bstride)
        return launch_kq32(a, b, col_b, xq, xs, ldx, M, out, ldo, mode, s);
    return -1;
}

int gw_k_matmul(const GwMat *w, const int8_t *xq, const float *xs, int ldx, int M, float *out, int ldo, int mode, hipStream_t s) {
    if (w->type == GW_Q8_0 && mode == 0 && (g_q8_batch == 2 ? M >= 2 : g_q8_batch == 1 ? M > GW_GEMV_MAX_ROWS : q8_gemm_rows(w, M))) {
        hipEvent_t e0, e1;
        gw_take_launch_events(&e0, &e1);
        const int cus = gemm_cus(), nt = (w->rows + GN - 1) / GN;
        const bool g64 = g_tile_rows ? g_tile_rows == 64 : (size_t)nt * ((M + 63) / 64) >= (size_t)4 * cus; // (64-row tiles: enough for several waves per SIMD)
        // (full stages, and every buffer offset inside 2^31: the descriptor-based kernel)
        const bool full = w->cols % GKB == 0 && (size_t)(M + 64) * ldx < ((size_t)1 << 31) && (size_t)GN * w->cols < ((size_t)1 << 31);
        const dim3 g64g(nt, (M + 63) / 64), g32g(nt, (M + 31) / 32);
#define GQ_ARGS (const int8_t *)w->codes, (const uint16_t *)w->scales, w->rows, w->cols, xq, xs, ldx, M, out, ldo
        const int mt = (M + 63) / 64, lq0 = full ? q8l_width(w->rows, M, w->cols) : 0,
                  lq1 = lq0 == 20 && w->cols % 512 ? 18 : lq0, lq = lq1 >= 16 && w->cols % 256 ? 17 : lq1;
        if (lq == 128)
            hipExtLaunchKernelGGL(k_gemm_q8l<128>, dim3(((nt + 7) / 8) * 8 * mt), dim3(512), 0, s, e0, e1, 0, GQ_ARGS, mt);
        else if (lq == 64)
            hipExtLaunchKernelGGL(k_gemm_q8l<64>, dim3(((w->rows + 511) / 512) * 8 * mt), dim3(256), 0, s, e0, e1, 0, GQ_ARGS, mt);
        else if (lq == 16) // (64 x 64 tiles, 4 stages of 256 bytes of K in the ring: 139 KB of LDS)
            hipExtLaunchKernelGGL((k_gemm_q8t<64, 64, 4, 2>), dim3(((w->rows + 511) / 512) * 8 * mt), dim3(1024), 0, s, e0, e1, 0, GQ_ARGS, mt);
        else if (lq == 17) // (stages of 128)
            hipExtLaunchKernelGGL((k_gemm_q8t<64, 64, 4, 1>), dim3(((w->rows + 511) / 512) * 8 * mt), dim3(1024), 0, s, e0, e1, 0, GQ_ARGS, mt);
        else if (lq == 18) // (32 x 32 tiles)
            hipExtLaunchKernelGGL((k_gemm_q8t<32, 32, 4, 2>), dim3(((w->rows + 255) / 256) * 8 * ((M + 31) / 32)), dim3(256), 0, s, e0, e1, 0,
                                  GQ_ARGS, (M + 31) / 32);
        else if (lq == 20) // (32 x 32 tiles, stages of 512 bytes of K: 140 KB of LDS, one block per CU)
            hipExtLaunchKernelGGL((k_gemm_q8t<32, 32, 4, 4>), dim3(((w->rows + 255) / 256) * 8 * ((M + 31) / 32)), dim3(256), 0, s, e0, e1, 0,
                                  GQ_ARGS, (M + 31) / 32);
        else if (lq == 19) // (32 x 16 tiles)
            hipExtLaunchKernelGGL((k_gemm_q8t<32, 16, 4, 2>), dim3(((w->rows + 127) / 128) * 8 * ((M + 31) / 32)), dim3(128), 0, s, e0, e1, 0,
                                  GQ_ARGS, (M + 31) / 32);
        else if (full && g64) hipExtLaunchKernelGGL(k_gemm_q8f<64>, g64g, dim3(256), 0, s, e0, e1, 0, GQ_ARGS);
        else if (full) hipExtLaunchKernelGGL(k_gemm_q8f<32>, g32g, dim3(256), 0, s, e0, e1, 0, GQ_ARGS);
        else if (g64) hipExtLaunchKernelGGL((k_gemm_q8<64>), g64g, dim3(256), 0, s, e0, e1, 0, GQ_ARGS);
        else hipExtLaunchKernelGGL((k_gemm_q8<32>), g32g, dim3(256), 0, s, e0, e1, 0, GQ_ARGS);
#undef GQ_ARGS
        return (int)hipGetLastError();
    }
    if (w->type == GW_Q8_0)
        return launch_gemv_mr<GW_Q8_0>((const uint8_t *)w->codes, w->scales, w->rows, w->cols, 0, xq, xs, ldx, M, out, ldo, mode, s);
    if (kq32_takes(w, M)) return launch_kq32(w, NULL, 0, xq, xs, ldx, M, out, ldo, mode, s);
    // K-quants above 32 rows: the MFMA GEMM where it has 64 blocks or more (a block streams its 128 rows' full K in
    // order, so a narrow matrix leaves the device idle) or its row tile is forced, else the batched GEMV in passes of
    // 8 rows
    if (GW_IS_KQ(w->type) && M > 8 && (g_tile_rows || (size_t)((w->rows + GN - 1) / GN) * ((M + 31) / 32) >= 64)) {
        hipEvent_t e0, e1;
        gw_take_launch_events(&e0, &e1);
        const int cus = gemm_cus(), nt = (w->rows + GN - 1) / GN;
        const bool g64 = g_tile_rows ? g_tile_rows == 64 : (size_t)nt * ((M + 63) / 64) >= (size_t)4 * cus;
        const dim3 grid(nt, g64 ? (M + 63) / 64 : (M + 31) / 32);
#define KQ_L(TT, GG) hipExtLaunchKernelGGL((k_gemm_kq<TT, GG>), grid, dim3(256), 0, s, e0, e1, 0, (const uint8_t *)w->blocks, \
                                           w->bstride, w->rows, w->cols, xq, xs, ldx, M, out, ldo, mode)
        if (w->type == GW_Q4_K) {
            if (g64) KQ_L(GW_Q4_K, 64);
            else KQ_L(GW_Q4_K, 32);
        } else if (w->type == GW_Q6_K) {
            if (g64) KQ_L(GW_Q6_K, 64);
            else KQ_L(GW_Q6_K, 32);
        } else if (w->type == GW_Q5_K) {
            if (g64) KQ_L(GW_Q5_K, 64);
            else KQ_L(GW_Q5_K, 32);
        } else if (w->type == GW_IQ4_XS) {
            if (g64) KQ_L(GW_IQ4_XS, 64);
            else KQ_L(GW_IQ4_XS, 32);
        } else if (w->type == GW_IQ2_XXS) {
            if (g64) KQ_L(GW_IQ2_XXS, 64);
            else KQ_L(GW_IQ2_XXS, 32);
        } else if (w->type == GW_IQ2_XS) {
            if (g64) KQ_L(GW_IQ2_XS, 64);
            else KQ_L(GW_IQ2_XS, 32);
        } else if (w->type == GW_IQ2_S) {
            if (g64) KQ_L(GW_IQ2_S, 64);
            else KQ_L(GW_IQ2_S, 32);
        } else if (w->type == GW_IQ3_XXS) {
            if (g64) KQ_L(GW_IQ3_XXS, 64);
            else KQ_L(GW_IQ3_XXS, 32);
        } else if (w->type == GW_IQ3_S) {
            if (g64) KQ_L(GW_IQ3_S, 64);
            else KQ_L(GW_IQ3_S, 32);
        } else if (w->type == GW_IQ1_S) {
            if (g64) KQ_L(GW_IQ1_S, 64);
            else KQ_L(GW_IQ1_S, 32);
        } else if (w->type == GW_IQ1_M) {
            if (g64) KQ_L(GW_IQ1_M, 64);
            else KQ_L(GW_IQ1_M, 32);
        } else if (w->type == GW_IQ3_XXS_R) {
            if (g64) KQ_L(GW_IQ3_XXS_R, 64);
            else KQ_L(GW_IQ3_XXS_R, 32);
        } else if (w->type == GW_IQ3_S_R) {
            if (g64) KQ_L(GW_IQ3_S_R, 64);
            else KQ_L(GW_IQ3_S_R, 32);
        } else if (w->type == GW_Q2_K) {
            if (g64) KQ_L(GW_Q2_K, 64);
            else KQ_L(GW_Q2_K, 32);
        } else {
            if (g64) KQ_L(GW_Q3_K, 64);
            else KQ_L(GW_Q3_K, 32);
        }
#undef KQ_L
        return (int)hipGetLastError();
    }
#define MRQ_L(TT) return launch_gemv_mr<TT>(w->blocks, NULL, w->rows, w->cols, w->bstride, xq, xs, ldx, M, out, ldo, mode, s)
    if (w->type == GW_Q4_K) MRQ_L(GW_Q4_K);
    if (w->type == GW_Q6_K) MRQ_L(GW_Q6_K);
    if (w->type == GW_Q5_K) MRQ_L(GW_Q5_K);
    if (w->type == GW_Q3_K) MRQ_L(GW_Q3_K);
    if (w->type == GW_IQ4_XS) MRQ_L(GW_IQ4_XS);
    if (w->type == GW_Q2_K) MRQ_L(GW_Q2_K);
    if (w->type == GW_IQ2_XXS) MRQ_L(GW_IQ2_XXS);
    if (w->type == GW_IQ2_XS) MRQ_L(GW_IQ2_XS);
    if (w->type == GW_IQ2_S) MRQ_L(GW_IQ2_S);
    if (w->type == GW_IQ3_XXS) MRQ_L(GW_IQ3_XXS);
    if (w->type == GW_IQ3_S) MRQ_L(GW_IQ3_S);
    if (w->type == GW_IQ1_S) MRQ_L(GW_IQ1_S);
    if (w->type == GW_IQ1_M) MRQ_L(GW_IQ1_M);
    if (w->type == GW_IQ3_XXS_R) MRQ_L(GW_IQ3_XXS_R);
    if (w->type == GW_IQ3_S_R) MRQ_L(GW_IQ3_S_R);
#undef MRQ_L
    return (int)hipErrorInvalidValue;
}

int gw_g_set_iq(const uint64_t *iq2xxs, const uint64_t *iq2xs, const uint64_t *iq2s, const uint64_t *iq1s,
                const uint32_t *iq3xxs, const uint32_t *iq3s) {
    /* the i-quant codebooks (gw_iq.h) on the current device: the 8-value grids as uint64, IQ1's as its two tables
     * (2 x 2048: 8 grid + 1, 8 grid - 1), the 4-value grids as uint32 */
    hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(gw_iq2xxs_g), iq2xxs, sizeof(uint64_t) * 256);
    if (e == hipSuccess) e = hipMemcpyToSymbol(HIP_SYMBOL(gw_iq2xs_g), iq2xs, sizeof(uint64_t) * 512);
    if (e == hipSuccess) e = hipMemcpyToSymbol(HIP_SYMBOL(gw_iq2s_g), iq2s, sizeof(uint64_t) * 1024);
    if (e == hipSuccess) e = hipMemcpyToSymbol(HIP_SYMBOL(gw_iq1s_g), iq1s, sizeof(uint64_t) * 2 * 2048);
    if (e == hipSuccess) e = hipMemcpyToSymbol(HIP_SYMBOL(gw_iq3xxs_g), iq3xxs, sizeof(uint32_t) * 256);
    if (e == hipSuccess) e = hipMemcpyToSymbol(HIP_SYMBOL(gw_iq3s_g), iq3s, sizeof(uint32_t) * 512);
    return (int)e;
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
    // one row: the decode GEMV (k_gemv1, as a decode step runs it: 8-row tiles, 2 above K = 4096) where it takes K
    if (M == 1 && K % 64 == 0 && K <= 12288 && (size_t)N * K < ((size_t)1 << 31))
        return gw_k_gemv1_q(&w, K <= 4096 ? 8 : 2, xq, xs, out, 0, NULL, 0, (hipStream_t)stream) ? RQ_ERR_STATE : RQ_OK;
    return gw_k_matmul(&w, xq, xs, K, M, out, N, 0, (hipStream_t)stream) ? RQ_ERR_STATE : RQ_OK;
}

int gw_q8_block_sums(int32_t *isum, const int8_t *codes, int N, int K, const int8_t *xq, int M, void *stream) {
    if (N <= 0 || K <= 0 || M <= 0 || K % 32 || !isum || !codes || !xq) return RQ_ERR_ARG;
    size_t tot = (size_t)M * N * (K / 32);
    hipLaunchKernelGGL(k_q8_block_sums, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, (hipStream_t)stream, isum, codes, N,
                       K, xq, M);
    return hipGetLastError() ? RQ_ERR_STATE : RQ_OK;
}

int gw_q8_gemm_kernel(int k) {
    if (k < 0 || k > 8) return -1;
    int prev = g_q8_lds;
    g_q8_lds = k;
    return prev;
}

int gw_q8_batch_kernel(int k) {
    if (k < 0 || k > 2) return -1;
    int prev = g_q8_batch;
    g_q8_batch = k;
    return prev;
}

int gw_kq_small_kernel(int kq16) {
    if (kq16 != 0 && kq16 != 1) return -1;
    int prev = g_kq16;
    g_kq16 = kq16;
    return prev;
}

int gw_kq32_step(int sb) {
    if (sb != 0 && sb != 1 && sb != 2) return -1;
    int prev = g_kq32_sb;
    g_kq32_sb = sb;
    return prev;
}

int gw_kq32_quads(int nqr) {
    if (nqr != 0 && nqr != 1 && nqr != 2 && nqr != 4) return -1;
    int prev = g_kq32_nqr;
    g_kq32_nqr = nqr;
    return prev;
}

int gw_matmul_tile_rows(int rows) {
    if (rows != 0 && rows != 32 && rows != 64) return -1;
    int prev = g_tile_rows;
    g_tile_rows = rows;
    return prev;
}

int gw_kq_matmul(float *out, int type, const void *blocks, int N, int K, const int8_t *xq, const float *xs, int M, void *stream) {
    if (N <= 0 || K <= 0 || M <= 0 || K % 256 || !GW_IS_KQ(type) || !out || !blocks || !xq || !xs) return RQ_ERR_ARG;
    if ((GW_IS_CB(type) || type == GW_IQ3_XXS_R || type == GW_IQ3_S_R) && gw_iq_init(NULL, 0) != RQ_OK) return RQ_ERR_STATE;
    const int fb = gw_kq_file_bytes(type), db = gw_kq_dev_bytes(type);
    GwMat w = { type, N, K, NULL, NULL, (uint8_t *)blocks, fb };
    if (fb == db) return gw_k_matmul(&w, xq, xs, K, M, out, N, 0, (hipStream_t)stream) ? RQ_ERR_STATE : RQ_OK;
    // Q6_K, Q3_K, Q2_K, the i-quants: the file's blocks put into the device layout first (a temporary copy)
    size_t nblk = (size_t)N * (K / 256);
    uint8_t *pad = NULL;
    if (hipMalloc((void **)&pad, nblk * db) != hipSuccess) return RQ_ERR_NOMEM;
    w.blocks = pad;
    w.bstride = db;
    int rc = gw_k_kq_to_dev((const uint8_t *)blocks, nblk, type, pad, (hipStream_t)stream) ||
             gw_k_matmul(&w, xq, xs, K, M, out, N, 0, (hipStream_t)stream) ? RQ_ERR_STATE : RQ_OK;
    if (hipStreamSynchronize((hipStream_t)stream) != hipSuccess) rc = RQ_ERR_STATE;
    (void)hipFree(pad);
    return rc;
}

} // extern "C"
