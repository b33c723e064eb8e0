// The single-row Q8_0 GEMV of the decode step with the producer of its activation fused in front (a prologue):
// every thread owns one 16-code chunk of the activation row, computes those 16 values from the producer's fp32 output,
// quantizes them (the group of 32 is the thread and its lane pair: forward.c:803-836) and takes them straight into its
// int8 dots with the R weight rows of the block. No activation round trip through memory, no kernel between the
// producer's output and the matmul. Prologues (each the arithmetic of the kernel it replaces, operation for operation):
//   GV_Q        none: the row is already quantized (xq, xs)
//   GV_NORM     rmsnorm (forward.c:886-901): the row into LDS transposed (chain j's values x[j], x[j + 16], ...
//               contiguous), the 16 fma chains, the tree, r = rsqrt_ref(fma(ss, 1/n, 1e-6)); o = (w * x) * r
//   GV_QF       none but the quantization: the fp32 row as it is (the SwiGLU output of the w1 / w3 matmul)
//   GV_COMBINE  att_combine (forward.c:1405-1431) over the row's <= GV_NBMAX key blocks: M = max m_b, c_b =
//               exp_att(m_b - M), L = fma chain of c_b l_b, o = (fma chain of c_b o_b) * (1 / L)
// Epilogue (swiglu_il = 4, with R = 8): the rows are w1 / w3 interleaved in blocks of 4, so a tile's rows r and r + 4
// are h and h2 of one output; its fold lanes write swiglu_ref(h, h2) (SwiGLU, forward.c:1953-1958) to out[tile 4 + r]
// instead of the two dots
// The prologue's loads are issued before the weight loads (vector memory counts complete in order, so the prologue's
// waits leave the weight loads in flight), the weight loads before any prologue arithmetic.
// Then, as in every Q8_0 kernel here: the exact int32 sum of a half-group by 4 v_dot4, the lane pair's sums added, the even lane's
// (ws * xs) * (float) isum into LDS, one lane per row folding the groups in order (forward.c:906-916).
#include <hip/hip_ext.h>

#include "gw_internal.h"
#include "gw_device.h"

enum { GV_Q = 0, GV_NORM = 1, GV_QF = 2, GV_COMBINE = 3 };
#define GV_NBMAX GW_GV_NBMAX

struct GvArgs {
    const int8_t *W;
    const uint16_t *WS;
    int nrows, K;
    const int8_t *xq; // GV_Q: the quantized row (K codes) and its scales
    const float *xs;
    const float *x;   // GV_NORM, GV_QF: the fp32 row; GV_NORM: the norm's weights
    const float *nw;
    const float *part; // GV_COMBINE: head h's block b at part + h pstride + b (hd + 2): o (hd), m, l; nb blocks
    int pstride, hd, nb;
    int swiglu_il;    // 4: the SwiGLU epilogue (R = 8), else 0
    float *out;       // out[row] (mode 1: out[row] + val, a residual add)
    int mode;
    int cmax;         // tiles whose partials the block keeps in LDS between folds
    float inv_k;      // GV_NORM: 1.0f / K (the host's division, as the reference's 1.0f / size)
    // the next matmul of the sequence (NULL: none): its codes and scales (n_cbytes, n_sbytes), its whole tiles' bytes
    // (n_tb codes, n_tsb scales; n_tb >= K), whole-tile count and grid; block b warms that matmul's tiles b, b + n_grid
    const int8_t *nW;
    const uint16_t *nWS;
    int n_cbytes, n_sbytes, n_tb, n_tsb, n_tiles, n_grid;
};

__device__ __forceinline__ float gv_fold(const float *p, int G) {
    // val = val + p[g] for g in order; the LDS reads of the next 32 before the adds of the current 32
    float v = 0.0f;
    int g = 0;
    if (G >= 32) {
        float4 a[8];
        #pragma unroll
        for (int u = 0; u < 8; u++) a[u] = *(const float4 *)(p + 4 * u);
        for (g = 32; g + 32 <= G; g += 32) {
            float4 b[8];
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
            for (int u = 0; u < 8; u++) a[u] = b[u];
        }
        #pragma unroll
        for (int u = 0; u < 8; u++) {
            v = v + a[u].x;
            v = v + a[u].y;
            v = v + a[u].z;
            v = v + a[u].w;
        }
    }
    for (; g < G; g++) v = v + p[g];
    return v;
}

// blockDim = H = K / 16 rounded up to whole waves, <= NT (K % 64 == 0, K <= 16 NT; NT = 256: K <= 4096, NT = 768:
// K <= 12288). Persistent over tiles of R weight rows: block b takes tiles b, b + grid, ... (grid <= the
// tile count); the prologue runs once per block, and the next tile's weight loads are issued before the current
// tile's dots
// One tile's loads: buffer loads, the row's offset (uniform: row K bytes, row G scales) in the scalar offset and the
// thread's part (16 j bytes) in the vector one, so no per-row address arithmetic in vector registers. Each scale is
// loaded as its aligned 32-bit word (G is even) and kept raw until used: a conversion, or two 16-bit values packed into
// one register, would wait for the loads just issued
// the weight loads are non-temporal (cache policy nt): each weight byte is read once per token, and a streaming
// insert keeps the caches for what is read again (the K / V cache, the activations, the exactness tables). Measured
// on the 8B decode step: 2.59 -> 2.51 ms per token
#ifndef GV_WNT
#define GV_WNT 2
#endif
// register sets of weight tiles per block (D - 1 tiles in flight): 3, and 4 behind the attention combine (wo: 4 tiles
// of 4 rows per block, so three of them load during the prologue). Measured on the 8B decode step, µs per token:
// D = 4 everywhere: wo 345 -> 304, qkv 324 -> 338, w1/w3 773 -> 804, w2 481 -> 511; D = 5 slower everywhere; wo alone
// at 4: 345 -> 301, at 5: 331
#define GV_DEPTH 3
#define GV_DEPTH_COMBINE 4 // (256-thread blocks only: at 768 threads a wave has 168 registers, and 4 sets spilled 141)
template <int R>
__device__ __forceinline__ void gv_load_rows(__amdgpu_buffer_rsrc_t rw, __amdgpu_buffer_rsrc_t rs, int cb, int cl, int sb, int sl,
                                             int j, int K, int G, int4 (&wv)[R], uint32_t (&ws)[R]) {
    // R rows' loads: row r's codes at byte cb + min(r K, cl) of rw, its scales at sb + min(r 2 G, sl) of rs (the clamps:
    // a partial last tile loads its last row again)
    #pragma unroll
    for (int r = 0; r < R; r++) {
        const int o = r * K < cl ? r * K : cl;
        wv[r] = __builtin_bit_cast(int4, __builtin_amdgcn_raw_buffer_load_b128(rw, 16 * j, cb + o, GV_WNT));
    }
    #pragma unroll
    for (int r = 0; r < R; r++) {
        const int o = r * G * 2 < sl ? r * G * 2 : sl;
        ws[r] = __builtin_amdgcn_raw_buffer_load_b32(rs, ((j >> 1) & ~1) * 2, sb + o, GV_WNT);
    }
}

template <int R>
__device__ __forceinline__ void gv_load_tile(__amdgpu_buffer_rsrc_t rw, __amdgpu_buffer_rsrc_t rs, int nrows, int tile, int j,
                                             int K, int G, int4 (&wv)[R], uint32_t (&ws)[R]) {
    const int last = nrows - 1 - tile * R; // (the tile's rows past the matrix's last row load that row)
    gv_load_rows<R>(rw, rs, tile * R * K, last * K, tile * R * G * 2, last * G * 2, j, K, G, wv, ws);
}

// the group of 32 (this lane's 16 values and its pair's): wmax, s = wmax / 127, q = trunc(v * inv + copysign(.49999997))
// (forward.c:803-836); the pair is lanes t, t ^ 1
__device__ __forceinline__ void gv_quant16(const float (&v)[16], int4 &xq, float &xs) {
    float wm = 0.0f;
    #pragma unroll
    for (int i = 0; i < 16; i++) wm = fmaxf(wm, fabsf(v[i]));
    float wo = __shfl_xor(wm, 1);
    wm = wo > wm ? wo : wm;
    xs = wm * (1.0f / 127.0f);
    uint32_t pk[4] = { 0, 0, 0, 0 };
    if (wm > 0.0f) {
        float inv = 127.0f / wm;
        #pragma unroll
        for (int i = 0; i < 16; i++) {
            float y = v[i] * inv;
            int32_t qi = (int32_t)(y + copysignf(0.49999997f, y));
            pk[i >> 2] |= ((uint32_t)qi & 0xffu) << (8 * (i & 3));
        }
    }
    xq = make_int4((int)pk[0], (int)pk[1], (int)pk[2], (int)pk[3]);
}

template <int R, int PRO, int NT, int D>
__global__ __launch_bounds__(NT) void k_gemv1(GvArgs a) {
    extern __shared__ float lds[];
    const int K = a.K, G = K >> 5, H = K >> 4, PS = (G + 7) & ~3; // (rows 16-byte aligned, 4+ banks apart)
    const int t = threadIdx.x, ntiles = (a.nrows + R - 1) / R;
    const bool act = t < H;
    const int j = act ? t : H - 1; // (threads past the row load its last chunk again: every load unconditional)
    float *xf = lds + a.cmax * R * PS; // GV_NORM: the row transposed, then its scale
    int tile = blockIdx.x;

    // 1. the prologue's loads (GV_Q: the row's codes and its group's scale themselves)
    int4 xv;
    float xsg;
    if (PRO == GV_Q) {
        xv = *(const int4 *)(a.xq + 16 * j);
        xsg = a.xs[j >> 1];
    }
    float4 p0[4], p1[4];
    float2 po[GV_NBMAX][8];
    float pm[GV_NBMAX], pl[GV_NBMAX];
    const int nb = PRO == GV_COMBINE ? a.nb : 1;
    if (PRO == GV_NORM || PRO == GV_QF) {
        #pragma unroll
        for (int u = 0; u < 4; u++) p0[u] = ((const float4 *)(a.x + 16 * j))[u];
    }
    if (PRO == GV_NORM) {
        #pragma unroll
        for (int u = 0; u < 4; u++) p1[u] = ((const float4 *)(a.nw + 16 * j))[u];
    }
    if (PRO == GV_COMBINE) {
        const int st = a.hd + 2, e0 = 16 * j, i0 = e0 % a.hd;
        const float *pb = a.part + (size_t)(e0 / a.hd) * a.pstride + i0;
        #pragma unroll
        for (int b = 0; b < GV_NBMAX; b++) {
            int bb = b < nb ? b : nb - 1;
            const float2 *q = (const float2 *)(pb + bb * st);
            #pragma unroll
            for (int u = 0; u < 8; u++) po[b][u] = q[u];
            pm[b] = pb[bb * st + a.hd - i0];
            pl[b] = pb[bb * st + a.hd - i0 + 1];
        }
    }
    // 2. the weight loads of the block's first D - 1 tiles (past the block's last tile: its first again)
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void *)a.W, (short)0, a.nrows * K, GW_RSRC_DW3);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)a.WS, (short)0, (a.nrows * G * 2 + 3) & ~3, GW_RSRC_DW3);
    const int odd = (j >> 1) & 1; // (the half of the scale's word)
    int4 wv[D][R];
    uint32_t ws[D][R];
    // the combine's partials arrive before the weight loads are issued: its 40 small loads per thread otherwise queue
    // behind the tiles (wo 301 -> 292 us per token); the rmsnorm's row does not gain from it (its row arrives no sooner)
    if (PRO == GV_COMBINE) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    #pragma unroll
    for (int d = 0; d + 1 < D; d++) {
        const int td = tile + d * (int)gridDim.x;
        gv_load_tile<R>(rw, rs, a.nrows, td < ntiles ? td : tile, j, K, G, wv[d], ws[d]);
    }
    // 3. this thread's 16 activation codes and its group's scale
    if (PRO != GV_Q) {
        float v[16];
        if (PRO == GV_QF) {
            #pragma unroll
            for (int u = 0; u < 4; u++) {
                v[4 * u + 0] = p0[u].x;
                v[4 * u + 1] = p0[u].y;
                v[4 * u + 2] = p0[u].z;
                v[4 * u + 3] = p0[u].w;
            }
        } else if (PRO == GV_NORM) {
            // the row in the chains' layout (rms_chain): value e at xf[(e % 16) LS + e / 16], LS = 4 NF + 4, zeros from
            // e / 16 = K / 16 to 4 NF; the scale after the 16 chains
            const int n4 = K >> 6, NF = rms_nf(n4), LS = 4 * NF + 4;
            if (act) {
                #pragma unroll
                for (int u = 0; u < 4; u++) {
                    xf[(4 * u + 0) * LS + t] = p0[u].x;
                    xf[(4 * u + 1) * LS + t] = p0[u].y;
                    xf[(4 * u + 2) * LS + t] = p0[u].z;
                    xf[(4 * u + 3) * LS + t] = p0[u].w;
                }
            }
            if (NF > n4)
                for (int z = t; z < 16 * (NF - n4); z += (int)blockDim.x)
                    ((float4 *)xf)[(z / (NF - n4)) * (NF + 1) + n4 + z % (NF - n4)] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            __syncthreads();
            if (t < 64) {
                float ss = 0.0f;
                if (t < 16) {
                    const float4 *c = (const float4 *)xf + t * (NF + 1);
                    if (NF == 16) ss = rms_chain<16>(c);
                    else if (NF == 32) ss = rms_chain<32>(c);
                    else ss = rms_chain<64>(c); // (K <= 4096)
                }
                // the tree over the 16 chains, as ss + shfl_down(ss, w) for w = 8, 4, 2, 1: lane 0's value from lanes
                // 0-15 by DPP row shifts (row_shl:w, lane j + w of the same 16-lane row), no LDS round trips
                ss = ss + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(ss), 0x108, 0xF, 0xF, true));
                ss = ss + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(ss), 0x104, 0xF, 0xF, true));
                ss = ss + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(ss), 0x102, 0xF, 0xF, true));
                ss = ss + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(ss), 0x101, 0xF, 0xF, true));
                if (t == 0) xf[16 * LS] = rsqrt_ref(__builtin_fmaf(ss, a.inv_k, 1e-6f));
            }
            __syncthreads();
            float r = xf[16 * LS];
            #pragma unroll
            for (int u = 0; u < 4; u++) {
                v[4 * u + 0] = (p1[u].x * p0[u].x) * r;
                v[4 * u + 1] = (p1[u].y * p0[u].y) * r;
                v[4 * u + 2] = (p1[u].z * p0[u].z) * r;
                v[4 * u + 3] = (p1[u].w * p0[u].w) * r;
            }
        } else { // GV_COMBINE
            if (nb == 1) {
                float inv = 1.0f / pl[0];
                #pragma unroll
                for (int u = 0; u < 8; u++) {
                    v[2 * u] = po[0][u].x * inv;
                    v[2 * u + 1] = po[0][u].y * inv;
                }
            } else {
                float M = pm[0];
                #pragma unroll
                for (int b = 1; b < GV_NBMAX; b++)
                    if (b < nb) M = pm[b] > M ? pm[b] : M;
                float cb[GV_NBMAX], L = 0.0f;
                #pragma unroll
                for (int b = 0; b < GV_NBMAX; b++)
                    if (b < nb) {
                        cb[b] = exp_att(pm[b] - M);
                        L = __builtin_fmaf(cb[b], pl[b], L);
                    }
                float inv = 1.0f / L;
                #pragma unroll
                for (int u = 0; u < 8; u++) {
                    float a0 = 0.0f, a1 = 0.0f;
                    #pragma unroll
                    for (int b = 0; b < GV_NBMAX; b++)
                        if (b < nb) {
                            a0 = __builtin_fmaf(cb[b], po[b][u].x, a0);
                            a1 = __builtin_fmaf(cb[b], po[b][u].y, a1);
                        }
                    v[2 * u] = a0 * inv;
                    v[2 * u + 1] = a1 * inv;
                }
            }
        }
        gv_quant16(v, xv, xsg);
    }
    // 4. the tiles: the load of the tile D - 1 ahead, this tile's dots into LDS slot k % C; every C tiles (and after the
    // last) one barrier and the fold of all C x R rows in parallel (one lane per row), so no fold stands between one
    // tile's loads and the next. D register sets take turns, D - 1 tiles in flight (a copy from a later tile's
    // registers would wait for their loads)
    const int C = a.cmax;
    // past the block's last tile, the loads of the tile D - 1 ahead warm the next matmul's first tiles for the block of
    // the same index instead (the same L2: a block's XCD is its index modulo the XCD count, and both grids are the
    // device's CUs), or load this tile again. Their registers are never read: the data go no further than the caches
    const bool pfon = a.nW && (int)blockIdx.x < a.n_grid;
    const __amdgpu_buffer_rsrc_t rwn = __builtin_amdgcn_make_buffer_rsrc((void *)(pfon ? a.nW : a.W), (short)0,
                                                                          pfon ? a.n_cbytes : a.nrows * K, GW_RSRC_DW3);
    const __amdgpu_buffer_rsrc_t rsn = __builtin_amdgcn_make_buffer_rsrc((void *)(pfon ? a.nWS : a.WS), (short)0,
                                                                          pfon ? a.n_sbytes : (a.nrows * G * 2 + 3) & ~3, GW_RSRC_DW3);
    int pfi = 0; // (the next matmul's tile blockIdx.x + pfi n_grid comes next)
    auto step = [&](const int4 (&cw)[R], const uint32_t (&cs)[R], int4 (&nw)[R], uint32_t (&ns)[R], int k) -> bool {
        const int nt = tile + gridDim.x, nta = tile + (D - 1) * (int)gridDim.x;
        const bool more = nt < ntiles;
        // the tile D - 1 ahead (unconditional, every choice below uniform: loads under a branch would make every later
        // wait count for the path without them)
        const int ti = (int)blockIdx.x + pfi * a.n_grid;
        const bool ahead = nta < ntiles, pf = !ahead && pfon && ti < a.n_tiles;
        const int tl = ahead ? nta : tile, last = a.nrows - 1 - tl * R;
        pfi += ahead ? 0 : 1;
        gv_load_rows<R>(pf ? rwn : rw, pf ? rsn : rs, pf ? ti * a.n_tb : tl * R * K, pf ? a.n_tb - K : last * K,
                        pf ? ti * a.n_tsb : tl * R * G * 2, pf ? a.n_tsb - G * 2 : last * G * 2, j, K, G, nw, ns);
        const int slot = k % C;
        float *P = lds + slot * R * PS;
        #pragma unroll
        for (int r = 0; r < R; r++) {
            int s = __builtin_amdgcn_sdot4(cw[r].x, xv.x, 0, false);
            s = __builtin_amdgcn_sdot4(cw[r].y, xv.y, s, false);
            s = __builtin_amdgcn_sdot4(cw[r].z, xv.z, s, false);
            s = __builtin_amdgcn_sdot4(cw[r].w, xv.w, s, false);
            s = s + __shfl_xor(s, 1);
            if (act && !(t & 1)) {
                float sc = h2f((uint16_t)(cs[r] >> (16 * odd))) * xsg;
                P[r * PS + (t >> 1)] = sc * (float)s;
            }
        }
        if (slot == C - 1 || !more) {
            __syncthreads();
            const int sl = t / R, row = (tile - (slot - sl) * (int)gridDim.x) * R + t % R;
            const bool fl = t < (slot + 1) * R && row < a.nrows;
            float v = fl ? gv_fold(lds + (size_t)t * PS, G) : 0.0f;
            if (a.swiglu_il) {
                // (R = 8: the tile's rows r and r + 4, h and h2 of output tile 4 + r, are lanes t and t + 4 of one wave)
                float h2 = __shfl_down(v, 4);
                if (fl && (t & 7) < 4) a.out[(row >> 3) * 4 + (row & 7)] = swiglu_ref(v, h2);
            } else if (fl) {
                a.out[row] = a.mode == 1 ? a.out[row] + v : v;
            }
            __syncthreads();
        }
        tile = nt;
        return more;
    };
    for (int k = 0;; k += D) {
        bool more = true;
        #pragma unroll
        for (int d = 0; d < D; d++) {
            more = step(wv[d], ws[d], wv[(d + D - 1) % D], ws[(d + D - 1) % D], k + d);
            if (!more) break;
        }
        if (!more) break;
    }
}

extern "C" {

// the matmul out[row] (+)= W row . act, act = the prologue's quantized row; R weight rows per block (4, 8 or 16)
static int gv_nwg = 0; // blocks per launch: the device's compute units (one block each)
static int gv_warm = 1; // gw_gemv_warm_next

static int gv_launch(int pro, int R, const GvArgs &a, const GwMat *nx, int nR, hipStream_t s) {
    if (!gv_nwg) {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return (int)hipErrorInvalidDevice;
        gv_nwg = cus > 0 ? cus : 256;
    }
    const int H = a.K / 16, nt = (H + 63) / 64 * 64, ntiles = (a.nrows + R - 1) / R, nwg = ntiles < gv_nwg ? ntiles : gv_nwg;
    // partial slots: the block's tile count, at most 16, 96 KiB of LDS and one fold lane per slot row (C R <= threads)
    size_t slot_bytes = (size_t)R * ((a.K / 32 + 7) & ~3) * sizeof(float);
    int tpw = (ntiles + nwg - 1) / nwg, cmax = (int)((96 << 10) / slot_bytes);
    cmax = cmax > 16 ? 16 : cmax;
    cmax = cmax > nt / R ? nt / R : cmax;
    cmax = cmax < 1 ? 1 : cmax;
    GvArgs b = a;
    b.cmax = tpw < cmax ? tpw : cmax;
    b.inv_k = 1.0f / (float)a.K;
    if (gv_warm && nx && nR > 0 && nx->type == GW_Q8_0 && nx->cols % 64 == 0 && (size_t)nx->rows * nx->cols < ((size_t)1 << 31) &&
        nx->rows >= nR && (size_t)nR * nx->cols >= (size_t)a.K) {
        /* the next matmul's launch as gv_launch makes it (whole tiles only: every warm load inside the matrix) */
        const int nnt = (nx->rows + nR - 1) / nR;
        b.nW = nx->codes, b.nWS = nx->scales;
        b.n_cbytes = nx->rows * nx->cols, b.n_sbytes = (nx->rows * (nx->cols / 32) * 2 + 3) & ~3;
        b.n_tb = nR * nx->cols, b.n_tsb = nR * (nx->cols / 32) * 2;
        b.n_tiles = nx->rows / nR, b.n_grid = nnt < gv_nwg ? nnt : gv_nwg;
    }
    size_t lds = (size_t)b.cmax * slot_bytes + (pro == GV_NORM ? (size_t)(16 * (4 * rms_nf(a.K / 64) + 4) + 4) * sizeof(float) : 0);
    dim3 grid(nwg);
    hipEvent_t e0, e1;
    gw_take_launch_events(&e0, &e1);
#define GV_L(RR, PP, NN)                                                                                               \
    hipExtLaunchKernelGGL((k_gemv1<RR, PP, NN, PP == GV_COMBINE && NN == 256 ? GV_DEPTH_COMBINE : GV_DEPTH>), grid, dim3(nt), \
                          (uint32_t)lds, s, e0, e1, 0, b)
#define GV_R(PP)                                                                                                        \
    if (nt <= 256) {                                                                                                    \
        if (R == 2) GV_L(2, PP, 256);                                                                                   \
        else if (R == 4) GV_L(4, PP, 256);                                                                              \
        else if (R == 8) GV_L(8, PP, 256);                                                                              \
        else GV_L(16, PP, 256);                                                                                         \
    } else { /* (the rmsnorm prologue only with K <= 4096, 256 threads: gw_k_gemv1_norm) */                            \
        constexpr int NTW = PP == GV_NORM ? 256 : 768;                                                                  \
        if (R == 2) GV_L(2, PP, NTW);                                                                                   \
        else if (R == 4) GV_L(4, PP, NTW);                                                                              \
        else GV_L(8, PP, NTW);                                                                                          \
    }
    switch (pro) {
    case GV_Q: GV_R(GV_Q); break;
    case GV_NORM: GV_R(GV_NORM); break;
    case GV_QF: GV_R(GV_QF); break;
    default: GV_R(GV_COMBINE); break;
    }
#undef GV_R
#undef GV_L
    return (int)hipGetLastError();
}

int gw_v_set_exact(const float *rsq, int bits, const uint64_t *rcp, const uint8_t *expd) {
    /* this file's copy of the host-measured tables (rsqrt_ref, swiglu_ref) on the current device */
    hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(gw_rsqrt_bits), &bits, sizeof(int));
    if (e == hipSuccess && bits) e = hipMemcpyToSymbol(HIP_SYMBOL(gw_rsqrt_tab), rsq, sizeof(float) << bits);
    if (e == hipSuccess) e = hipMemcpyToSymbol(HIP_SYMBOL(gw_rcp_blk), &rcp, sizeof(rcp));
    if (e == hipSuccess) e = hipMemcpyToSymbol(HIP_SYMBOL(gw_exp_delta), &expd, sizeof(expd));
    return (int)e;
}

static int gv_check(const GwMat *w, int R) {
    /* (K <= 4096: 256 threads, R 2, 4, 8 or 16; K <= 12288: 768 threads, R 2, 4 or 8; K % 64 == 0: whole scale words per row;
     * the matrix under 2 GiB: 32-bit buffer offsets) */
    return w->type == GW_Q8_0 && w->cols % 64 == 0 && w->cols <= 12288 && (size_t)w->rows * w->cols < ((size_t)1 << 31) &&
                   (R == 2 || R == 4 || R == 8 || (R == 16 && w->cols <= 4096)) ? 0 : (int)hipErrorInvalidValue;
}

int gw_gemv_warm_next(int on) {
    int prev = gv_warm;
    if (on >= 0) gv_warm = on ? 1 : 0;
    return prev;
}

int gw_k_gemv1_q(const GwMat *w, int R, const int8_t *xq, const float *xs, float *out, int mode, const GwMat *nx, int nR,
                 hipStream_t s) {
    if (gv_check(w, R)) return (int)hipErrorInvalidValue;
    GvArgs a = {};
    a.W = w->codes, a.WS = w->scales, a.nrows = w->rows, a.K = w->cols, a.xq = xq, a.xs = xs, a.out = out, a.mode = mode;
    return gv_launch(GV_Q, R, a, nx, nR, s);
}

int gw_k_gemv1_norm(const GwMat *w, int R, const float *x, const float *nw, float *out, int mode, int swiglu_il,
                    const GwMat *nx, int nR, hipStream_t s) {
    if (gv_check(w, R) || w->cols > 4096 || (swiglu_il && (swiglu_il != 4 || R != 8 || w->rows % 8)))
        return (int)hipErrorInvalidValue;
    GvArgs a = {};
    a.W = w->codes, a.WS = w->scales, a.nrows = w->rows, a.K = w->cols, a.x = x, a.nw = nw, a.out = out, a.mode = mode;
    a.swiglu_il = swiglu_il;
    return gv_launch(GV_NORM, R, a, nx, nR, s);
}

int gw_k_gemv1_qf(const GwMat *w, int R, const float *x, float *out, int mode, const GwMat *nx, int nR, hipStream_t s) {
    if (gv_check(w, R)) return (int)hipErrorInvalidValue;
    GvArgs a = {};
    a.W = w->codes, a.WS = w->scales, a.nrows = w->rows, a.K = w->cols, a.x = x, a.out = out, a.mode = mode;
    return gv_launch(GV_QF, R, a, nx, nR, s);
}

int gw_k_gemv1_combine(const GwMat *w, int R, const float *part, int pstride, int hd, int nb, float *out, int mode,
                       const GwMat *nx, int nR, hipStream_t s) {
    if (gv_check(w, R) || hd % 16 || nb < 1 || nb > GV_NBMAX) return (int)hipErrorInvalidValue;
    GvArgs a = {};
    a.W = w->codes, a.WS = w->scales, a.nrows = w->rows, a.K = w->cols, a.part = part, a.pstride = pstride, a.hd = hd;
    a.nb = nb, a.out = out, a.mode = mode;
    return gv_launch(GV_COMBINE, R, a, nx, nR, s);
}

} // extern "C"
