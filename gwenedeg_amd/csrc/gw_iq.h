// The i-quant weight formats on the device: each super-block (256 values of one row) read in the integer form the
// reference's definition is written in (iquants.h:33-47): w = D * S * v, D per super-block (fp32, exact), S an integer
// per half-group of 16 values, v a small integer per value. A kernel asks for one half-group at a time: iq_raw loads
// the (at most 20) bytes of the super-block that hold it, iq_dec turns them into its 16 values v (int8, in order) and
// its S, iq_d gives D. The codebooks (gw_iq_tables.h) are device arrays the host fills once per device (gw_g_set_iq).
//
// Device layouts: the file's fields, reordered so that every field a half-group reads is one aligned dword, the fp16 d
// moved to the end, 2 bytes of padding (IQ4_XS: 8); bytes per super-block (file: device)
//   IQ2_XXS  66: 68   +0 8 x (u32 grid indices a0, u32 signs + scale a1)   +64 d
//   IQ2_XS   74: 76   +0 u16 qs[32] (9-bit index, 7 sign bits)  +64 scales[8]  +72 d
//   IQ2_S    82: 84   +0 qs[32]  +32 signs[32]  +64 qh[8]  +72 scales[8]  +80 d
//   IQ3_XXS  98: 100  +0 qs[64]  +64 u32 a[8] (signs + scale)  +96 d
//   IQ3_S   110: 112  +0 qs[64]  +64 signs[32]  +96 qh[8]  +104 scales[4]  +108 d
//   IQ1_S    50: 52   +0 qs[32]  +32 u16 qh[8]  +48 d
//   IQ1_M    56: 56   the file's (qs[32], qh[16], u16 sc[4] with d in their top nibbles)
//   IQ4_XS  136: 144  +0 qs[128] (nibbles)  +128 int8 S = ls - 32 per group of 32  +136 D (fp32)
// and the IQ3 repack (RqModelOpts.repack, iquants.h:101-107): IQ3_XXS / IQ3_S as 4-bit codes n = e | (v < 0) << 3 (e the
// magnitude's index: |v| = 2 e + 1, IQ3_XXS 4, 12, .., 52, 62) in IQ4_XS's layout, S = 2 ls + 1, D as the base type's:
//   IQ3_XXS_R, IQ3_S_R  98 / 110: 144
#pragma once

// the codebooks, value j of an entry in its byte j; IQ1's as v = 8 grid + 1 ([0]) and 8 grid - 1 ([1]), its two deltas
__device__ uint64_t gw_iq2xxs_g[256], gw_iq2xs_g[512], gw_iq2s_g[1024], gw_iq1s_g[2][2048];
__device__ uint32_t gw_iq3xxs_g[256], gw_iq3s_g[512];

template <int TYPE>
struct IqCb {
    static constexpr bool cb = TYPE == GW_IQ2_XXS || TYPE == GW_IQ2_XS || TYPE == GW_IQ2_S || TYPE == GW_IQ3_XXS ||
                               TYPE == GW_IQ3_S || TYPE == GW_IQ1_S || TYPE == GW_IQ1_M;
    static constexpr bool nib = TYPE == GW_IQ4_XS || TYPE == GW_IQ3_XXS_R || TYPE == GW_IQ3_S_R; // (4-bit codes)
    static constexpr bool iform = cb || nib; // (the integer-form types: no Σx term)
};

// the bytes of one half-group's share of a super-block (fields as iq_raw documents per type)
struct IqRaw {
    uint32_t a, b, c, d;
    uint32_t e;
};

// sign byte -> 0xff in each byte whose value is negative (4 values per call: nibble n, bit j = value j)
__device__ __forceinline__ uint32_t iq_sm(uint32_t n) { return ((n * 0x00204081u) & 0x01010101u) * 0xffu; }
// 4 unsigned byte values g (each 1 .. 62) negated where m is 0xff: (g ^ m) + 1 there, no carry between bytes
__device__ __forceinline__ uint32_t iq_neg(uint32_t g, uint32_t m) { return (g ^ m) + (m & 0x01010101u); }
// 7 stored sign bits completed by the parity bit (iquants.h:9, :197)
__device__ __forceinline__ uint32_t iq_ks(uint32_t s7) { return s7 | (uint32_t)(__builtin_popcount(s7) & 1) << 7; }
// two chunks of 8 (grid entries as bytes, their sign bytes) -> 16 int8 values
__device__ __forceinline__ int4 iq_pair8(uint64_t e0, uint64_t e1, uint32_t s0, uint32_t s1) {
    return make_int4((int)iq_neg((uint32_t)e0, iq_sm(s0 & 15u)), (int)iq_neg((uint32_t)(e0 >> 32), iq_sm(s0 >> 4)),
                     (int)iq_neg((uint32_t)e1, iq_sm(s1 & 15u)), (int)iq_neg((uint32_t)(e1 >> 32), iq_sm(s1 >> 4)));
}

// the 4-bit code tables, value of code n in byte n: IQ4_XS's (ggml's kvalues_iq4nl, iq_grids.h:1082), the repacked
// IQ3 types' (iq_r_value, iquants.h:109-114: +m for n < 8, -m for n | 8)
constexpr int8_t gw_kv_iq4nl_c[16] = { -127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113 };
constexpr int8_t gw_kv_iq3xxs_r[16] = { 4, 12, 20, 28, 36, 44, 52, 62, -4, -12, -20, -28, -36, -44, -52, -62 };
constexpr int8_t gw_kv_iq3s_r[16] = { 1, 3, 5, 7, 9, 11, 13, 15, -1, -3, -5, -7, -9, -11, -13, -15 };
template <int TYPE>
constexpr uint32_t iq4_tw(int k) {
    const int8_t *t = TYPE == GW_IQ3_XXS_R ? gw_kv_iq3xxs_r : TYPE == GW_IQ3_S_R ? gw_kv_iq3s_r : gw_kv_iq4nl_c;
    return (uint32_t)(uint8_t)t[4 * k] | (uint32_t)(uint8_t)t[4 * k + 1] << 8 | (uint32_t)(uint8_t)t[4 * k + 2] << 16 |
           (uint32_t)(uint8_t)t[4 * k + 3] << 24;
}
// 4 codes (0 .. 15, one per byte) -> their values: bytes 0 .. 7 of the table by one v_perm, 8 .. 15 by another, bit 3
// choosing
template <int TYPE>
__device__ __forceinline__ uint32_t iq4_lut(uint32_t n) {
    constexpr uint32_t t0 = iq4_tw<TYPE>(0), t1 = iq4_tw<TYPE>(1), t2 = iq4_tw<TYPE>(2), t3 = iq4_tw<TYPE>(3);
    const uint32_t s = n & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(t1, t0, s), hi = __builtin_amdgcn_perm(t3, t2, s);
    const uint32_t m = ((n >> 3) & 0x01010101u) * 0xffu;
    return (hi & m) | (lo & ~m);
}

// the loads of half-group hg (values 16 hg .. 16 hg + 15; group ib = hg / 2) of super-block b
template <int TYPE>
__device__ __forceinline__ IqRaw iq_raw(const uint8_t *b, int hg) {
    const int ib = hg >> 1, h = hg & 1;
    auto w = [&](int o) -> uint32_t { return *(const uint32_t *)(b + o); };
    IqRaw r = { 0u, 0u, 0u, 0u, 0u };
    if constexpr (TYPE == GW_IQ2_XXS) { // a0, a1 of the group
        r.a = w(8 * ib);
        r.b = w(8 * ib + 4);
    } else if constexpr (TYPE == GW_IQ2_XS) { // qs of chunks 2h, 2h + 1; the scale byte's dword
        r.a = w(8 * ib + 4 * h);
        r.b = w(64 + 4 * (ib >> 2));
    } else if constexpr (TYPE == GW_IQ2_S) { // qs, signs of the group's 4 chunks; qh's and the scales' dwords
        r.a = w(4 * ib);
        r.b = w(32 + 4 * ib);
        r.c = w(64 + 4 * (ib >> 2));
        r.d = w(72 + 4 * (ib >> 2));
    } else if constexpr (TYPE == GW_IQ3_XXS) { // the half-group's 4 indices; a of the group
        r.a = w(8 * ib + 4 * h);
        r.b = w(64 + 4 * ib);
    } else if constexpr (TYPE == GW_IQ3_S) { // the 4 indices' low bytes; the group's sign bytes; qh's dword; the scales
        r.a = w(8 * ib + 4 * h);
        r.b = w(64 + 4 * ib);
        r.c = w(96 + 4 * (ib >> 2));
        r.d = w(104);
    } else if constexpr (TYPE == GW_IQ1_S) { // the group's 4 low index bytes; qh[ib]'s dword
        r.a = w(4 * ib);
        r.b = w(32 + 4 * (ib >> 1));
    } else if constexpr (TYPE == GW_IQ1_M) { // the low index bytes; qh byte 2 ib + h's dword; sc[ib / 2]'s dword
        r.a = w(4 * ib);
        r.b = w(32 + 4 * (ib >> 1));
        r.c = w(48 + 4 * (ib >> 2));
    } else if constexpr (IqCb<TYPE>::nib) { // the group's 16 nibble bytes; its S's dword
        const uint4 q = *(const uint4 *)(b + 16 * ib);
        r.a = q.x;
        r.b = q.y;
        r.c = q.z;
        r.d = q.w;
        r.e = w(128 + 4 * (ib >> 2));
    }
    return r;
}

// half-group hg's 16 values v (int8, in order) and its scale S, from its loads (iquants.h:8-32's formats: the
// reference's dequantization is (D S) v of these, iquants.h:33-47)
template <int TYPE>
__device__ __forceinline__ void iq_dec(const IqRaw &r, int hg, int4 &v, int &S) {
    const int ib = hg >> 1, h = hg & 1;
    if constexpr (TYPE == GW_IQ2_XXS) { // chunk l: index byte l of a0, signs ks(a1 >> 7 l), ls = a1 >> 28 (S = 2 ls + 1)
        const uint64_t e0 = gw_iq2xxs_g[(r.a >> 16 * h) & 255u], e1 = gw_iq2xxs_g[(r.a >> (16 * h + 8)) & 255u];
        v = iq_pair8(e0, e1, iq_ks((r.b >> 14 * h) & 127u), iq_ks((r.b >> (14 * h + 7)) & 127u));
        S = 2 * (int)(r.b >> 28) + 1;
    } else if constexpr (TYPE == GW_IQ2_XS) { // qs: 9-bit index, 7 sign bits; the half's scale nibble of scales[ib]
        const uint64_t e0 = gw_iq2xs_g[r.a & 511u], e1 = gw_iq2xs_g[(r.a >> 16) & 511u];
        v = iq_pair8(e0, e1, iq_ks((r.a >> 9) & 127u), iq_ks((r.a >> 25) & 127u));
        S = 2 * (int)((r.b >> (8 * (ib & 3) + 4 * h)) & 15u) + 1;
    } else if constexpr (TYPE == GW_IQ2_S) { // index = qs | bits 2 l, 2 l + 1 of qh[ib] << 8; raw sign bytes
        const uint32_t q = r.a >> 16 * h, qh = (r.c >> 8 * (ib & 3)) >> 4 * h, sg = r.b >> 16 * h;
        const uint64_t e0 = gw_iq2s_g[(q & 255u) | (qh & 3u) << 8], e1 = gw_iq2s_g[((q >> 8) & 255u) | ((qh >> 2) & 3u) << 8];
        v = iq_pair8(e0, e1, sg & 255u, (sg >> 8) & 255u);
        S = 2 * (int)((r.d >> (8 * (ib & 3) + 4 * h)) & 15u) + 1;
    } else if constexpr (TYPE == GW_IQ3_XXS) { // step t: 4 values of grid[qs byte t]; chunk signs ks(a >> 7 l)
        const uint32_t s0 = iq_ks((r.b >> 14 * h) & 127u), s1 = iq_ks((r.b >> (14 * h + 7)) & 127u);
        v = make_int4((int)iq_neg(gw_iq3xxs_g[r.a & 255u], iq_sm(s0 & 15u)), (int)iq_neg(gw_iq3xxs_g[(r.a >> 8) & 255u], iq_sm(s0 >> 4)),
                      (int)iq_neg(gw_iq3xxs_g[(r.a >> 16) & 255u], iq_sm(s1 & 15u)), (int)iq_neg(gw_iq3xxs_g[r.a >> 24], iq_sm(s1 >> 4)));
        S = 2 * (int)(r.b >> 28) + 1;
    } else if constexpr (TYPE == GW_IQ3_S) { // step t: index qs byte t | bit 4 h + t of qh[ib] << 8; raw sign bytes
        const uint32_t qh = (r.c >> (8 * (ib & 3) + 4 * h)) & 15u, sg = r.b >> 16 * h;
        const uint32_t s0 = sg & 255u, s1 = (sg >> 8) & 255u;
        v = make_int4((int)iq_neg(gw_iq3s_g[(r.a & 255u) | (qh & 1u) << 8], iq_sm(s0 & 15u)),
                      (int)iq_neg(gw_iq3s_g[((r.a >> 8) & 255u) | ((qh >> 1) & 1u) << 8], iq_sm(s0 >> 4)),
                      (int)iq_neg(gw_iq3s_g[((r.a >> 16) & 255u) | ((qh >> 2) & 1u) << 8], iq_sm(s1 & 15u)),
                      (int)iq_neg(gw_iq3s_g[(r.a >> 24) | ((qh >> 3) & 1u) << 8], iq_sm(s1 >> 4)));
        S = 2 * (int)((r.d >> 4 * ib) & 15u) + 1;
    } else if constexpr (TYPE == GW_IQ1_S) { // index = qs | 3 bits 3 l of qh << 8; the delta's sign and S from qh
        const uint32_t q = r.a >> 16 * h, qh = (r.b >> 16 * (ib & 1)) & 0xffffu, n = qh >> 15;
        const uint64_t e0 = gw_iq1s_g[n][(q & 255u) | ((qh >> 6 * h) & 7u) << 8];
        const uint64_t e1 = gw_iq1s_g[n][((q >> 8) & 255u) | ((qh >> (6 * h + 3)) & 7u) << 8];
        v = make_int4((int)(uint32_t)e0, (int)(uint32_t)(e0 >> 32), (int)(uint32_t)e1, (int)(uint32_t)(e1 >> 32));
        S = 2 * (int)((qh >> 12) & 7u) + 1;
    } else if constexpr (TYPE == GW_IQ1_M) { // chunk 2 h + c: index bits 8 .. 10 and the delta's sign in nibble c of
                                             // qh byte 2 ib + h; the 3-bit scale of half h in sc[ib / 2]
        const uint32_t q = r.a >> 16 * h, qb = (r.b >> (16 * (ib & 1) + 8 * h)) & 255u;
        const uint64_t e0 = gw_iq1s_g[(qb >> 3) & 1u][(q & 255u) | (qb & 7u) << 8];
        const uint64_t e1 = gw_iq1s_g[qb >> 7][((q >> 8) & 255u) | ((qb >> 4) & 7u) << 8];
        v = make_int4((int)(uint32_t)e0, (int)(uint32_t)(e0 >> 32), (int)(uint32_t)e1, (int)(uint32_t)(e1 >> 32));
        const uint32_t sc = (r.c >> 16 * ((ib >> 1) & 1)) & 0xffffu;
        S = 2 * (int)((sc >> (6 * (ib & 1) + 3 * h)) & 7u) + 1;
    } else if constexpr (IqCb<TYPE>::nib) { // nibble h of the group's 16 bytes: codes -> the type's values; S as stored
        const uint32_t sh = 4u * (uint32_t)h;
        v = make_int4((int)iq4_lut<TYPE>((r.a >> sh) & 0x0f0f0f0fu), (int)iq4_lut<TYPE>((r.b >> sh) & 0x0f0f0f0fu),
                      (int)iq4_lut<TYPE>((r.c >> sh) & 0x0f0f0f0fu), (int)iq4_lut<TYPE>((r.d >> sh) & 0x0f0f0f0fu));
        S = (int)(int8_t)(r.e >> 8 * (ib & 3));
    }
}

// where a super-block's d lies (the dword at this offset; IQ1_M: the two at 48, its scale words)
template <int TYPE>
constexpr int iq_d_off() {
    return TYPE == GW_IQ2_XXS ? 64 : TYPE == GW_IQ2_XS ? 72 : TYPE == GW_IQ2_S ? 80 : TYPE == GW_IQ3_XXS ? 96
         : TYPE == GW_IQ3_S ? 108 : TYPE == GW_IQ1_S ? 48 : TYPE == GW_IQ1_M ? 48 : 136;
}
// D from those dwords (fp32, exact: the fp16 d times the type's constant factor, iquants.h:178-183)
template <int TYPE>
__device__ __forceinline__ float iq_d_raw(uint32_t w0, uint32_t w1) {
    auto h16 = [](uint32_t x) -> float { return __half2float(__ushort_as_half((uint16_t)(x & 0xffffu))); };
    if constexpr (TYPE == GW_IQ2_XXS || TYPE == GW_IQ2_XS || TYPE == GW_IQ2_S || TYPE == GW_IQ1_S) return h16(w0) * 0.125f;
    else if constexpr (TYPE == GW_IQ3_XXS) return h16(w0) * 0.25f;
    else if constexpr (TYPE == GW_IQ3_S) return h16(w0);
    else if constexpr (TYPE == GW_IQ1_M) { // (d in the top nibbles of sc[0..3], iquants.h:200-205)
        const uint32_t d = (w0 >> 12 & 0x000fu) | (w0 >> 24 & 0x00f0u) | (w1 >> 4 & 0x0f00u) | (w1 >> 16 & 0xf000u);
        return h16(d) * 0.125f;
    } else return __uint_as_float(w0); // IQ4_XS, the repacked IQ3 types
}
template <int TYPE>
__device__ __forceinline__ float iq_d(const uint8_t *b) {
    const uint32_t *p = (const uint32_t *)(b + iq_d_off<TYPE>());
    return iq_d_raw<TYPE>(p[0], TYPE == GW_IQ1_M ? p[1] : 0u);
}

// the whole half-group from memory
template <int TYPE>
__device__ __forceinline__ void iq_half(const uint8_t *b, int hg, int4 &v, int &S) {
    iq_dec<TYPE>(iq_raw<TYPE>(b, hg), hg, v, S);
}
