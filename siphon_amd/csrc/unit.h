// Per-unit load and decode of the planar weight layout (formats.h), shared
// by the gfx950 matvec kernel and its host emulation (tests/emu), so the
// exact same indexing and bit manipulation can be checked on a CPU.
//
// A unit is 32 consecutive elements of one row. load_unit reads its plane
// records; compute_unit decodes them into 8 dwords q[t] (byte k = element
// 4t+k, canonical order) and accumulates the unit's contribution against
// NC activation columns held in LDS (pair format, layout of matvec.h):
//   Q8_K column: int8 qs[n] | f32 d[n/256] | int16 bsums[n/16]
//   Q8_0 column: int8 qs[n] | f32 d[n/32]  | int32 qsum[n/32]
//   F16  column: f16 h[n]
// Record indices and byte offsets are 32-bit (a plane is < 4 GiB), so the
// device addresses every load as (plane base in SGPRs) + (32-bit VGPR
// offset) + (immediate).
#pragma once

#include <stdint.h>
#include <string.h>

#include "formats.h"

namespace sihip {

struct alignas(16) U4 { uint32_t x, y, z, w; };
struct alignas(8) U2 { uint32_t x, y; };

// ---- portable primitives (one instruction each on gfx950) ----------------

SIHD inline int sdot4_i8(uint32_t a, uint32_t b, int c) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
#else
    for (int k = 0; k < 4; k++) c += (int)(int8_t)(a >> (8 * k)) * (int)(int8_t)(b >> (8 * k));
    return c;
#endif
}

// a.lo*b.lo + a.hi*b.hi + c on signed 16-bit halves
SIHD inline int sdot2_i16(uint32_t a, uint32_t b, int c) {
#if defined(__HIP_DEVICE_COMPILE__)
    typedef short s2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, a), __builtin_bit_cast(s2, b), c, false);
#else
    return c + (int)(int16_t)(a & 0xffffu) * (int)(int16_t)(b & 0xffffu) +
           (int)(int16_t)(a >> 16) * (int)(int16_t)(b >> 16);
#endif
}

// unsigned bit-field extract; width 0 gives 0
SIHD inline uint32_t ubfe(uint32_t v, uint32_t off, uint32_t w) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_ubfe(v, off, w);
#else
    return w ? (v >> off) & ((1u << w) - 1u) : 0u;
#endif
}

// signed 8-bit field extract
SIHD inline int sbfe8(uint32_t v, uint32_t off) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_sbfe((int)v, off, 8);
#else
    return (int)(int8_t)((v >> off) & 0xffu);
#endif
}

SIHD inline float half_to_float(uint32_t h) {
#if defined(__HIP_DEVICE_COMPILE__)
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
#else
    const uint32_t sign = (h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        float v = (float)m * 0x1p-24f;
        memcpy(&bits, &v, 4);
        bits |= sign;
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
#endif
}

// acc + a.lo*b.lo + a.hi*b.hi on f16 pairs
SIHD inline float fdot2_f16(uint32_t a, uint32_t b, float acc) {
#if defined(__HIP_DEVICE_COMPILE__)
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b), acc, false);
#else
    const float p0 = half_to_float(a & 0xffffu) * half_to_float(b & 0xffffu);
    const float p1 = half_to_float(a >> 16) * half_to_float(b >> 16);
    return acc + (p0 + p1);
#endif
}

SIHD inline float fma_f32(float a, float b, float c) { return __builtin_fmaf(a, b, c); }

// Load a T from p. Every call site is naturally aligned for T; on the device
// the typed load lets the compiler emit one load of the full width.
template <typename T>
SIHD inline T ldp(const uint8_t *p) {
#if defined(__HIP_DEVICE_COMPILE__)
    return *reinterpret_cast<const T *>(__builtin_assume_aligned(p, sizeof(T) > 16 ? 16 : sizeof(T)));
#else
    T v;
    memcpy(&v, p, sizeof(T));
    return v;
#endif
}

SIHD inline int dot8(const uint32_t q[8], const U4 &x0, const U4 &x1, int &g1) {
    int g0 = sdot4_i8(q[0], x0.x, 0);
    g0 = sdot4_i8(q[1], x0.y, g0);
    g0 = sdot4_i8(q[2], x0.z, g0);
    g0 = sdot4_i8(q[3], x0.w, g0);
    int h = sdot4_i8(q[4], x1.x, 0);
    h = sdot4_i8(q[5], x1.y, h);
    h = sdot4_i8(q[6], x1.z, h);
    h = sdot4_i8(q[7], x1.w, h);
    g1 = h;
    return g0;
}

// nib16: low nibbles are elements 0..15, high nibbles elements 16..31
SIHD inline void nib_split(const U4 &n, uint32_t q[8]) {
    q[0] = n.x & 0x0F0F0F0Fu; q[1] = n.y & 0x0F0F0F0Fu;
    q[2] = n.z & 0x0F0F0F0Fu; q[3] = n.w & 0x0F0F0F0Fu;
    q[4] = (n.x >> 4) & 0x0F0F0F0Fu; q[5] = (n.y >> 4) & 0x0F0F0F0Fu;
    q[6] = (n.z >> 4) & 0x0F0F0F0Fu; q[7] = (n.w >> 4) & 0x0F0F0F0Fu;
}

// bit4: bit t of every byte, moved to bit position `pos`
SIHD inline void add_bit4(uint32_t q[8], uint32_t hb, int pos) {
    for (int t = 0; t < 8; t++) q[t] |= ((hb >> t) & 0x01010101u) << pos;
}

// two8: 2-bit field t of every byte of h0 (elements 0..15) and h1 (16..31)
SIHD inline void two8_split(uint32_t h0, uint32_t h1, uint32_t q[8], int pos, bool orr) {
    for (int t = 0; t < 4; t++) {
        const uint32_t a = ((h0 >> (2 * t)) & 0x03030303u) << pos;
        const uint32_t b = ((h1 >> (2 * t)) & 0x03030303u) << pos;
        q[t] = orr ? (q[t] | a) : a;
        q[4 + t] = orr ? (q[4 + t] | b) : b;
    }
}

// ---- per-lane constants ------------------------------------------------------

// Everything that depends only on the lane's sub-block index j (0..7) of the
// K-quant super-block, computed once per kernel so the unit loop holds no
// lane-divergent branches.
struct LaneK {
    int j;
    uint32_t k4_hi;                 // Q4_K/Q5_K: j >= 4
    uint32_t sc_sh, sc_w, mn_sh, mn_w, h_sh, h_w;
    uint32_t q3_lsh, q3_hsh0, q3_hsh1;
    uint32_t pair_sh;               // 16 * (j & 1): Q2_K/Q6_K scale byte pair
    uint32_t rec4;                  // byte offset of the dword holding scales 2j, 2j+1
    uint32_t q3rec4;                // Q3_K: dword with the low nibbles of scales 2j, 2j+1
};

SIHD inline LaneK lane_consts(int j) {
    LaneK K;
    K.j = j;
    // 6-bit scale/min of sub-block j (reference kernels.c:648-656):
    //   j < 4: sc = s[j] & 63,             mn = s[j+4] & 63
    //   j >=4: sc = lo4(s[j+4]) | hi2(s[j-4]) << 4, mn = hi4(s[j+4]) | hi2(s[j]) << 4
    const uint32_t jj = (uint32_t)(j & 3);
    K.k4_hi = j >= 4;
    K.sc_sh = 8 * jj;
    K.sc_w = j < 4 ? 6 : 4;
    K.mn_sh = j < 4 ? 8 * jj : 8 * jj + 4;
    K.mn_w = j < 4 ? 6 : 4;
    K.h_sh = 8 * jj + 6;
    K.h_w = j < 4 ? 0 : 2;
    // Q3_K 6-bit scale k for k = 2j, 2j+1 (reference kernels.c:328-333):
    // low nibble from byte k%8 (its high nibble when k >= 8), two high bits
    // from byte 8 + k%4 at bit 2*(k/4)
    const int k0 = 2 * j;
    K.q3_lsh = (uint32_t)(8 * (k0 & 3) + (k0 >= 8 ? 4 : 0));
    K.q3_hsh0 = (uint32_t)(8 * (k0 & 3) + 2 * (k0 >> 2));
    K.q3_hsh1 = (uint32_t)(8 * ((k0 + 1) & 3) + 2 * ((k0 + 1) >> 2));
    K.pair_sh = 16u * (uint32_t)(j & 1);
    K.rec4 = 4u * (uint32_t)(j >> 1);
    K.q3rec4 = 4u * (uint32_t)((j & 3) >> 1);
    return K;
}

// ---- loads -------------------------------------------------------------------

struct Planes {
    const uint8_t *p[4];
};

// Raw plane data of one unit, loaded before any of it is consumed.
struct Raw {
    U4 a, b, c, d;   // unit-plane data (up to 64 bytes)
    U4 m;            // block-plane record fields
    uint32_t e, f;   // small unit-plane fields
};

// ur: unit-plane record index of this lane; br: block-plane record index.
template <uint32_t FMT>
SIHD inline void load_unit(const Planes &P, uint32_t ur, uint32_t br, const LaneK &K, Raw &w) {
    if constexpr (FMT == T_Q4_K) {
        w.a = ldp<U4>(P.p[0] + ur * 16u);
        w.m = ldp<U4>(P.p[1] + br * 16u);
    } else if constexpr (FMT == T_Q5_K) {
        w.a = ldp<U4>(P.p[0] + ur * 16u);
        w.e = ldp<uint32_t>(P.p[1] + ur * 4u);
        w.m = ldp<U4>(P.p[2] + br * 16u);
    } else if constexpr (FMT == T_Q6_K) {
        w.a = ldp<U4>(P.p[0] + ur * 16u);
        const U2 h = ldp<U2>(P.p[1] + ur * 8u);
        w.e = h.x; w.f = h.y;
        w.m.x = ldp<uint32_t>(P.p[2] + br * 16u + K.rec4);  // int8 scales 2j, 2j+1
        w.m.y = ldp<uint16_t>(P.p[3] + br * 2u);
    } else if constexpr (FMT == T_Q3_K) {
        const U2 h = ldp<U2>(P.p[0] + ur * 8u);
        w.e = h.x; w.f = h.y;
        w.m.x = ldp<uint32_t>(P.p[1] + ur * 4u);
        const uint8_t *sc = P.p[2] + br * 12u;
        w.m.y = ldp<uint32_t>(sc + K.q3rec4);  // low nibbles of scales 2j, 2j+1
        w.m.z = ldp<uint32_t>(sc + 8);         // bytes 8..11: high bits
        w.m.w = ldp<uint16_t>(P.p[3] + br * 2u);
    } else if constexpr (FMT == T_Q2_K) {
        const U2 h = ldp<U2>(P.p[0] + ur * 8u);
        w.e = h.x; w.f = h.y;
        w.m.x = ldp<uint32_t>(P.p[1] + br * 16u + K.rec4);  // scale|min bytes 2j, 2j+1
        w.m.y = ldp<uint32_t>(P.p[2] + br * 4u);            // d, dmin
    } else if constexpr (FMT == T_Q4_0) {
        w.a = ldp<U4>(P.p[0] + ur * 16u);
        w.e = ldp<uint16_t>(P.p[1] + ur * 2u);
    } else if constexpr (FMT == T_Q5_0) {
        w.a = ldp<U4>(P.p[0] + ur * 16u);
        w.f = ldp<uint32_t>(P.p[1] + ur * 4u);
        w.e = ldp<uint16_t>(P.p[2] + ur * 2u);
    } else if constexpr (FMT == T_Q8_0) {
        w.a = ldp<U4>(P.p[0] + ur * 32u);
        w.b = ldp<U4>(P.p[0] + ur * 32u + 16u);
        w.e = ldp<uint16_t>(P.p[1] + ur * 2u);
    } else {  // F16
        const uint8_t *p = P.p[0] + ur * 64u;
        w.a = ldp<U4>(p); w.b = ldp<U4>(p + 16); w.c = ldp<U4>(p + 32); w.d = ldp<U4>(p + 48);
    }
}

// ---- decode --------------------------------------------------------------------

// Decoded quants of the unit: unsigned biased values for Q4_0 (0..15),
// Q5_0 (0..31), Q3_K (0..7), Q6_K (0..63); signed for Q8_0; unsigned
// without bias for Q2_K (0..3), Q4_K (0..15), Q5_K (0..31).
template <uint32_t FMT>
SIHD inline void unit_quants(const Raw &w, uint32_t q[8]) {
    if constexpr (FMT == T_Q4_K || FMT == T_Q4_0 || FMT == T_Q5_0 || FMT == T_Q5_K ||
                  FMT == T_Q6_K) {
        nib_split(w.a, q);
    }
    if constexpr (FMT == T_Q5_K) add_bit4(q, w.e, 4);
    if constexpr (FMT == T_Q5_0) add_bit4(q, w.f, 4);
    if constexpr (FMT == T_Q6_K) two8_split(w.e, w.f, q, 4, true);
    if constexpr (FMT == T_Q3_K) {
        two8_split(w.e, w.f, q, 0, false);
        add_bit4(q, w.m.x, 2);
    }
    if constexpr (FMT == T_Q2_K) two8_split(w.e, w.f, q, 0, false);
    if constexpr (FMT == T_Q8_0) {
        q[0] = w.a.x; q[1] = w.a.y; q[2] = w.a.z; q[3] = w.a.w;
        q[4] = w.b.x; q[5] = w.b.y; q[6] = w.b.z; q[7] = w.b.w;
    }
}

// Accumulate unit u into acc[0..NC). lds holds NC activation columns of
// col_bytes each; n is the row length.
template <uint32_t FMT, int NC>
SIHD inline void compute_unit(const uint8_t *lds, uint32_t col_bytes, uint32_t n, uint32_t u,
                              const LaneK &K, const Raw &w, float *acc) {
    if constexpr (FMT == T_F16) {
        const uint32_t wv[16] = {w.a.x, w.a.y, w.a.z, w.a.w, w.b.x, w.b.y, w.b.z, w.b.w,
                                 w.c.x, w.c.y, w.c.z, w.c.w, w.d.x, w.d.y, w.d.z, w.d.w};
        for (int c = 0; c < NC; c++) {
            const uint8_t *xp = lds + c * col_bytes + u * 64u;
            const U4 x0 = ldp<U4>(xp), x1 = ldp<U4>(xp + 16), x2 = ldp<U4>(xp + 32),
                     x3 = ldp<U4>(xp + 48);
            const uint32_t xv[16] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w,
                                     x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w};
            float s = acc[c];
            for (int i = 0; i < 16; i++) s = fdot2_f16(wv[i], xv[i], s);
            acc[c] = s;
        }
        return;
    }
    uint32_t q[8];
    unit_quants<FMT>(w, q);

    if constexpr (FMT == T_Q4_0 || FMT == T_Q5_0 || FMT == T_Q8_0) {
        // 32-blocks: d_w * d_x * (sum(u * x) - bias * sum(x))
        const float dw = half_to_float(w.e);
        const uint32_t nb = n / 32;
        for (int c = 0; c < NC; c++) {
            const uint8_t *col = lds + c * col_bytes;
            int g1;
            const int g0 = dot8(q, ldp<U4>(col + u * 32u), ldp<U4>(col + u * 32u + 16u), g1);
            int isum = g0 + g1;
            if constexpr (FMT == T_Q4_0) isum -= 8 * ldp<int>(col + n + nb * 4 + u * 4u);
            if constexpr (FMT == T_Q5_0) isum -= 16 * ldp<int>(col + n + nb * 4 + u * 4u);
            const float dx = ldp<float>(col + n + u * 4u);
            acc[c] = fma_f32(dw * dx, (float)isum, acc[c]);
        }
        return;
    }

    // K-quants: super-block kb; the unit covers its 16-element groups 2j, 2j+1
    const uint32_t kb = u >> 3;
    const uint32_t nb = n / 256;
    const uint32_t bs_off = n + nb * 4 + kb * 32 + (uint32_t)K.j * 4;
    if constexpr (FMT == T_Q4_K || FMT == T_Q5_K) {
        // one 6-bit scale and min for the whole unit
        const uint32_t s03 = w.m.y, s47 = w.m.z, s811 = w.m.w;
        const uint32_t A = K.k4_hi ? s811 : s03;
        const uint32_t B = K.k4_hi ? s811 : s47;
        const int sc = (int)(ubfe(A, K.sc_sh, K.sc_w) | (ubfe(s03, K.h_sh, K.h_w) << 4));
        const uint32_t mn = ubfe(B, K.mn_sh, K.mn_w) | (ubfe(s47, K.h_sh, K.h_w) << 4);
        const uint32_t mn2 = mn | (mn << 16);
        const float d = half_to_float(w.m.x & 0xffffu);
        const float dmin = half_to_float(w.m.x >> 16);
        for (int c = 0; c < NC; c++) {
            const uint8_t *col = lds + c * col_bytes;
            int g1;
            const int g0 = dot8(q, ldp<U4>(col + u * 32u), ldp<U4>(col + u * 32u + 16u), g1);
            const int isum = sc * (g0 + g1);
            const int imin = sdot2_i16(ldp<uint32_t>(col + bs_off), mn2, 0);  // m*(bs0+bs1)
            const float dx = ldp<float>(col + n + kb * 4);
            const float t = fma_f32(-dmin, (float)imin, d * (float)isum);
            acc[c] = fma_f32(dx, t, acc[c]);
        }
    } else if constexpr (FMT == T_Q2_K) {
        const uint32_t sw = w.m.x >> K.pair_sh;  // bytes: scale|min << 4 of groups 2j, 2j+1
        const int sc0 = (int)(sw & 15u), sc1 = (int)((sw >> 8) & 15u);
        const uint32_t mn2 = ((sw >> 4) & 15u) | (((sw >> 12) & 15u) << 16);
        const float d = half_to_float(w.m.y & 0xffffu);
        const float dmin = half_to_float(w.m.y >> 16);
        for (int c = 0; c < NC; c++) {
            const uint8_t *col = lds + c * col_bytes;
            int g1;
            const int g0 = dot8(q, ldp<U4>(col + u * 32u), ldp<U4>(col + u * 32u + 16u), g1);
            const int isum = sc0 * g0 + sc1 * g1;
            const int imin = sdot2_i16(ldp<uint32_t>(col + bs_off), mn2, 0);
            const float dx = ldp<float>(col + n + kb * 4);
            const float t = fma_f32(-dmin, (float)imin, d * (float)isum);
            acc[c] = fma_f32(dx, t, acc[c]);
        }
    } else {  // Q3_K, Q6_K: sum_g sc_g * (sum(u*x) - bias * bsum_g)
        int sc0, sc1;
        float d;
        if constexpr (FMT == T_Q6_K) {
            sc0 = sbfe8(w.m.x, K.pair_sh);
            sc1 = sbfe8(w.m.x, K.pair_sh + 8);
            d = half_to_float(w.m.y);
        } else {
            sc0 = (int)(ubfe(w.m.y, K.q3_lsh, 4) | (ubfe(w.m.z, K.q3_hsh0, 2) << 4)) - 32;
            sc1 = (int)(ubfe(w.m.y, K.q3_lsh + 8, 4) | (ubfe(w.m.z, K.q3_hsh1, 2) << 4)) - 32;
            d = half_to_float(w.m.w);
        }
        constexpr int bias = (FMT == T_Q6_K) ? 32 : 4;
        const uint32_t sc2 = ((uint32_t)sc0 & 0xffffu) | ((uint32_t)sc1 << 16);
        for (int c = 0; c < NC; c++) {
            const uint8_t *col = lds + c * col_bytes;
            int g1;
            const int g0 = dot8(q, ldp<U4>(col + u * 32u), ldp<U4>(col + u * 32u + 16u), g1);
            const int ib = sdot2_i16(ldp<uint32_t>(col + bs_off), sc2, 0);  // sc0*bs0 + sc1*bs1
            const int isum = sc0 * g0 + sc1 * g1 - bias * ib;
            const float dx = ldp<float>(col + n + kb * 4);
            acc[c] = fma_f32(d * dx, (float)isum, acc[c]);
        }
    }
}

// ---- reduction order ------------------------------------------------------------

// Lane partner of step `k` in the reduction of a G-lane group (G a power of
// two, groups aligned to G): within 16 lanes the DPP patterns quad_perm
// [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror; beyond, xor 16
// and xor 32. Any step pairs a lane with one in the other half of its
// current group, so after log2(G) steps every lane holds the group total.
SIHD inline int reduce_partner(int lane, int k) {
    switch (k) {
        case 0: return lane ^ 1;
        case 1: return lane ^ 2;
        case 2: return (lane & ~7) | (7 - (lane & 7));
        case 3: return (lane & ~15) | (15 - (lane & 15));
        case 4: return lane ^ 16;
        default: return lane ^ 32;
    }
}

}  // namespace sihip
