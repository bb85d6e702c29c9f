// Per-unit load and decode of the planar weight layout (formats.h), shared
// by the gfx950 matvec kernel and its host emulation (tests/emu), so the
// exact same indexing and bit manipulation can be checked on a CPU.
//
// A unit is 32 consecutive elements of one row. load_unit reads its plane
// records; compute_unit decodes them into 8 dwords q[t] (byte k = element
// 4t+k, canonical order) and accumulates the unit's contribution against
// NC activation columns held in LDS (pair format, layout of matvec.h):
//   Q8_K column: int8 qs[n] (unit-major, q8k_lds_unit) | f32 d[n/256] |
//                int16 bsums[n/16]
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

// Load a T of weight-plane data from p with the nontemporal hint: weights
// stream through once per launch. Used where one load instruction of a wave
// reads whole consecutive records (64 lanes x T bytes, full lines). Measured
// on a plain 4 GiB read: 6.5 TB/s with the hint against 6.0 without, at
// two workgroups per CU.
template <typename T>
SIHD inline T ldw(const uint8_t *p) {
#if defined(__HIP_DEVICE_COMPILE__)
    if constexpr (sizeof(T) == 16) {
        typedef unsigned int v4u_t __attribute__((ext_vector_type(4)));
        return __builtin_bit_cast(T, __builtin_nontemporal_load(
                                         reinterpret_cast<const v4u_t *>(__builtin_assume_aligned(p, 16))));
    } else if constexpr (sizeof(T) == 8) {
        typedef unsigned int v2u_t __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(T, __builtin_nontemporal_load(
                                         reinterpret_cast<const v2u_t *>(__builtin_assume_aligned(p, 8))));
    } else if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(T, __builtin_nontemporal_load(
                                         reinterpret_cast<const unsigned int *>(__builtin_assume_aligned(p, 4))));
    } else {
        static_assert(sizeof(T) == 2, "weight loads are 2, 4, 8 or 16 bytes");
        return __builtin_bit_cast(T, __builtin_nontemporal_load(
                                         reinterpret_cast<const unsigned short *>(__builtin_assume_aligned(p, 2))));
    }
#else
    return ldp<T>(p);
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

// ---- 32-element formats: one unit per column -----------------------------------

// rec: plane record of this lane's unit
template <uint32_t FMT>
SIHD inline void load_unit(const Planes &P, uint32_t rec, Raw &w) {
    if constexpr (FMT == T_Q4_0) {
        w.a = ldw<U4>(P.p[0] + rec * 16u);
        w.e = ldw<uint16_t>(P.p[1] + rec * 2u);
    } else if constexpr (FMT == T_Q5_0) {
        w.a = ldw<U4>(P.p[0] + rec * 16u);
        w.f = ldw<uint32_t>(P.p[1] + rec * 4u);
        w.e = ldw<uint16_t>(P.p[2] + rec * 2u);
    } else if constexpr (FMT == T_Q8_0) {
        // 32- and 64-byte records read 16 bytes at a time: each load covers
        // part of every line, so the lines must stay cached for the next
        // load (no nontemporal hint: F16 ffn_up 27648 x 5120 took 91 us
        // with it, 56 without)
        w.a = ldp<U4>(P.p[0] + rec * 32u);
        w.b = ldp<U4>(P.p[0] + rec * 32u + 16u);
        w.e = ldw<uint16_t>(P.p[1] + rec * 2u);
    } else {  // F16
        const uint8_t *p = P.p[0] + rec * 64u;
        w.a = ldp<U4>(p); w.b = ldp<U4>(p + 16); w.c = ldp<U4>(p + 32); w.d = ldp<U4>(p + 48);
    }
}

// Accumulate unit u (its LDS position; clamped into the row by the caller)
// into acc[0..NC). lds holds NC activation columns of col_bytes each.
template <uint32_t FMT, int NC>
SIHD inline void compute_unit(const uint8_t *lds, uint32_t col_bytes, uint32_t n, uint32_t u,
                              const Raw &w, float *acc) {
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
    } else {
        // 32-blocks: d_w * d_x * (sum(u * x) - bias * sum(x))
        uint32_t q[8];
        if constexpr (FMT == T_Q8_0) {
            q[0] = w.a.x; q[1] = w.a.y; q[2] = w.a.z; q[3] = w.a.w;
            q[4] = w.b.x; q[5] = w.b.y; q[6] = w.b.z; q[7] = w.b.w;
        } else {
            nib_split(w.a, q);
            if constexpr (FMT == T_Q5_0) add_bit4(q, w.f, 4);
        }
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
    }
}

// ---- K-quants: one super-block per column ------------------------------------------

// LDS byte offset of unit k (elements 32k..32k+31) of super-block b in a Q8_K
// column of nb super-blocks. Unit-major order: the lanes of a wave that read
// unit k of consecutive super-blocks read consecutive 32-byte spans, so
// their 16-byte LDS reads spread over all banks.
SIHD inline uint32_t q8k_lds_unit(uint32_t nb, uint32_t b, uint32_t k) {
    return (k * nb + b) * 32u;
}

struct KRaw {
    U4 a[8];          // 16-byte unit records: Q4_K/Q5_K qs, Q6_K ql
    U2 b[8];          // 8-byte unit records: Q6_K qh, Q3_K/Q2_K low 2 bits
    uint32_t c[8];    // 4-byte unit records: Q5_K qh, Q3_K high bit
    U4 m;             // block record: Q4_K/Q5_K d|dmin + scales, Q6_K/Q2_K scales
    uint32_t e;       // Q6_K/Q3_K d, Q2_K d|dmin
};

// urec: unit-plane record of unit 0 of this lane's super-block (unit k is
// 64 records further per k); brec: its block-plane record.
template <uint32_t FMT>
SIHD inline void load_kblock(const Planes &P, uint32_t urec, uint32_t brec, KRaw &w) {
    for (int k = 0; k < 8; k++) {
        const uint32_t r = urec + 64u * (uint32_t)k;
        if constexpr (FMT == T_Q4_K) w.a[k] = ldw<U4>(P.p[0] + r * 16u);
        if constexpr (FMT == T_Q5_K) {
            w.a[k] = ldw<U4>(P.p[0] + r * 16u);
            w.c[k] = ldw<uint32_t>(P.p[1] + r * 4u);
        }
        if constexpr (FMT == T_Q6_K) {
            w.a[k] = ldw<U4>(P.p[0] + r * 16u);
            w.b[k] = ldw<U2>(P.p[1] + r * 8u);
        }
        if constexpr (FMT == T_Q3_K) {
            w.b[k] = ldw<U2>(P.p[0] + r * 8u);
            w.c[k] = ldw<uint32_t>(P.p[1] + r * 4u);
        }
        if constexpr (FMT == T_Q2_K) w.b[k] = ldw<U2>(P.p[0] + r * 8u);
    }
    if constexpr (FMT == T_Q4_K) w.m = ldw<U4>(P.p[1] + brec * 16u);
    if constexpr (FMT == T_Q5_K) w.m = ldw<U4>(P.p[2] + brec * 16u);
    if constexpr (FMT == T_Q6_K) {
        w.m = ldw<U4>(P.p[2] + brec * 16u);
        w.e = ldw<uint16_t>(P.p[3] + brec * 2u);
    }
    if constexpr (FMT == T_Q3_K) {
        const uint8_t *sc = P.p[2] + brec * 12u;  // 12-byte records: as Q8_0's
        w.m.x = ldp<uint32_t>(sc);
        w.m.y = ldp<uint32_t>(sc + 4);
        w.m.z = ldp<uint32_t>(sc + 8);
        w.e = ldw<uint16_t>(P.p[3] + brec * 2u);
    }
    if constexpr (FMT == T_Q2_K) {
        w.m = ldw<U4>(P.p[1] + brec * 16u);
        w.e = ldw<uint32_t>(P.p[2] + brec * 4u);
    }
}

SIHD inline uint32_t u4_word(const U4 &v, int i) {
    return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

// 6-bit scale and min of sub-block j of Q4_K/Q5_K (reference kernels.c:648-656)
SIHD inline void k4_scale_min(const U4 &m, int j, int &sc, int &mn) {
    if (j < 4) {
        sc = (int)((m.y >> (8 * j)) & 63u);
        mn = (int)((m.z >> (8 * j)) & 63u);
    } else {
        const int jj = j - 4;
        sc = (int)(((m.w >> (8 * jj)) & 15u) | (((m.y >> (8 * jj + 6)) & 3u) << 4));
        mn = (int)(((m.w >> (8 * jj + 4)) & 15u) | (((m.z >> (8 * jj + 6)) & 3u) << 4));
    }
}

// signed 6-bit scale g of Q3_K (reference kernels.c:328-333): low nibble
// from byte g%8 (its high nibble for g >= 8), two high bits from byte
// 8 + g%4 at bit 2*(g/4); minus 32
SIHD inline int k3_scale(const U4 &m, int g) {
    const int lb = g & 7;
    const uint32_t lo = (u4_word(m, lb >> 2) >> (8 * (lb & 3) + (g >= 8 ? 4 : 0))) & 15u;
    const uint32_t hi = (m.z >> (8 * (g & 3) + 2 * (g >> 2))) & 3u;
    return (int)(lo | (hi << 4)) - 32;
}

// Accumulate the super-block (kb: its index in the row, clamped by the
// caller) into acc[0..NC). The integer sums of all 8 units accumulate
// exactly; the block scales are applied once.
template <uint32_t FMT, int NC>
SIHD inline void compute_kblock(const uint8_t *lds, uint32_t col_bytes, uint32_t n, uint32_t kb,
                                const KRaw &w, float *acc) {
    const uint32_t nb = n / 256;
    int isum[NC];
    for (int c = 0; c < NC; c++) isum[c] = 0;
    for (int k = 0; k < 8; k++) {
        uint32_t q[8];
        if constexpr (FMT == T_Q4_K || FMT == T_Q5_K || FMT == T_Q6_K) nib_split(w.a[k], q);
        if constexpr (FMT == T_Q5_K) add_bit4(q, w.c[k], 4);
        if constexpr (FMT == T_Q6_K) two8_split(w.b[k].x, w.b[k].y, q, 4, true);
        if constexpr (FMT == T_Q3_K) {
            two8_split(w.b[k].x, w.b[k].y, q, 0, false);
            add_bit4(q, w.c[k], 2);
        }
        if constexpr (FMT == T_Q2_K) two8_split(w.b[k].x, w.b[k].y, q, 0, false);
        // integer scales of this unit's two 16-groups (2k, 2k+1)
        int s0, s1;
        if constexpr (FMT == T_Q4_K || FMT == T_Q5_K) {
            int mn;
            k4_scale_min(w.m, k, s0, mn);
            s1 = s0;
        } else if constexpr (FMT == T_Q6_K) {
            const uint32_t sw = u4_word(w.m, k >> 1);
            s0 = sbfe8(sw, 16 * (k & 1));
            s1 = sbfe8(sw, 16 * (k & 1) + 8);
        } else if constexpr (FMT == T_Q3_K) {
            s0 = k3_scale(w.m, 2 * k);
            s1 = k3_scale(w.m, 2 * k + 1);
        } else {  // Q2_K: low nibble of scale bytes 2k, 2k+1
            const uint32_t sw = u4_word(w.m, k >> 1) >> (16 * (k & 1));
            s0 = (int)(sw & 15u);
            s1 = (int)((sw >> 8) & 15u);
        }
        for (int c = 0; c < NC; c++) {
            const uint8_t *xp = lds + c * col_bytes + q8k_lds_unit(nb, kb, (uint32_t)k);
            int g1;
            const int g0 = dot8(q, ldp<U4>(xp), ldp<U4>(xp + 16), g1);
            isum[c] += s0 * g0 + s1 * g1;
        }
    }
    // per-block terms: the mins (Q4_K/Q5_K/Q2_K) or the bias of the unsigned
    // quants (Q3_K: 4, Q6_K: 32) against the activation group sums
    uint32_t pair[8];  // packed 16-bit factors of groups (2j, 2j+1)
    for (int j = 0; j < 8; j++) {
        if constexpr (FMT == T_Q4_K || FMT == T_Q5_K) {
            int sc, mn;
            k4_scale_min(w.m, j, sc, mn);
            pair[j] = (uint32_t)mn | ((uint32_t)mn << 16);
        } else if constexpr (FMT == T_Q2_K) {
            const uint32_t sw = u4_word(w.m, j >> 1) >> (16 * (j & 1));
            pair[j] = ((sw >> 4) & 15u) | (((sw >> 12) & 15u) << 16);
        } else if constexpr (FMT == T_Q6_K) {
            const uint32_t sw = u4_word(w.m, j >> 1);
            pair[j] = ((uint32_t)sbfe8(sw, 16 * (j & 1)) & 0xffffu) |
                      ((uint32_t)sbfe8(sw, 16 * (j & 1) + 8) << 16);
        } else {  // Q3_K
            pair[j] = ((uint32_t)k3_scale(w.m, 2 * j) & 0xffffu) |
                      ((uint32_t)k3_scale(w.m, 2 * j + 1) << 16);
        }
    }
    float d, dmin = 0.0f;
    if constexpr (FMT == T_Q4_K || FMT == T_Q5_K) {
        d = half_to_float(w.m.x & 0xffffu);
        dmin = half_to_float(w.m.x >> 16);
    } else if constexpr (FMT == T_Q2_K) {
        d = half_to_float(w.e & 0xffffu);
        dmin = half_to_float(w.e >> 16);
    } else {
        d = half_to_float(w.e);
    }
    for (int c = 0; c < NC; c++) {
        const uint8_t *col = lds + c * col_bytes;
        const U4 bs0 = ldp<U4>(col + n + nb * 4 + kb * 32u);
        const U4 bs1 = ldp<U4>(col + n + nb * 4 + kb * 32u + 16u);
        const uint32_t bsw[8] = {bs0.x, bs0.y, bs0.z, bs0.w, bs1.x, bs1.y, bs1.z, bs1.w};
        int t = 0;
        for (int j = 0; j < 8; j++) t = sdot2_i16(bsw[j], pair[j], t);
        const float dx = ldp<float>(col + n + kb * 4u);
        if constexpr (FMT == T_Q4_K || FMT == T_Q5_K || FMT == T_Q2_K) {
            const float v = fma_f32(-dmin, (float)t, d * (float)isum[c]);  // t = sum m*bsum
            acc[c] = fma_f32(dx, v, acc[c]);
        } else {
            constexpr int bias = (FMT == T_Q6_K) ? 32 : 4;
            acc[c] = fma_f32(d * dx, (float)(isum[c] - bias * t), acc[c]);
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

// ---- dequantization (reference kernels.c:599-817, float semantics) ----------
//
// Weight values of one unit, as the reference dequantizer computes them:
//   Q4_0/Q5_0/Q8_0: (float)q * d                      (q signed: u - 8, u - 16)
//   Q2_K/Q4_K/Q5_K: (d * (float)s) * (float)q - dmin * (float)m
//   Q3_K/Q6_K:      (d * (float)s) * (float)q         (q signed: u - 4, u - 32)
// with s, m the scale and min of the element's 16-group (Q4_K/Q5_K: of the
// unit), each product rounded to f32 (no contraction). The quants come from
// the same decode as the dot products.

// Unit k of the super-block w into out[0..31].
template <uint32_t FMT>
SIHD inline void dequant_kunit(const KRaw &w, int k, float out[32]) {
    uint32_t q[8];
    int s0, s1, m0 = 0, m1 = 0, bias = 0;
    float d, dmin = 0.0f;
    if constexpr (FMT == T_Q4_K || FMT == T_Q5_K) {
        nib_split(w.a[k], q);
        if constexpr (FMT == T_Q5_K) add_bit4(q, w.c[k], 4);
        k4_scale_min(w.m, k, s0, m0);
        s1 = s0;
        m1 = m0;
        d = half_to_float(w.m.x & 0xffffu);
        dmin = half_to_float(w.m.x >> 16);
    } else if constexpr (FMT == T_Q6_K) {
        nib_split(w.a[k], q);
        two8_split(w.b[k].x, w.b[k].y, q, 4, true);
        const uint32_t sw = u4_word(w.m, k >> 1);
        s0 = sbfe8(sw, 16 * (k & 1));
        s1 = sbfe8(sw, 16 * (k & 1) + 8);
        d = half_to_float(w.e & 0xffffu);
        bias = 32;
    } else if constexpr (FMT == T_Q3_K) {
        two8_split(w.b[k].x, w.b[k].y, q, 0, false);
        add_bit4(q, w.c[k], 2);
        s0 = k3_scale(w.m, 2 * k);
        s1 = k3_scale(w.m, 2 * k + 1);
        d = half_to_float(w.e & 0xffffu);
        bias = 4;
    } else {  // Q2_K
        two8_split(w.b[k].x, w.b[k].y, q, 0, false);
        const uint32_t sw = u4_word(w.m, k >> 1) >> (16 * (k & 1));
        s0 = (int)(sw & 15u);
        m0 = (int)((sw >> 4) & 15u);
        s1 = (int)((sw >> 8) & 15u);
        m1 = (int)((sw >> 12) & 15u);
        d = half_to_float(w.e & 0xffffu);
        dmin = half_to_float(w.e >> 16);
    }
    for (int e = 0; e < 32; e++) {
        const int u = (int)((q[e >> 2] >> (8 * (e & 3))) & 0xffu) - bias;
        const float dl = d * (float)(e < 16 ? s0 : s1);
        if constexpr (FMT == T_Q3_K || FMT == T_Q6_K) {
            out[e] = dl * (float)u;
        } else {
            const float ml = dmin * (float)(e < 16 ? m0 : m1);
            out[e] = dl * (float)u - ml;
        }
    }
}

// The 32-element unit w into out[0..31].
template <uint32_t FMT>
SIHD inline void dequant_unit(const Raw &w, float out[32]) {
    if constexpr (FMT == T_F16) {
        const uint32_t v[16] = {w.a.x, w.a.y, w.a.z, w.a.w, w.b.x, w.b.y, w.b.z, w.b.w,
                                w.c.x, w.c.y, w.c.z, w.c.w, w.d.x, w.d.y, w.d.z, w.d.w};
        for (int e = 0; e < 32; e++) out[e] = half_to_float((v[e >> 1] >> (16 * (e & 1))) & 0xffffu);
    } else {
        uint32_t q[8];
        int bias = 0;
        if constexpr (FMT == T_Q8_0) {
            q[0] = w.a.x; q[1] = w.a.y; q[2] = w.a.z; q[3] = w.a.w;
            q[4] = w.b.x; q[5] = w.b.y; q[6] = w.b.z; q[7] = w.b.w;
        } else {
            nib_split(w.a, q);
            if constexpr (FMT == T_Q5_0) add_bit4(q, w.f, 4);
            bias = FMT == T_Q4_0 ? 8 : 16;
        }
        const float d = half_to_float(w.e & 0xffffu);
        for (int e = 0; e < 32; e++) {
            const uint32_t byte = (q[e >> 2] >> (8 * (e & 3))) & 0xffu;
            const int v = FMT == T_Q8_0 ? (int)(int8_t)byte : (int)byte - bias;
            out[e] = (float)v * d;
        }
    }
}

}  // namespace sihip
