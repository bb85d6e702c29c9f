// Bit-exact activation quantizers on gfx950.
//
// The library is compiled with -ffp-contract=off and every float step below
// is one IEEE operation with round-to-nearest-even, so quants, scales and
// group sums equal the reference's bit for bit:
//   Q8_K: reference src/kernels.c:561-595 (+ nearest_int, 528-533)
//   Q8_0: reference src/kernels_avx2.c:594-645 (the SIMD quantizer x86
//         production dispatches to; reference kernels.c:536-541)
//   F16 : reference src/backend.c:19-27 via kernels.c:124-176
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sihip {

// ---- IEEE binary16 ------------------------------------------------------

__device__ inline float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// RNE narrowing done in integer arithmetic so the result does not depend on
// the hardware's fp16 denormal mode. Used for the per-block Q8_0 scale.
__device__ inline uint16_t f32_to_f16_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) {
        if (a == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
        uint32_t m = (a >> 13) & 0x3ffu;
        if (m == 0) m = 1;
        return (uint16_t)(sign | 0x7c00u | 0x200u | m);
    }
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (a < 0x38800000u) {
        const int e = (int)(a >> 23) - 127;
        if (e < -25) return (uint16_t)sign;
        const uint32_t mant = (a & 0x7fffffu) | 0x800000u;
        const int shift = -(e + 1);
        uint32_t m = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (m & 1u))) m++;
        return (uint16_t)(sign | m);
    }
    uint32_t r = a - 0x38000000u;
    r += 0xfffu + ((r >> 13) & 1u);
    return (uint16_t)(sign | (r >> 13));
}

// ---- Q8_K -----------------------------------------------------------------

__device__ inline int nearest_int_magic(float v) {
    const float t = __fadd_rn(v, 12582912.0f);
    return (int)(__float_as_uint(t) & 0x7fffffu) - 0x400000;
}

// DPP row permutations (within 16-lane rows): quad_perm [1,0,3,2],
// quad_perm [2,3,0,1], row_half_mirror, row_mirror. Applied in this order they
// pair every lane of a 16-lane row with lanes of every other quarter, so a
// commutative, associative combine ends with the row total in all 16 lanes.
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

__device__ inline uint32_t dpp_u32(uint32_t v, int ctrl) {
    switch (ctrl) {
        case kDppXor1: return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kDppXor1, 0xf, 0xf, false);
        case kDppXor2: return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kDppXor2, 0xf, 0xf, false);
        case kDppHalfMirror:
            return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kDppHalfMirror, 0xf, 0xf, false);
        default: return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, kDppMirror, 0xf, 0xf, false);
    }
}

struct Q8KRow {
    uint4 q;     // quants of this lane's 16 elements
    float d;     // block scale
    int gsum;    // sum of those 16 quants (= the block's bsums[lane16])
};

// 16 lanes quantize one 256-element block; lane16 holds elements
// 16*lane16 .. 16*lane16+15 (x16). The abs-max key is (|x| bits, 255 - index,
// sign): its maximum is the largest |x| at its first occurrence, exactly the
// reference's "if (ax > amax)" scan; |x| of a non-negative float orders like
// its bit pattern, and NaN never enters (it is never > amax). This is the
// general routine; q8k_block_row16 below takes it for the blocks of a wave
// that its shorter path does not cover.
__device__ inline Q8KRow q8k_block_row16_scan(const float x16[16], int lane16) {
    uint32_t abits = 0, key = 0;
    for (int k = 0; k < 16; k++) {
        const float a = fabsf(x16[k]);
        if (a > __uint_as_float(abits)) {
            abits = __float_as_uint(a);
            key = ((uint32_t)(255 - (16 * lane16 + k)) << 1) | (__float_as_uint(x16[k]) >> 31);
        }
    }
    const int ctrls[4] = {kDppXor1, kDppXor2, kDppHalfMirror, kDppMirror};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t a2 = dpp_u32(abits, ctrls[i]);
        const uint32_t k2 = dpp_u32(key, ctrls[i]);
        if (a2 > abits || (a2 == abits && k2 > key)) { abits = a2; key = k2; }
    }
    Q8KRow r;
    if (abits == 0) {
        r.q = make_uint4(0, 0, 0, 0);
        r.d = 0.0f;
        r.gsum = 0;
        return r;
    }
    const float vmax = __uint_as_float(abits | ((key & 1u) << 31));
    const float iscale = -127.0f / vmax;
    uint32_t w[4] = {0, 0, 0, 0};
    int s = 0;
#pragma unroll
    for (int k = 0; k < 16; k++) {
        int v = nearest_int_magic(__fmul_rn(iscale, x16[k]));
        v = v < 127 ? v : 127;
        s += (int)(int8_t)(uint8_t)(v & 0xff);
        w[k >> 2] |= (uint32_t)(v & 0xff) << (8 * (k & 3));
    }
    r.q = make_uint4(w[0], w[1], w[2], w[3]);
    r.d = 1.0f / iscale;
    r.gsum = s;
    return r;
}

// The same block quantization (bit for bit) with fewer instructions, for
// blocks whose 16 elements of every lane are finite and whose lanes do not
// hold both +a and -a for their largest |x| = a; when any block of the
// wave misses that, the whole wave takes q8k_block_row16_scan.
//   abs-max: the largest positive value is the signed integer maximum of
//   the bit patterns, the largest-magnitude negative one the unsigned
//   maximum; the larger magnitude of the two is the lane's |x| maximum,
//   and its sign is the sign at the lane's first occurrence unless both
//   signs reach it. Across the 16 lanes the lowest lane with the block's
//   maximum has its first occurrence (lane16 holds the lower indices).
//   quants: with every element finite, |iscale * x| rounds to at most 127
//   (or is +-inf or 0 * inf = NaN when -127 / vmax overflows), so
//   t = iscale * x + 12582912 lies in [2^23, 2^24), or is +-inf or a NaN
//   without payload, and the reference's quant (t's low 23 bits - 2^22,
//   capped at 127, taken as a byte) is the low byte of t's bits: the cap
//   never applies. The bytes are packed with two permutes and an or, and
//   each packed word is summed with one 4-way byte dot product.
__device__ inline Q8KRow q8k_block_row16(const float x16[16], int lane16) {
    int pmax = (int)__float_as_uint(x16[0]);
    uint32_t nmax = __float_as_uint(x16[0]);
#pragma unroll
    for (int k = 1; k < 16; k++) {
        const uint32_t b = __float_as_uint(x16[k]);
        pmax = (int)b > pmax ? (int)b : pmax;
        nmax = b > nmax ? b : nmax;
    }
    const uint32_t pa = pmax >= 0 ? (uint32_t)pmax : 0u;              // largest x >= +0
    const uint32_t na = nmax >= 0x80000000u ? nmax & 0x7fffffffu : 0u;  // largest |x| of x <= -0
    const uint32_t lane_abits = pa > na ? pa : na;
    const bool general = lane_abits >= 0x7f800000u || (pa == na && pa != 0u);
    if (__builtin_amdgcn_ballot_w64(general) != 0) return q8k_block_row16_scan(x16, lane16);
    const int ctrls[4] = {kDppXor1, kDppXor2, kDppHalfMirror, kDppMirror};
    uint32_t abits = lane_abits;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t a2 = dpp_u32(abits, ctrls[i]);
        abits = a2 > abits ? a2 : abits;
    }
    // the lowest lane holding the maximum, and its sign
    uint32_t key = lane_abits == abits ? ((uint32_t)(15 - lane16) << 1) | (na > pa ? 1u : 0u) : 0u;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t k2 = dpp_u32(key, ctrls[i]);
        key = k2 > key ? k2 : key;
    }
    Q8KRow r;
    if (abits == 0) {
        r.q = make_uint4(0, 0, 0, 0);
        r.d = 0.0f;
        r.gsum = 0;
        return r;
    }
    const float vmax = __uint_as_float(abits | ((key & 1u) << 31));
    const float iscale = -127.0f / vmax;
    uint32_t w[4];
    int s = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        uint32_t t[4];
#pragma unroll
        for (int k = 0; k < 4; k++)
            t[k] = __float_as_uint(__fadd_rn(__fmul_rn(iscale, x16[4 * j + k]), 12582912.0f));
        // bytes 0 of t[0], t[1] into bytes 0, 1; of t[2], t[3] into 2, 3
        const uint32_t lo = __builtin_amdgcn_perm(t[1], t[0], 0x0c0c0400u);
        const uint32_t hi = __builtin_amdgcn_perm(t[3], t[2], 0x04000c0cu);
        w[j] = lo | hi;
        s = __builtin_amdgcn_sdot4((int)w[j], 0x01010101, s, false);
    }
    r.q = make_uint4(w[0], w[1], w[2], w[3]);
    r.d = 1.0f / iscale;
    r.gsum = s;
    return r;
}

// ---- Q8_0 -----------------------------------------------------------------

__device__ inline float vmaxsel(float a, float b) { return a > b ? a : b; }

// x86 cvtps_epi32 of an already rounded value: NaN or out of range gives
// INT32_MIN, which the saturating packs then turn into -128.
__device__ inline int cvt_i32_indef(float r) {
    if (!(r >= -2147483648.0f && r < 2147483648.0f)) return (int)0x80000000u;
    return (int)r;
}

// One thread quantizes one 32-block. The abs-max follows the SIMD
// reduction tree (per-lane max over 4 vectors, then 8 -> 4 -> 2 -> 1 with
// maxps operand order), which only matters for NaN inputs.
struct Q80Block {
    uint16_t dbits;
    float d;          // f32 value of the stored f16 scale
    int sum;          // sum of the 32 quants
    uint32_t q[8];    // quants, byte k of q[t] = element 4t+k
};

__device__ inline Q80Block q80_block_v(const float (&v)[32]) {
    float lane[8];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        float m = fabsf(v[k]);
        m = vmaxsel(m, fabsf(v[8 + k]));
        m = vmaxsel(m, fabsf(v[16 + k]));
        m = vmaxsel(m, fabsf(v[24 + k]));
        lane[k] = m;
    }
    float m4[4], m2[2];
#pragma unroll
    for (int k = 0; k < 4; k++) m4[k] = vmaxsel(lane[4 + k], lane[k]);
#pragma unroll
    for (int k = 0; k < 2; k++) m2[k] = vmaxsel(m4[k], m4[k + 2]);
    const float mx = vmaxsel(m2[0], m2[1]);
    Q80Block b;
    b.dbits = f32_to_f16_bits(mx / 127.0f);
    b.d = f16_bits_to_f32(b.dbits);
    const float id = (mx != 0.0f) ? 127.0f / mx : 0.0f;
    int s = 0;
#pragma unroll
    for (int t = 0; t < 8; t++) {
        uint32_t w = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float r = __builtin_rintf(__fmul_rn(v[4 * t + k], id));
            int q = cvt_i32_indef(r);
            q = q > 127 ? 127 : (q < -128 ? -128 : q);
            s += q;
            w |= (uint32_t)(q & 0xff) << (8 * k);
        }
        b.q[t] = w;
    }
    b.sum = s;
    return b;
}

__device__ inline void q80_load(const float *x, float (&v)[32]) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 t = reinterpret_cast<const float4 *>(x)[i];
        v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
}

__device__ inline Q80Block q80_block(const float *x) {
    float v[32];
    q80_load(x, v);
    return q80_block_v(v);
}

// The portable scalar Q8_0 quantizer (reference src/kernels.c:542-558),
// which the reference selects instead of the SIMD one when SI_SCALAR is set
// (kernels.c:80-83): amax by the running comparison amax > |v| ? amax : |v|
// in element order, d = amax / 127 (then stored as f16), id = 1 / d (0 for
// d == 0) and q = roundf(x * id), halves away from zero. |x * id| stays
// within 127 (plus rounding), so the clamp below never changes a value; it
// only keeps the conversion defined.
__device__ inline Q80Block q80_block_scalar_v(const float (&v)[32]) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) {
        const float a = fabsf(v[j]);
        amax = amax > a ? amax : a;
    }
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    Q80Block b;
    b.dbits = f32_to_f16_bits(d);
    b.d = f16_bits_to_f32(b.dbits);
    int s = 0;
#pragma unroll
    for (int t = 0; t < 8; t++) {
        uint32_t w = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float r = __builtin_roundf(__fmul_rn(v[4 * t + k], id));
            int q = cvt_i32_indef(r);
            q = q > 127 ? 127 : (q < -128 ? -128 : q);
            s += q;
            w |= (uint32_t)(q & 0xff) << (8 * k);
        }
        b.q[t] = w;
    }
    b.sum = s;
    return b;
}

__device__ inline Q80Block q80_block_scalar(const float *x) {
    float v[32];
    q80_load(x, v);
    return q80_block_scalar_v(v);
}

// q80_block_v spread over the 4 lanes of a quad (lanes 4i .. 4i+3 of a
// wave, all active): lane j of the quad holds elements 8i + 2j and
// 8i + 2j + 1 (i = 0..3), which are lanes 2j and 2j + 1 of the four 8-float
// vectors the abs-max runs over, so those lanes' maxima are the quad lane's
// own; the rest of the tree runs, in q80_block_v's order, in every lane on
// the 8 values broadcast from the quad. Quants stay with their lanes:
// q2[i] holds elements 8i + 2j (low byte) and 8i + 2j + 1. The sum is the
// quad's total.
struct Q80Quad {
    uint16_t dbits;
    float d;
    int sum;
    uint32_t q2[4];
};

__device__ inline void q80_quad_load(const float *blk, int j, float2 (&t)[4]) {
#pragma unroll
    for (int i = 0; i < 4; i++) t[i] = *reinterpret_cast<const float2 *>(blk + 8 * i + 2 * j);
}

template <int J>
__device__ inline float quad_bcast(float v) {  // quad_perm [J, J, J, J]
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), J * 0x55, 0xf, 0xf, false));
}

__device__ inline Q80Quad q80_quad_v(const float2 (&t)[4]) {
    float a0 = fabsf(t[0].x), a1 = fabsf(t[0].y);
#pragma unroll
    for (int i = 1; i < 4; i++) {
        a0 = vmaxsel(a0, fabsf(t[i].x));
        a1 = vmaxsel(a1, fabsf(t[i].y));
    }
    const float lane[8] = {quad_bcast<0>(a0), quad_bcast<0>(a1), quad_bcast<1>(a0), quad_bcast<1>(a1),
                           quad_bcast<2>(a0), quad_bcast<2>(a1), quad_bcast<3>(a0), quad_bcast<3>(a1)};
    float m4[4], m2[2];
#pragma unroll
    for (int k = 0; k < 4; k++) m4[k] = vmaxsel(lane[4 + k], lane[k]);
#pragma unroll
    for (int k = 0; k < 2; k++) m2[k] = vmaxsel(m4[k], m4[k + 2]);
    const float mx = vmaxsel(m2[0], m2[1]);
    Q80Quad b;
    b.dbits = f32_to_f16_bits(mx / 127.0f);
    b.d = f16_bits_to_f32(b.dbits);
    const float id = (mx != 0.0f) ? 127.0f / mx : 0.0f;
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float e[2] = {t[i].x, t[i].y};
        uint32_t w = 0;
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const float r = __builtin_rintf(__fmul_rn(e[k], id));
            int q = cvt_i32_indef(r);
            q = q > 127 ? 127 : (q < -128 ? -128 : q);
            s += q;
            w |= (uint32_t)(q & 0xff) << (8 * k);
        }
        b.q2[i] = w;
    }
    s += __builtin_amdgcn_mov_dpp(s, kDppXor1, 0xf, 0xf, false);
    s += __builtin_amdgcn_mov_dpp(s, kDppXor2, 0xf, 0xf, false);
    b.sum = s;
    return b;
}

// The Q8_0 quantizer a launch uses: the SIMD semantics (q80_block), or
// the scalar ones when `scalar` is set (a wave-uniform launch argument).
__device__ inline Q80Block q80_block_sel(const float *x, int scalar) {
    return scalar ? q80_block_scalar(x) : q80_block(x);
}
__device__ inline Q80Block q80_block_sel_v(const float (&v)[32], int scalar) {
    return scalar ? q80_block_scalar_v(v) : q80_block_v(v);
}

}  // namespace sihip
