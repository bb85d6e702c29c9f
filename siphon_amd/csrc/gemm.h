// Prefill GEMM on the matrix cores of gfx950: Y[M x n_out] = X[M x n_in] *
// W^T for K-quant weights, with X quantized per row to Q8_K by the same
// bit-exact quantizer as the matvec path (reference kernels.c:561-595).
//
// Arithmetic (per 256-element super-block c, weight row n, activation row
// m), restating the reference dot (reference kernels.c:349-410 for Q4_K):
//   S[m,n] = sum_j sc_j[n] * sum_{k in unit j} q[n,k] * x[m,k]      (exact int)
//   T[m,n] = sum_g mn_{g/2}[n] * bsum_g[m]                            (exact)
//   y[m,n] += dx[m,c] * d[n,c] * S - dx[m,c] * dmin[n,c] * T
// S runs on v_mfma_i32_32x32x32_i8, one MFMA per 32-element unit. The 6-bit
// unit scale is split as sc = 8 * sh + sl (sh, sl in 0..7) so that both
// weight operands sh * q and sl * q fit in int8 (<= 105): two MFMAs per
// unit accumulate 8 * H + L = S exactly in int32. T runs on one
// v_mfma_f32_32x32x16_f16 per super-block (mins <= 63 and group sums
// |bsum| <= 2032 are exact in f16, and every partial sum stays below 2^24,
// so the f32 result is exact). Only the per-super-block f32 epilogue rounds.
//
// Q2_K (reference kernels.c:249-287) has the same form with 16 groups of
// 16: S[m,n] = sum_g sc_g[n] * sum_{k in g} q[n,k] * x[m,k] with 4-bit
// scales and 2-bit quants, so the weight operand sc * q <= 45 fits int8
// and one MFMA per 32-element unit accumulates S exactly; T takes the
// 4-bit group mins. Q3_K (reference kernels.c:289-347) runs the same way
// with biased operand bytes and a group-sum correction in place of the mins
// (q3_neg_scale below).
//
// MFMA operand layout (gfx950, checked on the device): for the 32x32x32 i8
// and 32x32x16 f16 forms lane l supplies row (l % 32) of A and column
// (l % 32) of B at the k positions of its half h = l / 32; A and B use the
// same k positions, so any consistent assignment of unit elements to the
// (h, slot) pairs is valid. Accumulator register r of lane l holds
// D[8 * (r / 4) + 4 * h + r % 4][l % 32]. Here A is the activation tile
// (rows m) and B the weight tile (columns n), so every lane owns one weight
// row n and its scales.
//
// Element assignment: lane half h takes unit elements 8h..8h+7 and
// 16+8h..16+8h+7. For the weights these are exactly the low and high nibbles
// of bytes 8h..8h+7 of the nib16 unit record (formats.h); the activation
// quants are stored with each unit permuted to [0..7, 16..23, 8..15, 24..31]
// so a lane's 16 bytes are contiguous.
#pragma once

#include "agent.h"
#include "formats.h"
#include "quant.h"
#include "unit.h"

namespace sihip {

typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef int v16i_t __attribute__((ext_vector_type(16)));
typedef float v16f_t __attribute__((ext_vector_type(16)));
typedef _Float16 v8h_t __attribute__((ext_vector_type(8)));
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));

constexpr int kGemmThreads = 256;
constexpr int kGemmBN = 128;                   // weight rows per workgroup (32 per wave)
constexpr int kXRow = 256 + 16;                // LDS bytes per activation row (padded)

// Tile geometry for MT 32-row MFMA tiles per wave along m (BM activation
// rows per workgroup) and the LDS activation buffer of one super-block.
template <int MT>
struct GemmGeo {
    static constexpr int BM = 32 * MT;
    static constexpr int XQBytes = BM * kXRow;       // quant tile
    static constexpr int XDOff = XQBytes;            // f32 dx[BM]
    static constexpr int XBOff = XDOff + BM * 4;     // f16 bsums[BM][16]
    static constexpr int XTile = XBOff + BM * 32;    // one LDS buffer
    static constexpr int XPieces = BM * 16 / kGemmThreads;  // 16-byte quant pieces per thread
    static constexpr int XE = BM * 2 + BM / 4;       // 16-byte pieces of group sums + scales
    static constexpr int XEPieces = (XE + kGemmThreads - 1) / kGemmThreads;
};

// Activation planes written by gemm_quantize_x (Mp = M rounded up to BM;
// rows M..Mp-1 are zero).
struct GemmX {
    int8_t *q;       // [Mp][K] quants, units permuted as described above
    float *d;        // [K/256][Mp] block scales
    _Float16 *bs;    // [K/256][Mp][16] group sums
};

struct GemmArgs {
    const uint8_t *w;    // weights in GEMM order (gemm_layout_kernel)
    int64_t n_out, nb;   // weight rows, super-blocks per row
    int64_t M, Mp;
    GemmX X;
    float *y;
    int64_t ldy;
    int MB, NB;          // workgroup tiles along m and n
    // K slices (S == 1: one workgroup per output tile). S > 1: slice s of
    // a tile covers super-blocks [s * SBK, (s + 1) * SBK); its partial sums
    // go to part[(s * Mp + m) * NB * BN + n] and the last slice of the tile
    // to arrive (counted in cnt[mblk * NB + nblk], zero between launches)
    // adds them in slice order into y and resets the counter.
    int S, SBK;
    float *part;
    uint32_t *cnt;
};

__host__ __device__ inline int64_t gemm_x_bytes(int64_t Mp, int64_t K) {
    return Mp * K + (K / 256) * Mp * 4 + (K / 256) * Mp * 32;
}

// One 16-lane row per Q8_K block of X (row m, super-block c); rows past M
// write zeros. Grid: ceil(Mp * nb / 16) workgroups of 256.
__global__ __launch_bounds__(kGemmThreads) void gemm_quantize_x(const float *x, int64_t ldx,
                                                                int64_t M, int64_t Mp,
                                                                int64_t nb, GemmX X) {
    const int lane16 = threadIdx.x & 15;
    const int64_t blk = (int64_t)blockIdx.x * (kGemmThreads / 16) + (threadIdx.x >> 4);
    if (blk >= Mp * nb) return;  // whole 16-lane rows leave together
    const int64_t m = blk / nb, c = blk % nb;
    const int64_t K = nb * 256;
    Q8KRow r;
    if (m < M) {
        const float4 *src = reinterpret_cast<const float4 *>(x + m * ldx + c * 256 + lane16 * 16);
        float v[16];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 t = src[i];
            v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
        }
        r = q8k_block_row16(v, lane16);
    } else {
        r.q = make_uint4(0, 0, 0, 0);
        r.gsum = 0;
        r.d = 0.0f;
    }
    // this lane holds elements 16 * (lane16 & 1) .. +15 of unit lane16 / 2
    int8_t *unit = X.q + m * K + c * 256 + (lane16 >> 1) * 32;
    const int half = lane16 & 1;
    *reinterpret_cast<uint2 *>(unit + 8 * half) = make_uint2(r.q.x, r.q.y);
    *reinterpret_cast<uint2 *>(unit + 16 + 8 * half) = make_uint2(r.q.z, r.q.w);
    X.bs[(c * Mp + m) * 16 + lane16] = (_Float16)(float)r.gsum;
    if (lane16 == 0) X.d[c * Mp + m] = r.d;
}

// Weight data of one super-block for this lane's row: 8 unit halves and
// the block record.
struct GemmW {
    uint2 u[8];
    uint4 scb;   // Q4_K: sh_0..sh_7 (x, y), sl_0..sl_7 (z, w); Q2_K: sc_0..sc_15; Q3_K: |s_g|
    float2 dd;   // d, dmin
    v8h_t bm;    // mins of groups 8h..8h+7 (this lane's half; Q4_K: unit mins twice)
    uint4 hb[2]; // Q2_K: quant words (q2_word) of units 0..7; Q5_K: hb[0], fifth-bit words
};

// ---- GEMM weight order ---------------------------------------------------------
//
// The matvec layout interleaves the rows of a tile G columns apart, so the
// 32 rows one GEMM wave needs for a super-block are spread over many cache
// lines. Prefill uses a second copy in GEMM order, built on device from the
// matvec planes on first use: for each block of 32 rows and super-block c,
// 5888 contiguous bytes (Q2_K 3840, Q5_K 6912; see gemm_quant_bytes)
//   4 x 1024 B: for q = 0..3 and lane L = 32 h + r (r = row in the block),
//               bytes 16 L .. 16 L + 7 = half h of unit 2q of row r,
//               bytes 16 L + 8 .. 16 L + 15 = half h of unit 2q + 1 of row r
//               (Q3_K: the sign-folded quants u' of q3_neg_scale; Q2_K
//               instead 2048 B, per lane L one q2_word per unit at 32 L)
//   512 B:      per row, the unit scales sc_j = 8 sh_j + sl_j split in
//               bytes: sh_0..sh_7, then sl_0..sl_7 (Q2_K: the 16 group
//               scales, one byte each; Q3_K: |s_g|)
//   256 B:      per row, f32 d and dmin (Q3_K: -d and 0)
//   1024 B:     per lane L, f16 mins of units 4h..4h+3 of row r, each twice
//               (Q2_K: of groups 8h..8h+7, Q3_K: c_g; the B operand of the
//               group-sum MFMA)
// so a wave loads a super-block with 8 coalesced loads per lane, each unit
// half already where the MFMA B operand wants it and no scale decoding left
// in the loop.
// Q2_K keeps 2-bit quants: per lane L, 32 bytes at 32 L, one word per unit
// (q2_word), so its quant section is 2048 bytes and the later sections move
// up. Q5_K appends its fifth quant bits: per lane L, 16 bytes at 16 L, word
// t holding units 2t (bits 4-7 of each byte, q5_bit_word) and 2t + 1 (bits
// 0-3).
__host__ __device__ constexpr int gemm_quant_bytes(uint32_t type) { return type == T_Q2_K ? 2048 : 4096; }
__host__ __device__ constexpr int gemm_sc_off(uint32_t type) { return gemm_quant_bytes(type); }
__host__ __device__ constexpr int gemm_d_off(uint32_t type) { return gemm_sc_off(type) + 512; }
__host__ __device__ constexpr int gemm_min_off(uint32_t type) { return gemm_d_off(type) + 256; }
__host__ __device__ constexpr int gemm_bit_off(uint32_t type) { return gemm_min_off(type) + 1024; }
__host__ __device__ constexpr int gemm_chunk_bytes(uint32_t type) {
    return gemm_bit_off(type) + (type == T_Q5_K ? 1024 : 0);
}

__host__ __device__ inline int64_t gemm_layout_bytes(int64_t nblk32, int64_t nb, uint32_t type) {
    return nblk32 * nb * gemm_chunk_bytes(type);
}

// Q2_K / Q3_K plane helpers: the 2-bit quant of element e (0..31) of a unit
// record (element 16 i + 4 t + k at bits 8 k + 2 t of word i) and the
// Q3_K high-mask bit of element e (element 4 t + k at bit 8 k + t).
__device__ inline uint32_t two_bit_quant(uint32_t w0, uint32_t w1, int e) {
    const int in = e & 15;
    return ((e < 16 ? w0 : w1) >> (8 * (in & 3) + 2 * (in >> 2))) & 3u;
}
__device__ inline uint32_t hmask_bit(uint32_t hb, int e) { return (hb >> (8 * (e & 3) + (e >> 2))) & 1u; }

// Q3_K in the GEMM copy. With s = -sc (sc = 6-bit scale - 32, so s is in
// -31..32) and u = q + 4 (0..7), the unit operand byte is P - 128 with
// P = |s| * u', u' = u for s >= 0 and 8 - u otherwise (P <= 248, so
// P - 128 fits int8 and |s| * (u' - 4) = s * q). Summed over a group g:
//   sum s q x = sum (P - 128) x + (128 - 4 |s_g|) * bsum_g,
// so the group-sum MFMA takes c_g = 128 - 4 |s_g| (0..128, exact in f16) in
// place of the mins, and the super-block sum is -(S + T) with d stored
// negated.
__device__ inline int q3_neg_scale(const uint8_t *sc12, int g) {
    U4 m;
    m.x = ldp<uint32_t>(sc12);
    m.y = ldp<uint32_t>(sc12 + 4);
    m.z = ldp<uint32_t>(sc12 + 8);
    m.w = 0;
    return -k3_scale(m, g);
}

// Q2_K quants of one unit for lane half h, placed for the kernel's words:
// byte b carries at bits 0-1 element 8h + b (q0), at bits 2-3 element
// 8h + 4 + b (q1), at bits 4-5 element 16 + 8h + b (q2) and at bits 6-7
// element 16 + 8h + 4 + b (q3). w0, w1 are the matvec unit record.
__device__ inline uint32_t q2_word(uint32_t w0, uint32_t w1, int h) {
    uint32_t w = 0;
    for (int b = 0; b < 4; b++) {
        const uint32_t f = two_bit_quant(w0, w1, 8 * h + b) | (two_bit_quant(w0, w1, 8 * h + 4 + b) << 2) |
                           (two_bit_quant(w0, w1, 16 + 8 * h + b) << 4) |
                           (two_bit_quant(w0, w1, 16 + 8 * h + 4 + b) << 6);
        w |= f << (8 * b);
    }
    return w;
}

// Q5_K fifth bits of one unit for lane half h, placed for the kernel's
// nibble words: byte b carries at bit 4 the bit of element 8h + b (low
// nibble word q0), at bit 5 of 8h + 4 + b (q1), at bit 6 of 16 + 8h + b
// (q2) and at bit 7 of 16 + 8h + 4 + b (q3). hb is the matvec bit record.
__device__ inline uint32_t q5_bit_word(uint32_t hb, int h) {
    uint32_t w = 0;
    for (int b = 0; b < 4; b++) {
        const uint32_t bits = hmask_bit(hb, 8 * h + b) | (hmask_bit(hb, 8 * h + 4 + b) << 1) |
                              (hmask_bit(hb, 16 + 8 * h + b) << 2) |
                              (hmask_bit(hb, 16 + 8 * h + 4 + b) << 3);
        w |= bits << (8 * b + 4);
    }
    return w;
}

// One thread per (32-row block, super-block, 16-byte slot); rows past n_out
// are written as zeros.
__global__ __launch_bounds__(256) void gemm_layout_kernel(Layout L, const uint8_t *planes,
                                                          uint8_t *out, int64_t nblk32) {
    const int64_t nb = L.n_in / 256;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t per = gemm_chunk_bytes(L.type) / 16;  // 368 slots per chunk (Q5_K: 496)
    if (i >= nblk32 * nb * per) return;
    const int64_t chunk = i / per;
    const int slot = (int)(i % per);
    const int64_t blk = chunk / nb, c = chunk % nb;
    uint32_t v[4] = {0, 0, 0, 0};
    const bool q2 = L.type == T_Q2_K, q3 = L.type == T_Q3_K;
    const int kp = L.type == T_Q5_K ? 2 : 1;  // block plane of d, dmin and the 6-bit scales
    const int sc_off = gemm_sc_off(L.type), d_off = gemm_d_off(L.type);
    const int min_off = gemm_min_off(L.type), bit_off = gemm_bit_off(L.type);
    if (slot >= bit_off / 16) {  // Q5_K: fifth bits of lane L, units 2t and 2t + 1 per word
        const int lane = slot - bit_off / 16, h = lane >> 5, r = lane & 31;
        const int64_t row = blk * 32 + r;
        if (row < L.n_out)
            for (int t = 0; t < 4; t++)
                v[t] = q5_bit_word(ldp<uint32_t>(planes + unit_off(L, 1, row, c * 8 + 2 * t)), h) |
                       (q5_bit_word(ldp<uint32_t>(planes + unit_off(L, 1, row, c * 8 + 2 * t + 1)), h) >> 4);
    } else if (q2 && slot < sc_off / 16) {  // Q2_K: 2-bit words of lane L, units 4 p .. 4 p + 3
        const int lane = slot >> 1, p = slot & 1, h = lane >> 5, r = lane & 31;
        const int64_t row = blk * 32 + r;
        if (row < L.n_out)
            for (int t = 0; t < 4; t++) {
                const uint8_t *src = planes + unit_off(L, 0, row, c * 8 + 4 * p + t);
                v[t] = q2_word(ldp<uint32_t>(src), ldp<uint32_t>(src + 4), h);
            }
    } else if (slot < sc_off / 16) {  // unit halves
        const int q = slot >> 6, lane = slot & 63, h = lane >> 5, r = lane & 31;
        const int64_t row = blk * 32 + r;
        if (row < L.n_out) {
            for (int k = 0; k < 2; k++) {
                if (q3) {
                    const int j = 2 * q + k;
                    const uint8_t *src = planes + unit_off(L, 0, row, c * 8 + j);
                    const uint32_t w0 = ldp<uint32_t>(src), w1 = ldp<uint32_t>(src + 4);
                    const uint32_t hb = ldp<uint32_t>(planes + unit_off(L, 1, row, c * 8 + j));
                    const uint8_t *sc12 = planes + block_off(L, 2, row, c * 8);
                    const int s0 = q3_neg_scale(sc12, 2 * j), s1 = q3_neg_scale(sc12, 2 * j + 1);
                    for (int b = 0; b < 8; b++) {
                        const int el = 8 * h + b, eh = 16 + 8 * h + b;
                        const uint32_t ul = two_bit_quant(w0, w1, el) + 4 * hmask_bit(hb, el);
                        const uint32_t uh = two_bit_quant(w0, w1, eh) + 4 * hmask_bit(hb, eh);
                        const uint32_t nib = (s0 >= 0 ? ul : 8 - ul) | ((s1 >= 0 ? uh : 8 - uh) << 4);
                        v[2 * k + (b >> 2)] |= nib << (8 * (b & 3));
                    }
                } else if (q2) {
                    // Q2_K plane record: element 16 i + 4 t + e of the unit at
                    // bits 8 e + 2 t of word i; byte b of half h takes element
                    // 8 h + b (low nibble) and 16 + 8 h + b (high nibble)
                    const uint8_t *src = planes + unit_off(L, 0, row, c * 8 + 2 * q + k);
                    const uint32_t w0 = ldp<uint32_t>(src), w1 = ldp<uint32_t>(src + 4);
                    for (int b = 0; b < 8; b++) {
                        const int e = 8 * h + b;
                        const int sh = 8 * (e & 3) + 2 * (e >> 2);
                        const uint32_t nib = ((w0 >> sh) & 3u) | (((w1 >> sh) & 3u) << 4);
                        v[2 * k + (b >> 2)] |= nib << (8 * (b & 3));
                    }
                } else {
                    const uint8_t *src = planes + unit_off(L, 0, row, c * 8 + 2 * q + k) + 8 * h;
                    v[2 * k] = ldp<uint32_t>(src);
                    v[2 * k + 1] = ldp<uint32_t>(src + 4);
                }
            }
        }
    } else if (slot < d_off / 16) {  // scale bytes of one row
        const int64_t row = blk * 32 + (slot - sc_off / 16);
        if (row < L.n_out) {
            if (q3) {  // |s_g| for the 16 groups
                const uint8_t *sc12 = planes + block_off(L, 2, row, c * 8);
                for (int g = 0; g < 16; g++) {
                    const int sg = q3_neg_scale(sc12, g);
                    v[g >> 2] |= (uint32_t)(sg < 0 ? -sg : sg) << (8 * (g & 3));
                }
            } else if (q2) {  // the 4-bit group scales sc_0..sc_15
                const U4 m = ldp<U4>(planes + block_off(L, 1, row, c * 8));
                v[0] = m.x & 0x0F0F0F0Fu; v[1] = m.y & 0x0F0F0F0Fu;
                v[2] = m.z & 0x0F0F0F0Fu; v[3] = m.w & 0x0F0F0F0Fu;
            } else {
                const U4 m = ldp<U4>(planes + block_off(L, kp, row, c * 8));
                for (int j = 0; j < 8; j++) {
                    int sc, mn;
                    k4_scale_min(m, j, sc, mn);
                    v[j >> 2] |= (uint32_t)(sc >> 3) << (8 * (j & 3));
                    v[2 + (j >> 2)] |= (uint32_t)(sc & 7) << (8 * (j & 3));
                }
            }
        }
    } else if (slot < min_off / 16) {  // d, dmin of rows 2k, 2k + 1
        const int k = slot - d_off / 16;
        for (int t = 0; t < 2; t++) {
            const int64_t row = blk * 32 + 2 * k + t;
            if (row < L.n_out) {
                if (q3) {  // -d; no mins
                    const uint32_t dh = ldp<uint16_t>(planes + block_off(L, 3, row, c * 8));
                    v[2 * t] = __float_as_uint(-half_to_float(dh));
                } else {
                    const uint32_t dd = q2 ? ldp<uint32_t>(planes + block_off(L, 2, row, c * 8))
                                           : ldp<U4>(planes + block_off(L, kp, row, c * 8)).x;
                    v[2 * t] = __float_as_uint(half_to_float(dd & 0xffffu));
                    v[2 * t + 1] = __float_as_uint(half_to_float(dd >> 16));
                }
            }
        }
    } else {  // mins of lane L
        const int lane = slot - min_off / 16, h = lane >> 5, r = lane & 31;
        const int64_t row = blk * 32 + r;
        if (row < L.n_out && q3) {  // c_g = 128 - 4 |s_g| of groups 8 h .. 8 h + 7
            const uint8_t *sc12 = planes + block_off(L, 2, row, c * 8);
            for (int t = 0; t < 4; t++) {
                uint32_t hv[2];
                for (int e = 0; e < 2; e++) {
                    const int sg = q3_neg_scale(sc12, 8 * h + 2 * t + e);
                    hv[e] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)(128 - 4 * (sg < 0 ? -sg : sg)));
                }
                v[t] = hv[0] | (hv[1] << 16);
            }
        } else if (row < L.n_out) {
            const U4 m = ldp<U4>(planes + block_off(L, kp, row, c * 8));
            for (int t = 0; t < 4; t++) {
                if (q2) {  // groups 8 h + 2 t and 8 h + 2 t + 1: high nibbles
                    const uint32_t word = (h ? (t < 2 ? m.z : m.w) : (t < 2 ? m.x : m.y));
                    const int b = 2 * (t & 1);
                    const uint32_t m0 = (word >> (8 * b + 4)) & 15u, m1 = (word >> (8 * b + 12)) & 15u;
                    v[t] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)m0) |
                           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)m1) << 16);
                } else {
                    int sc, mn;
                    k4_scale_min(m, 4 * h + t, sc, mn);
                    const uint32_t hb = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(float)mn);
                    v[t] = hb | (hb << 16);
                }
            }
        }
    }
    *reinterpret_cast<uint4 *>(out + i * 16) = make_uint4(v[0], v[1], v[2], v[3]);
}

// This lane's operands of super-block c from the GEMM-ordered copy (base of
// the wave's 32-row block).
template <uint32_t FMT>
__device__ inline void gemm_load_w(const uint8_t *blk_base, int64_t c, int lane, GemmW &w) {
    const uint8_t *chunk = blk_base + c * gemm_chunk_bytes(FMT);
    if constexpr (FMT == T_Q2_K) {
        w.hb[0] = *reinterpret_cast<const uint4 *>(chunk + 32 * lane);
        w.hb[1] = *reinterpret_cast<const uint4 *>(chunk + 32 * lane + 16);
    } else {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint4 v = *reinterpret_cast<const uint4 *>(chunk + q * 1024 + 16 * lane);
            w.u[2 * q] = make_uint2(v.x, v.y);
            w.u[2 * q + 1] = make_uint2(v.z, v.w);
        }
    }
    w.scb = *reinterpret_cast<const uint4 *>(chunk + gemm_sc_off(FMT) + 16 * (lane & 31));
    w.dd = *reinterpret_cast<const float2 *>(chunk + gemm_d_off(FMT) + 8 * (lane & 31));
    w.bm = *reinterpret_cast<const v8h_t *>(chunk + gemm_min_off(FMT) + 16 * lane);
    if constexpr (FMT == T_Q5_K) w.hb[0] = *reinterpret_cast<const uint4 *>(chunk + gemm_bit_off(FMT) + 16 * lane);
}

// Bytewise q * f for bytes and products below 256 (no carries between
// bytes); f2 holds the factor in both 16-bit halves.
__device__ inline uint32_t bytes_times(uint32_t q, uint32_t f2) {
    const u16x2_t a = __builtin_bit_cast(u16x2_t, q);
    const u16x2_t b = __builtin_bit_cast(u16x2_t, f2);
    return __builtin_bit_cast(uint32_t, (u16x2_t)(a * b));
}

// Byte j (0..7) of the 8 bytes lo:hi in both 16-bit halves (v_perm_b32;
// selector 0x0c gives a zero byte).
__device__ inline uint32_t byte_pair(uint32_t lo, uint32_t hi, int j) {
    const uint32_t sel = (uint32_t)j | (0x0cu << 8) | ((uint32_t)j << 16) | (0x0cu << 24);
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// MT: 32-row MFMA tiles per wave along m (2 for large M; 1 for small M,
// which doubles the workgroups). NBUF: super-blocks of weights in flight
// per wave (registers for 4 fit at MT = 1), so a small-M launch, whose few
// workgroups each stream a long run of weights, keeps more bytes in flight.
template <uint32_t FMT, int MT, int NBUF>
__global__ __launch_bounds__(kGemmThreads)
__attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_kq_kernel(GemmArgs A) {
    static_assert(FMT == T_Q4_K || FMT == T_Q5_K || FMT == T_Q2_K || FMT == T_Q3_K,
                  "MFMA prefill: Q4_K, Q5_K, Q2_K, Q3_K");
    // Q4_K and Q5_K: two MFMAs per unit (8 sh + sl); Q2_K (sc * q <= 45)
    // and Q3_K (bytes P - 128) one. Q5_K's products sh * q, sl * q <= 217
    // go in as bytes P - 128 too.
    constexpr bool kSplit = FMT == T_Q4_K || FMT == T_Q5_K;
    constexpr uint32_t kBias = (FMT == T_Q3_K || FMT == T_Q5_K) ? 0x80808080u : 0u;
    constexpr int kAccL = kSplit ? MT : 1;
    static_assert(NBUF % 2 == 0, "LDS buffers alternate with the super-block parity");
    using Geo = GemmGeo<MT>;
    constexpr int kGemmMT = MT;
    constexpr int kGemmBM = Geo::BM;
    constexpr int kXDOff = Geo::XDOff, kXBOff = Geo::XBOff;
    constexpr int kXPieces = Geo::XPieces, kXE = Geo::XE, kXEPieces = Geo::XEPieces;
    __shared__ __attribute__((aligned(16))) uint8_t sx[2][Geo::XTile];
    // XCD-aware tile order: workgroups are dispatched round-robin over the 8
    // XCDs, so the m-tiles of one n-tile (which read the same weights) are
    // given to consecutive workgroups of the same XCD and share its L2.
    // (the m-tiles of one n-tile and K slice are consecutive)
    const int b = blockIdx.x;
    const int xcd = b & 7, t = b >> 3;
    const int per = A.MB * A.S;
    const int nblk = (t / per) * 8 + xcd, rest = t % per;
    const int slice = rest / A.MB, mblk = rest % A.MB;
    if (nblk >= A.NB) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int ln = lane & 31, h = lane >> 5;
    const int64_t m0 = (int64_t)mblk * kGemmBM;
    const int64_t n = (int64_t)nblk * kGemmBN + wave * 32 + ln;  // this lane's weight row
    const uint8_t *wblk = A.w + (int64_t)(nblk * (kGemmBN / 32) + wave) * A.nb * gemm_chunk_bytes(FMT);

    v16f_t y[kGemmMT];
#pragma unroll
    for (int i = 0; i < kGemmMT; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) y[i][r] = 0.0f;

    // one super-block: weights w (this lane's row), activation tile in buf
    auto compute = [&](const uint8_t *buf, const GemmW &w) {
        const float d = w.dd.x, dmin = w.dd.y;
        v16i_t acc_h[kGemmMT], acc_l[kAccL];
#pragma unroll
        for (int i = 0; i < kGemmMT; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc_h[i][r] = 0;
#pragma unroll
        for (int i = 0; i < kAccL; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc_l[i][r] = 0;
        // The MFMA section runs at a raised wave priority: of the two waves
        // on a SIMD, the one issuing MFMAs wins the issue slot, and the
        // other one's scalar-core work fills the gaps (measured ~6% faster
        // than equal priorities).
        __builtin_amdgcn_s_setprio(1);
        // activation operands are read two units ahead of the MFMAs using them
        v4i_t aa[8][kGemmMT];
#pragma unroll
        for (int i = 0; i < kGemmMT; i++) {
            aa[0][i] = *reinterpret_cast<const v4i_t *>(buf + (32 * i + ln) * kXRow + 16 * h);
            aa[1][i] = *reinterpret_cast<const v4i_t *>(buf + (32 * i + ln) * kXRow + 32 + 16 * h);
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            v4i_t ac[kGemmMT];
#pragma unroll
            for (int i = 0; i < kGemmMT; i++) {
                ac[i] = aa[j][i];
                if (j < 6)
                    aa[j + 2][i] = *reinterpret_cast<const v4i_t *>(buf + (32 * i + ln) * kXRow + 32 * (j + 2) + 16 * h);
            }
            // keep the reads of unit j + 2 ahead of the MFMAs of unit j
            __builtin_amdgcn_sched_barrier(0);
            // Q2_K: word j & 3 of hb[j / 4]; Q5_K: word j / 2 of hb[0], unit
            // j odd in its low nibbles (the other formats load no hb)
            uint32_t b = 0;
            if constexpr (FMT == T_Q2_K || FMT == T_Q5_K) {
                const uint4 hw = w.hb[FMT == T_Q5_K ? 0 : j >> 2];
                const int wi = FMT == T_Q5_K ? j >> 1 : j & 3;
                b = wi == 0 ? hw.x : wi == 1 ? hw.y : wi == 2 ? hw.z : hw.w;
                if (FMT == T_Q5_K && (j & 1)) b <<= 4;
            }
            uint32_t q0, q1, q2, q3;
            if constexpr (FMT == T_Q2_K) {  // quant words (q2_word)
                q0 = b & 0x03030303u;
                q1 = (b >> 2) & 0x03030303u;
                q2 = (b >> 4) & 0x03030303u;
                q3 = (b >> 6) & 0x03030303u;
            } else {
                const uint32_t w0 = w.u[j].x, w1 = w.u[j].y;
                q0 = w0 & 0x0F0F0F0Fu;
                q1 = w1 & 0x0F0F0F0Fu;
                q2 = (w0 >> 4) & 0x0F0F0F0Fu;
                q3 = (w1 >> 4) & 0x0F0F0F0Fu;
            }
            if constexpr (FMT == T_Q5_K) {  // fifth bits (q5_bit_word)
                q0 |= b & 0x10101010u;
                q1 |= (b >> 1) & 0x10101010u;
                q2 |= (b >> 2) & 0x10101010u;
                q3 |= (b >> 3) & 0x10101010u;
            }
            if constexpr (kSplit) {
                const uint32_t sh = byte_pair(w.scb.x, w.scb.y, j), sl = byte_pair(w.scb.z, w.scb.w, j);
                const v4i_t bh = {(int)(bytes_times(q0, sh) ^ kBias), (int)(bytes_times(q1, sh) ^ kBias),
                                  (int)(bytes_times(q2, sh) ^ kBias), (int)(bytes_times(q3, sh) ^ kBias)};
                const v4i_t bl = {(int)(bytes_times(q0, sl) ^ kBias), (int)(bytes_times(q1, sl) ^ kBias),
                                  (int)(bytes_times(q2, sl) ^ kBias), (int)(bytes_times(q3, sl) ^ kBias)};
#pragma unroll
                for (int i = 0; i < kGemmMT; i++) {
                    acc_h[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ac[i], bh, acc_h[i], 0, 0, 0);
                    acc_l[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ac[i], bl, acc_l[i], 0, 0, 0);
                }
            } else {
                // low nibbles (q0, q1) are group 2j of the unit, high
                // nibbles (q2, q3) group 2j + 1
                const uint32_t s0 = j < 4 ? byte_pair(w.scb.x, w.scb.y, 2 * j)
                                          : byte_pair(w.scb.z, w.scb.w, 2 * j - 8);
                const uint32_t s1 = j < 4 ? byte_pair(w.scb.x, w.scb.y, 2 * j + 1)
                                          : byte_pair(w.scb.z, w.scb.w, 2 * j - 7);
                const v4i_t b = {(int)(bytes_times(q0, s0) ^ kBias), (int)(bytes_times(q1, s0) ^ kBias),
                                 (int)(bytes_times(q2, s1) ^ kBias), (int)(bytes_times(q3, s1) ^ kBias)};
#pragma unroll
                for (int i = 0; i < kGemmMT; i++)
                    acc_h[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ac[i], b, acc_h[i], 0, 0, 0);
            }
        }
        __builtin_amdgcn_s_setprio(0);
        // mins against the group sums: slot s of half h is group 8h + s
        const v8h_t bm = w.bm;
        const float *dx = reinterpret_cast<const float *>(buf + kXDOff);
#pragma unroll
        for (int i = 0; i < kGemmMT; i++) {
            const v8h_t abs_ = *reinterpret_cast<const v8h_t *>(buf + kXBOff + (32 * i + ln) * 32 + 16 * h);
            v16f_t tz;
#pragma unroll
            for (int r = 0; r < 16; r++) tz[r] = 0.0f;
            const v16f_t T = __builtin_amdgcn_mfma_f32_32x32x16_f16(abs_, bm, tz, 0, 0, 0);
            // Q5_K: the row's quant sum (sum of its 16 group sums, exact)
            // for the operand bias, 9 * 128 per element over both passes
            v16f_t X;
            if constexpr (FMT == T_Q5_K) {
                v8h_t ones;
#pragma unroll
                for (int e = 0; e < 8; e++) ones[e] = (_Float16)1.0f;
                X = __builtin_amdgcn_mfma_f32_32x32x16_f16(abs_, ones, tz, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float dxr = dx[32 * i + 8 * (r / 4) + 4 * h + (r % 4)];
                float u;
                if constexpr (FMT == T_Q3_K) {
                    // -(S + T) in integers (T is an exact integer < 2^24),
                    // the sign in d
                    u = d * (float)(acc_h[i][r] + (int)T[r]);
                } else {
                    int S = kSplit ? 8 * acc_h[i][r] + acc_l[kSplit ? i : 0][r] : acc_h[i][r];
                    if constexpr (FMT == T_Q5_K) S += 1152 * (int)X[r];
                    // y += dx * (d * S - dmin * T)
                    u = fma_f32(-dmin, T[r], d * (float)S);
                }
                y[i][r] = fma_f32(dxr, u, y[i][r]);
            }
        }
    };

    // Activation tile of super-block c (rows m0..m0+BM-1) from the planes
    // into registers: BM/16 pieces of 16 quant bytes per thread and one
    // piece of the group sums (pieces 0..2BM-1) or scales (the next BM/4)
    // per thread; threads past them load the last piece again and do not
    // store it, so no load is predicated.
    v4i_t xq[kXPieces], xe[kXEPieces];
    const int tid = threadIdx.x;
    const int64_t K = A.nb * 256;
    auto load_x = [&](int64_t c) {
#pragma unroll
        for (int i = 0; i < kXPieces; i++) {
            const int piece = tid + 256 * i, row = piece >> 4, col = piece & 15;
            xq[i] = *reinterpret_cast<const v4i_t *>(A.X.q + (m0 + row) * K + c * 256 + col * 16);
        }
#pragma unroll
        for (int i = 0; i < kXEPieces; i++) {
            const int t = tid + 256 * i;
            const int p = t < kXE - 1 ? t : kXE - 1;
            const v4i_t *e = p < 2 * kGemmBM
                                 ? reinterpret_cast<const v4i_t *>(A.X.bs + (c * A.Mp + m0) * 16) + p
                                 : reinterpret_cast<const v4i_t *>(A.X.d + c * A.Mp + m0) + (p - 2 * kGemmBM);
            xe[i] = *e;
        }
    };
    auto store_x = [&](uint8_t *buf) {
#pragma unroll
        for (int i = 0; i < kXPieces; i++) {
            const int piece = tid + 256 * i, row = piece >> 4, col = piece & 15;
            *reinterpret_cast<v4i_t *>(buf + row * kXRow + col * 16) = xq[i];
        }
        // group sums (pieces 0 .. 2BM-1) follow the scales (BM / 4 pieces)
#pragma unroll
        for (int i = 0; i < kXEPieces; i++) {
            const int t = tid + 256 * i;
            if (t < kXE)
                reinterpret_cast<v4i_t *>(buf + kXDOff + (t < 2 * kGemmBM ? kGemmBM * 4 : -kGemmBM * 32))[t] = xe[i];
        }
    };

    // A ring of NBUF weight buffers and two LDS activation buffers in
    // ping-pong: the weights of super-block c + NBUF - 1 and the activation
    // tile of c + 1 are requested before c is computed. Loads are
    // unconditional (past the end they repeat the last super-block), so the
    // memory counters always hold them in issue order.
    const int64_t c0 = (int64_t)slice * A.SBK;
    const int64_t last = (c0 + A.SBK < A.nb ? c0 + A.SBK : A.nb) - 1;  // this slice's super-blocks
    auto clamp = [&](int64_t c) { return c < last ? c : last; };
    GemmW wb[NBUF];
    load_x(c0);
#pragma unroll
    for (int k = 0; k < NBUF - 1; k++) gemm_load_w<FMT>(wblk, clamp(c0 + k), lane, wb[k]);
    store_x(sx[0]);
    __syncthreads();
    for (int64_t c = c0;; c += NBUF) {
        bool done = false;
#pragma unroll
        for (int k = 0; k < NBUF; k++) {
            const int64_t cc = c + k;
            gemm_load_w<FMT>(wblk, clamp(cc + NBUF - 1), lane, wb[(k + NBUF - 1) % NBUF]);
            load_x(clamp(cc + 1));
            compute(sx[k & 1], wb[k]);
            store_x(sx[(k + 1) & 1]);
            __syncthreads();
            if (cc >= last) {
                done = true;
                break;
            }
        }
        if (done) break;
    }
    if (A.S == 1) {
        if (n < A.n_out) {
#pragma unroll
            for (int i = 0; i < kGemmMT; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int64_t m = m0 + 32 * i + 8 * (r / 4) + 4 * h + (r % 4);
                    if (m < A.M) A.y[m * A.ldy + n] = y[i][r];
                }
        }
        return;
    }
    // K slices: partial sums through agent-scope stores and loads (they
    // write through and read past the per-XCD L2s; no cache write-back or
    // invalidation is needed), each wave waiting for its stores before the
    // workgroup counts its arrival; nothing waits on another workgroup.
    const int64_t ldp = (int64_t)A.NB * kGemmBN;
    if (n < A.n_out) {
#pragma unroll
        for (int i = 0; i < kGemmMT; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t m = m0 + 32 * i + 8 * (r / 4) + 4 * h + (r % 4);
                if (m < A.M)
                    __hip_atomic_store(A.part + ((int64_t)slice * A.Mp + m) * ldp + n, y[i][r],
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
    }
    slices_finish<kGemmBM, kGemmBN, kGemmThreads>(A.part, A.cnt + (int64_t)mblk * A.NB + nblk, A.S,
                                                 A.Mp, ldp, m0, A.M, (int64_t)nblk * kGemmBN,
                                                 A.n_out, A.y, A.ldy);
}

}  // namespace sihip
