// Small-M GEMM for the K-quant weights (Q2_K, Q3_K, Q4_K, Q5_K, Q6_K; M <= 16
// activation rows, the batched decode step) on v_mfma_i32_16x16x64_i8, from
// a weight copy of (nearly) the GGUF size: Y[M x n_out] = X[M x n_in] * W^T
// with X quantized per row to Q8_K (records of gemm2_quantize_x<16>), each
// output within the tolerance of the reference dot (reference
// kernels.c:249-523). Per super-block c, weight row n, activation row m:
//   Q2_K, Q4_K, Q5_K:  y += dx * (d * sum_g s_g * sum_{k in g} q * x  -  dmin * sum_g m_g * bsum_g)
//   Q3_K, Q6_K:        y += dx * d * sum_g s_g * sum_{k in g} (q - bias) * x
// with s_g, m_g the scale and min of the group (16 elements) or unit (32
// elements) k lies in, and bias 4 (Q3_K) or 32 (Q6_K).
//
// The 16x16x64 MFMA gives each lane group (16 lanes) 16 K slots: half a
// unit, or one 16-element group, of one weight row per lane. With the
// activation operand masked so that output row 4 j + i only sees the K
// slots of lane group j,
//   A'[4 j + i][k] = x[4 h + i][k] if k is in lane group j, else 0,
// result register i of lane l is the unscaled sum of the lane's own slots,
//   P[i] = sum_{k in lane group l / 16} w[k, n] * x[4 h + i, k],  n = l % 16,
// for activation rows 4 h + i. So the weight operand is the plain quant
// (Q3_K and Q6_K: minus the bias, as int8), no scale is folded in and no
// digit split is needed; each lane applies its own scale with an integer
// multiply-add per result, S[h][i] += s * P[i]. The mins take the same
// masked product against an all-ones weight operand (the group sums of x),
// T[h][i] += m * P1[i]. One MFMA per K-step, n tile and 4 activation rows
// (h = 0 .. NH - 1, NH = ceil(M / 4)), plus one per K-step and 4 rows for
// the mins. A lane's sums cover its own slots only; the 4 lane groups are
// added (lane shuffles in a fixed order) after the last super-block.
//
// Launch: a workgroup per 32 weight rows whose KW waves split the
// super-blocks (wave w takes c = w, w + KW, ...), the next super-block's
// weights and activation fragments in flight while one computes; the waves'
// partial tiles meet in LDS at the end and wave 0 adds them in wave order.
#pragma once

#include "gemm2.h"
#include "unit.h"

namespace sihip {

// ---- weight copy ------------------------------------------------------------
//
// Per block of 32 weight rows and super-block c, one chunk:
//   quant plane 0 (QA bytes): the low bits of the 16 slots of lane l (rows
//     16 nt + l % 16, elements 64 ks + 16 (l / 16) + slot) for both n tiles:
//     nibble formats (Q4_K, Q5_K, Q6_K) at 1024 ks + 16 l, per n tile two
//     words, byte b of w0 = slot b | slot 8 + b << 4, of w1 = slot 4 + b |
//     slot 12 + b << 4; 2-bit formats (Q2_K, Q3_K) at 32 l + 8 ks, per n
//     tile one word, byte b = slot b | slot 4 + b << 2 | slot 8 + b << 4 |
//     slot 12 + b << 6
//   quant plane 1 (QB bytes, at QA): Q6_K the high 2-bit fields, at 32 l +
//     8 ks, per n tile a word as the 2-bit formats'; Q5_K the fifth bits and
//     Q3_K the high-mask bits, at 16 l + 4 ks, one word for both n tiles:
//     bit i of byte b = the bit of slot 4 i + b for n tile 0, bit 4 + i for
//     n tile 1
//   scales (512 bytes, at QA + QB): per row 16 bytes, in the order the lanes
//     read them: Q4_K and Q5_K the 6-bit unit scales and mins as s_0 s_2 s_4
//     s_6, m_0 m_2 m_4 m_6, s_1 s_3 s_5 s_7, m_1 m_3 m_5 m_7 (lane group g
//     reads 8 bytes at 8 (g / 2): its units 2 ks + g / 2 at byte ks); Q2_K
//     (GGUF scale bytes: s in the low, m in the high nibble), Q3_K (6-bit
//     scale minus 32, int8) and Q6_K (int8) the 16 group bytes as groups g,
//     4 + g, 8 + g, 12 + g for g = 0..3 (lane group g reads 4 bytes at 4 g:
//     group 4 ks + g at byte ks)
//   d (at QA + QB + 512): per row f16 d and dmin (Q2_K, Q4_K, Q5_K), or f16 d
// Sizes: Q2_K 2688 (the GGUF bytes), Q3_K 3648 (3520), Q4_K 4736 (4608),
// Q5_K 5760 (5632), Q6_K 6720 (6720).
template <uint32_t FMT>
struct KS {
    static constexpr bool nib = FMT == T_Q4_K || FMT == T_Q5_K || FMT == T_Q6_K;
    static constexpr bool mins = FMT == T_Q2_K || FMT == T_Q4_K || FMT == T_Q5_K;
    static constexpr bool unit32 = FMT == T_Q4_K || FMT == T_Q5_K;  // scales per 32 elements
    static constexpr int QA = nib ? 4096 : 2048;
    static constexpr int QB = FMT == T_Q6_K ? 2048 : (FMT == T_Q5_K || FMT == T_Q3_K) ? 1024 : 0;
    static constexpr int SC = QA + QB;
    static constexpr int D = SC + 512;
    static constexpr int DB = mins ? 4 : 2;  // bytes of d per row
    static constexpr int chunk = D + 32 * DB;
};

__host__ __device__ inline int gemmks_chunk(uint32_t t) {
    switch (t) {
        case T_Q2_K: return KS<T_Q2_K>::chunk;
        case T_Q3_K: return KS<T_Q3_K>::chunk;
        case T_Q4_K: return KS<T_Q4_K>::chunk;
        case T_Q5_K: return KS<T_Q5_K>::chunk;
        default: return KS<T_Q6_K>::chunk;
    }
}

// The 32 values of unit u of a row from the matvec planes, byte k of q[t]
// = element 4 t + k: Q4_K 0..15, Q5_K 0..31, Q6_K 0..63, Q3_K 0..7 (low
// bits + 4 * high-mask bit), Q2_K 0..3.
template <uint32_t FMT>
__device__ inline void ks_unit_values(const Layout &L, const uint8_t *planes, int64_t row, int64_t u,
                                      uint32_t q[8]) {
    if constexpr (FMT == T_Q4_K || FMT == T_Q5_K || FMT == T_Q6_K)
        nib_split(ldp<U4>(planes + unit_off(L, 0, row, u)), q);
    if constexpr (FMT == T_Q5_K) add_bit4(q, ldp<uint32_t>(planes + unit_off(L, 1, row, u)), 4);
    if constexpr (FMT == T_Q6_K) {
        const U2 h = ldp<U2>(planes + unit_off(L, 1, row, u));
        two8_split(h.x, h.y, q, 4, true);
    }
    if constexpr (FMT == T_Q2_K || FMT == T_Q3_K) {
        const U2 h = ldp<U2>(planes + unit_off(L, 0, row, u));
        two8_split(h.x, h.y, q, 0, false);
    }
    if constexpr (FMT == T_Q3_K) add_bit4(q, ldp<uint32_t>(planes + unit_off(L, 1, row, u)), 2);
}

// One thread per 16-byte piece of a chunk; rows past n_out are zero.
template <uint32_t FMT>
__global__ __launch_bounds__(256) void gemmks_layout(Layout L, const uint8_t *planes, uint8_t *out,
                                                     int64_t nblk32) {
    using F = KS<FMT>;
    const int64_t nb = L.n_in / 256;
    constexpr int per = F::chunk / 16;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nblk32 * nb * per) return;
    const int64_t chunk = i / per;
    const int p = (int)(i % per);
    const int64_t blk = chunk / nb, c = chunk % nb;
    uint32_t v[4] = {0, 0, 0, 0};
    // the 16 values of lane l's slots at K-step ks for n tile nt
    auto values = [&](int ks, int l, int nt, uint32_t qv[16]) -> bool {
        const int64_t row = blk * 32 + 16 * nt + (l & 15);
        if (row >= L.n_out) return false;
        const int g = l >> 4;
        const int k = 2 * ks + (g >> 1), half = g & 1;  // unit, half of it
        uint32_t q[8];
        ks_unit_values<FMT>(L, planes, row, c * 8 + k, q);
        for (int e = 0; e < 16; e++) {
            const int idx = 16 * half + e;
            qv[e] = (q[idx >> 2] >> (8 * (idx & 3))) & 0xffu;
        }
        return true;
    };
    // the word of 2-bit fields (field (v >> sh) & 3 of slot 4 i + b at bits
    // 2 i of byte b)
    auto two_word = [](const uint32_t qv[16], int sh) {
        uint32_t w = 0;
        for (int b = 0; b < 4; b++)
            for (int t = 0; t < 4; t++) w |= ((qv[4 * t + b] >> sh) & 3u) << (8 * b + 2 * t);
        return w;
    };
    if (p < F::QA / 16) {
        if constexpr (F::nib) {  // K-step p / 64, lane p % 64
            const int ks = p >> 6, l = p & 63;
            for (int nt = 0; nt < 2; nt++) {
                uint32_t qv[16];
                if (!values(ks, l, nt, qv)) continue;
                for (int b = 0; b < 4; b++) {
                    v[2 * nt] |= ((qv[b] & 15u) | ((qv[8 + b] & 15u) << 4)) << (8 * b);
                    v[2 * nt + 1] |= ((qv[4 + b] & 15u) | ((qv[12 + b] & 15u) << 4)) << (8 * b);
                }
            }
        } else {  // lane p / 2, K-steps 2 (p % 2), + 1
            const int l = p >> 1, h2 = p & 1;
            for (int kk = 0; kk < 2; kk++)
                for (int nt = 0; nt < 2; nt++) {
                    uint32_t qv[16];
                    if (values(2 * h2 + kk, l, nt, qv)) v[2 * kk + nt] = two_word(qv, 0);
                }
        }
    } else if (p < F::SC / 16) {
        const int q16 = p - F::QA / 16;
        if constexpr (FMT == T_Q6_K) {  // high fields of lane q16 / 2, K-steps 2 (q16 % 2), + 1
            const int l = q16 >> 1, h2 = q16 & 1;
            for (int kk = 0; kk < 2; kk++)
                for (int nt = 0; nt < 2; nt++) {
                    uint32_t qv[16];
                    if (values(2 * h2 + kk, l, nt, qv)) v[2 * kk + nt] = two_word(qv, 4);
                }
        } else {  // Q5_K fifth bits / Q3_K high-mask bits of lane q16, one word per K-step
            const int l = q16;
            const int bit = FMT == T_Q5_K ? 4 : 2;
            for (int ks = 0; ks < 4; ks++)
                for (int nt = 0; nt < 2; nt++) {
                    uint32_t qv[16];
                    if (!values(ks, l, nt, qv)) continue;
                    for (int b = 0; b < 4; b++)
                        for (int t = 0; t < 4; t++)
                            v[ks] |= ((qv[4 * t + b] >> bit) & 1u) << (8 * b + t + 4 * nt);
                }
        }
    } else if (p < F::D / 16) {  // the 16 scale bytes of one row
        const int64_t row = blk * 32 + (p - F::SC / 16);
        if (row < L.n_out) {
            if constexpr (F::unit32) {  // unit j = 2 ks + hb: word 2 hb (scale), 2 hb + 1 (min), byte ks
                const U4 m = ldp<U4>(planes + block_off(L, FMT == T_Q4_K ? 1 : 2, row, c * 8));
                for (int j = 0; j < 8; j++) {
                    int sc, mn;
                    k4_scale_min(m, j, sc, mn);
                    const int hb = j & 1, ks = j >> 1;
                    v[2 * hb] |= (uint32_t)sc << (8 * ks);
                    v[2 * hb + 1] |= (uint32_t)mn << (8 * ks);
                }
            } else {  // group 4 ks + g at word g, byte ks
                uint32_t gb[16];
                if constexpr (FMT == T_Q3_K) {
                    const uint8_t *sc12 = planes + block_off(L, 2, row, c * 8);
                    U4 m;
                    m.x = ldp<uint32_t>(sc12);
                    m.y = ldp<uint32_t>(sc12 + 4);
                    m.z = ldp<uint32_t>(sc12 + 8);
                    m.w = 0;
                    for (int gg = 0; gg < 16; gg++) gb[gg] = (uint32_t)k3_scale(m, gg) & 0xffu;
                } else {  // Q2_K and Q6_K: the uploaded bytes
                    const uint8_t *src = planes + block_off(L, FMT == T_Q2_K ? 1 : 2, row, c * 8);
                    for (int gg = 0; gg < 16; gg++) gb[gg] = src[gg];
                }
                for (int gg = 0; gg < 16; gg++) v[gg & 3] |= gb[gg] << (8 * (gg >> 2));
            }
        }
    } else {  // d (and dmin) of 16 / DB rows
        const int k = p - F::D / 16;
        constexpr int rows = 16 / F::DB;
        for (int t = 0; t < rows; t++) {
            const int64_t row = blk * 32 + rows * k + t;
            if (row >= L.n_out) continue;
            if constexpr (F::mins) {
                const uint32_t dd = FMT == T_Q2_K ? ldp<uint32_t>(planes + block_off(L, 2, row, c * 8))
                                                  : ldp<U4>(planes + block_off(L, FMT == T_Q4_K ? 1 : 2, row, c * 8)).x;
                v[t] = dd;
            } else {
                v[t >> 1] |= (uint32_t)ldp<uint16_t>(planes + block_off(L, 3, row, c * 8)) << (16 * (t & 1));
            }
        }
    }
    *reinterpret_cast<uint4 *>(out + i * 16) = make_uint4(v[0], v[1], v[2], v[3]);
}

// ---- the GEMM -----------------------------------------------------------------

struct GKSArgs {
    const uint8_t *w;     // chunks [nblk32][nb]
    const uint8_t *x;     // activation records of one 16-row block [nb] (g2_rec_bytes(16))
    float *y;             // Y[m * ldy + n]
    int64_t ldy;
    int64_t n_out, M;
    int nb;
};

// Weight super-blocks in registers per wave (gemmks_kernel SW) that fit the
// 256 VGPRs of two waves per SIMD without spills: the 2-bit formats leave
// room for deeper rings at up to 8 activation rows.
template <uint32_t FMT, int NH>
__host__ __device__ constexpr int gemmks_sw() {
    return NH > 2 ? 2 : FMT == T_Q3_K ? 4 : FMT == T_Q2_K ? 3 : 2;
}

// One super-block of a lane's weights (a 32-row block's chunk) and of its
// activation fragments.
template <uint32_t FMT>
struct KSWStage {
    uint4 qa[4];    // quant plane 0: nibble formats K-step ks; 2-bit formats [0..1] used
    uint4 qb[2];    // quant plane 1 (Q6_K: 2 pieces, Q5_K/Q3_K: [0])
    uint32_t sc[2][KS<FMT>::unit32 ? 2 : 1];  // n tile: this lane group's scale (and min) words
    uint32_t d[2];  // n tile: f16 d and dmin (Q3_K, Q6_K: the word holding d)
};
template <int NH>
struct KSXStage {
    uint4 a[NH][4]; // masked activation fragments of rows 4 h + l % 4, K-step ks
    float4 dx[NH];  // block scales of rows 4 h .. 4 h + 3
};

__device__ inline uint4 ks_ld4(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// A weight load: nontemporal (the weights are read once per call; at M = 8
// the Llama-3-8B batch-8 decode step took 1.90 ms with default loads, 1.84
// with these).
__device__ inline uint4 ks_ld4nt(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 2));
}

// The weights of super-block c (wave-uniform) of the chunk column behind wr,
// with nontemporal loads (cache policy 2 on gfx950: nt).
// readfirstlane keeps the offsets scalar (a loop counter the compiler holds
// in a VGPR would make every buffer load a waterfall loop over lanes).
template <uint32_t FMT>
__device__ inline void ks_load_w(__amdgpu_buffer_rsrc_t wr, int c, int lane, KSWStage<FMT> &s) {
    using F = KS<FMT>;
    const int g = lane >> 4, r16 = lane & 15;
    const int so = __builtin_amdgcn_readfirstlane(c) * F::chunk;
    if constexpr (F::nib) {
#pragma unroll
        for (int ks = 0; ks < 4; ks++) s.qa[ks] = ks_ld4nt(wr, ks * 1024 + lane * 16, so);
    } else {
#pragma unroll
        for (int j = 0; j < 2; j++) s.qa[j] = ks_ld4nt(wr, lane * 32 + j * 16, so);
    }
    if constexpr (FMT == T_Q6_K) {
#pragma unroll
        for (int j = 0; j < 2; j++) s.qb[j] = ks_ld4nt(wr, F::QA + lane * 32 + j * 16, so);
    } else if constexpr (F::QB > 0) {
        s.qb[0] = ks_ld4nt(wr, F::QA + lane * 16, so);
    }
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        if constexpr (F::unit32) {
            const uint2 t = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(
                                                          wr, F::SC + (16 * nt + r16) * 16 + 8 * (g >> 1), so, 2));
            s.sc[nt][0] = t.x;
            s.sc[nt][1] = t.y;
        } else {
            s.sc[nt][0] = __builtin_amdgcn_raw_buffer_load_b32(wr, F::SC + (16 * nt + r16) * 16 + 4 * g, so, 2);
        }
    }
    if constexpr (F::mins) {
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
            s.d[nt] = __builtin_amdgcn_raw_buffer_load_b32(wr, F::D + (16 * nt + r16) * 4, so, 2);
    } else {
        s.d[0] = __builtin_amdgcn_raw_buffer_load_b32(wr, F::D + (r16 >> 1) * 4, so, 2);
        s.d[1] = __builtin_amdgcn_raw_buffer_load_b32(wr, F::D + 32 + (r16 >> 1) * 4, so, 2);
    }
}

// The weight operand of K-step ks, n tile nt: dword i holds slots 4 i .. 4 i + 3.
template <uint32_t FMT>
__device__ inline v4i2_t ks_operand(const KSWStage<FMT> &s, int ks, int nt) {
    const uint32_t m4 = 0x0F0F0F0Fu, m2 = 0x03030303u, m1 = 0x01010101u;
    uint32_t q[4];
    if constexpr (KS<FMT>::nib) {
        const uint32_t w0 = nt ? s.qa[ks].z : s.qa[ks].x;
        const uint32_t w1 = nt ? s.qa[ks].w : s.qa[ks].y;
        q[0] = w0 & m4;
        q[1] = w1 & m4;
        q[2] = (w0 >> 4) & m4;
        q[3] = (w1 >> 4) & m4;
    } else {
        const uint4 wv = s.qa[ks >> 1];
        const uint32_t W = (ks & 1) ? (nt ? wv.w : wv.z) : (nt ? wv.y : wv.x);
#pragma unroll
        for (int t = 0; t < 4; t++) q[t] = (W >> (2 * t)) & m2;
    }
    if constexpr (FMT == T_Q6_K) {
        const uint4 hv = s.qb[ks >> 1];
        const uint32_t H = (ks & 1) ? (nt ? hv.w : hv.z) : (nt ? hv.y : hv.x);
#pragma unroll
        for (int t = 0; t < 4; t++) q[t] |= ((H >> (2 * t)) & m2) << 4;
    }
    if constexpr (FMT == T_Q5_K || FMT == T_Q3_K) {
        const uint32_t Fw = ks == 0 ? s.qb[0].x : ks == 1 ? s.qb[0].y : ks == 2 ? s.qb[0].z : s.qb[0].w;
        constexpr int pos = FMT == T_Q5_K ? 4 : 2;
#pragma unroll
        for (int t = 0; t < 4; t++) q[t] |= ((Fw >> (t + 4 * nt)) & m1) << pos;
    }
    // Q3_K: q - 4 (q + 124 < 256, bit 7 flipped); Q6_K: q - 32 (q + 96)
    if constexpr (FMT == T_Q3_K) {
#pragma unroll
        for (int t = 0; t < 4; t++) q[t] = (q[t] + 0x7C7C7C7Cu) ^ 0x80808080u;
    }
    if constexpr (FMT == T_Q6_K) {
#pragma unroll
        for (int t = 0; t < 4; t++) q[t] = (q[t] + 0x60606060u) ^ 0x80808080u;
    }
    return (v4i2_t){(int)q[0], (int)q[1], (int)q[2], (int)q[3]};
}

// This lane's scale and min at K-step ks, n tile nt.
template <uint32_t FMT>
__device__ inline void ks_scale(const KSWStage<FMT> &s, int ks, int nt, int &sv, int &mv) {
    if constexpr (KS<FMT>::unit32) {  // unit 2 ks + g / 2 at byte ks
        sv = (int)((s.sc[nt][0] >> (8 * ks)) & 0xffu);
        mv = (int)((s.sc[nt][1] >> (8 * ks)) & 0xffu);
    } else if constexpr (FMT == T_Q2_K) {  // group 4 ks + g at byte ks
        const uint32_t b = (s.sc[nt][0] >> (8 * ks)) & 0xffu;
        sv = (int)(b & 15u);
        mv = (int)(b >> 4);
    } else {
        sv = sbfe8(s.sc[nt][0], 8u * (uint32_t)ks);
        mv = 0;
    }
}

// One super-block: y[h][nt][i] += its contribution for activation rows
// 4 h + i (the sums of this lane's own K slots; the 4 lane groups are added
// after the last super-block).
template <uint32_t FMT, int NH>
__device__ inline void ks_compute(const KSWStage<FMT> &s, const KSXStage<NH> &x, int r16,
                                  v4f2_t (&y)[NH][2]) {
    using F = KS<FMT>;
    v4i2_t S[NH][2], T[NH][2];
#pragma unroll
    for (int h = 0; h < NH; h++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            S[h][nt] = (v4i2_t){0, 0, 0, 0};
            T[h][nt] = (v4i2_t){0, 0, 0, 0};
        }
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        v4i2_t am[NH];
#pragma unroll
        for (int h = 0; h < NH; h++) am[h] = __builtin_bit_cast(v4i2_t, x.a[h][ks]);
        v4i2_t P1[NH];
        if constexpr (F::mins) {
            const v4i2_t ones = {0x01010101, 0x01010101, 0x01010101, 0x01010101};
            const v4i2_t z = {0, 0, 0, 0};
#pragma unroll
            for (int h = 0; h < NH; h++) P1[h] = __builtin_amdgcn_mfma_i32_16x16x64_i8(am[h], ones, z, 0, 0, 0);
        }
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const v4i2_t b = ks_operand<FMT>(s, ks, nt);
            int sv, mv;
            ks_scale<FMT>(s, ks, nt, sv, mv);
#pragma unroll
            for (int h = 0; h < NH; h++) {
                const v4i2_t z = {0, 0, 0, 0};
                const v4i2_t P = __builtin_amdgcn_mfma_i32_16x16x64_i8(am[h], b, z, 0, 0, 0);
                // |P|, |P1| < 2^17 and |s|, |m| <= 128: 24-bit products
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    S[h][nt][i] += __mul24(sv, P[i]);
                    if constexpr (F::mins) T[h][nt][i] += __mul24(mv, P1[h][i]);
                }
            }
        }
    }
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        // mins formats: d in the low, dmin in the high half; Q3_K, Q6_K:
        // the word of rows 2 (r16 / 2), + 1
        const uint32_t dword = s.d[nt];
        const float dw = half_to_float(F::mins ? (dword & 0xffffu) : (dword >> (16 * (r16 & 1))) & 0xffffu);
        const float ndm = F::mins ? -half_to_float(dword >> 16) : 0.0f;
#pragma unroll
        for (int h = 0; h < NH; h++) {
            const float dxv[4] = {x.dx[h].x, x.dx[h].y, x.dx[h].z, x.dx[h].w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                if constexpr (F::mins) {
                    const float u = fma_f32(dw, (float)S[h][nt][i], ndm * (float)T[h][nt][i]);
                    y[h][nt][i] = fma_f32(dxv[i], u, y[h][nt][i]);
                } else {
                    y[h][nt][i] = fma_f32(dxv[i] * dw, (float)S[h][nt][i], y[h][nt][i]);
                }
            }
        }
    }
}

// Adds the 4 lane groups (each holds the sums over its own slots):
// partners l ^ 16, then l ^ 32, the same order in every lane.
template <int NH>
__device__ inline void ks_add_groups(v4f2_t (&y)[NH][2]) {
#pragma unroll
    for (int h = 0; h < NH; h++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float v = y[h][nt][i];
                v += __shfl_xor(v, 16, 64);
                v += __shfl_xor(v, 32, 64);
                y[h][nt][i] = v;
            }
}

// NH: 4-row activation groups (M <= 4 NH); KW: waves per workgroup, which
// split the super-blocks of its 32 rows; SW: super-blocks of weights a wave
// has in registers (the one computed and SW - 1 in flight).
template <uint32_t FMT, int NH, int KW, int SW = 2>
__global__ __launch_bounds__(64 * KW)
__attribute__((amdgpu_waves_per_eu(2))) void gemmks_kernel(GKSArgs A) {
    using F = KS<FMT>;
    constexpr int BM = 16;
    constexpr int kRec = g2_rec_bytes(BM);
    constexpr int kChunk = F::chunk;
    __shared__ __attribute__((aligned(16))) float red[KW - 1][NH][2][4][64];
    const int blk = blockIdx.x;  // 32-row block
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, r16 = lane & 15;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(A.w + (int64_t)blk * A.nb * kChunk), (short)0, A.nb * kChunk, 0x00020000);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)A.x, (short)0, A.nb * kRec, 0x00020000);
    // masked activation operand: output row 4 j + i sees lane group j only,
    // so lane l carries row 4 h + (l % 4) of K group l / 16 when l % 16 / 4
    // == l / 16, else zeros; its source is lane 16 g + 4 h + l % 4 of the
    // record fragment. The other lanes load from past the end of the buffer
    // resource, which returns zeros without a memory access.
    const int a_off = (r16 >> 2) == g ? 0 : 0x40000000;
    using WStage = KSWStage<FMT>;
    using XStage = KSXStage<NH>;
    auto load_w = [&](int c, WStage &s) { ks_load_w<FMT>(wr, c, lane, s); };
    auto load_x = [&](int c, XStage &s) {
        const int xo = __builtin_amdgcn_readfirstlane(c) * kRec;
#pragma unroll
        for (int h = 0; h < NH; h++) {
            const int src = 16 * g + 4 * h + (lane & 3);
#pragma unroll
            for (int ks = 0; ks < 4; ks++) s.a[h][ks] = ks_ld4(xr, a_off + ks * 1024 + src * 16, xo);
            s.dx[h] = __builtin_bit_cast(float4, ks_ld4(xr, g2_rec_dx(BM) + 16 * h, xo));
        }
    };
    v4f2_t y[NH][2];
#pragma unroll
    for (int h = 0; h < NH; h++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++) y[h][nt] = (v4f2_t){0.0f, 0.0f, 0.0f, 0.0f};
    auto compute = [&](const WStage &s, const XStage &x) { ks_compute<FMT, NH>(s, x, r16, y); };
    // rings of register sets: super-block c computes from weight set j %
    // SW and activation set j % 2 while the weights of the next SW - 1
    // super-blocks of this wave (from HBM) and the activations of the next
    // one (from the L2) are in flight; the ring indices are compile-time
    // constants in the unrolled body. Whole rounds (every super-block of
    // the round exists) load without conditions (past the end a load reads
    // the last super-block again, which nothing computes): a load under a
    // condition makes the compiler count it as possibly missing, and every
    // compute after it then waits for all loads in flight, the ring's later
    // sets too. A memory clobber and a scheduling barrier keep the loads
    // ahead of the compute (else the compiler sinks them below it, next to
    // their use, or moves the compute above them). The last partial round
    // loads and computes under conditions (for a wave with at most U
    // super-blocks that is the whole loop).
    // The whole rounds take a second copy of the compute, which spills at
    // NH > 2 and for Q5_K; those run one loop whose loads are unconditional
    // and whose compute is not.
    constexpr int U = SW % 2 ? 2 * SW : SW;
    constexpr bool kRounds = NH <= 2 && FMT != T_Q5_K;
    WStage ws[SW];
    XStage xs[2];
    const int last = A.nb - 1;
    auto cl = [&](int c) { return c < last ? c : last; };
#pragma unroll
    for (int k = 0; k < SW - 1; k++) load_w(cl(wave + k * KW), ws[k]);
    load_x(cl(wave), xs[0]);
    if constexpr (kRounds) {
        int c0 = wave;
        for (; c0 + (U - 1) * KW < A.nb; c0 += U * KW) {
#pragma unroll
            for (int j = 0; j < U; j++) {
                const int c = c0 + j * KW;
                load_w(cl(c + (SW - 1) * KW), ws[(j + SW - 1) % SW]);
                load_x(cl(c + KW), xs[(j + 1) % 2]);
                asm volatile("" ::: "memory");
                __builtin_amdgcn_sched_barrier(0);
                compute(ws[j % SW], xs[j % 2]);
            }
        }
#pragma unroll
        for (int j = 0; j < U; j++) {
            const int c = c0 + j * KW;
            if (c < A.nb) {
                const int cw = c + (SW - 1) * KW, cx = c + KW;
                if (cw < A.nb) load_w(cw, ws[(j + SW - 1) % SW]);
                if (cx < A.nb) load_x(cx, xs[(j + 1) % 2]);
                compute(ws[j % SW], xs[j % 2]);
            }
        }
    } else {
        // one copy of the compute: loads without conditions, the compute
        // under its own
        for (int c0 = wave; c0 < A.nb; c0 += U * KW) {
#pragma unroll
            for (int j = 0; j < U; j++) {
                const int c = c0 + j * KW;
                load_w(cl(c + (SW - 1) * KW), ws[(j + SW - 1) % SW]);
                load_x(cl(c + KW), xs[(j + 1) % 2]);
                asm volatile("" ::: "memory");
                __builtin_amdgcn_sched_barrier(0);
                if (c < A.nb) compute(ws[j % SW], xs[j % 2]);
            }
        }
    }
    ks_add_groups<NH>(y);
    if (wave > 0) {
#pragma unroll
        for (int h = 0; h < NH; h++)
#pragma unroll
            for (int nt = 0; nt < 2; nt++)
#pragma unroll
                for (int i = 0; i < 4; i++) red[wave - 1][h][nt][i][lane] = y[h][nt][i];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int wv = 0; wv < KW - 1; wv++)
#pragma unroll
        for (int h = 0; h < NH; h++)
#pragma unroll
            for (int nt = 0; nt < 2; nt++)
#pragma unroll
                for (int i = 0; i < 4; i++) y[h][nt][i] += red[wv][h][nt][i][lane];
    // lane group h stores activation rows 4 h .. 4 h + 3
    const int64_t n0 = (int64_t)blk * 32;
#pragma unroll
    for (int h = 0; h < NH; h++) {
        if (g != h) continue;
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const int64_t n = n0 + 16 * nt + r16;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int64_t m = 4 * h + i;
                if (m < A.M && n < A.n_out) A.y[m * A.ldy + n] = y[h][nt][i];
            }
        }
    }
}

}  // namespace sihip
