// Small-M GEMM for Q6_K weights (M <= 16 activation rows, the batched
// decode step) on v_mfma_i32_16x16x64_i8, from a weight copy of the GGUF
// size: Y[M x n_out] = X[M x n_in] * W^T with X quantized per row to Q8_K
// (records of gemm2_quantize_x<16>), each output within the tolerance of
// the reference dot (reference kernels.c:480-523):
//   y[m,n] = sum_c dx[m,c] * d[n,c] * sum_g sc_g[n] * sum_{k in g} (q[n,k] - 32) * x[m,k]
// over super-blocks c and their 16 groups g of 16 elements.
//
// The 16x16x64 MFMA gives a lane group (16 lanes) 16 K slots, exactly one
// scale group of one weight row per lane. With the activation operand
// masked so that output row 4 j + i only sees the K slots of lane group j,
//   A'[4 j + i][k] = x[4 h + i][k] if k is in lane group j, else 0,
// result register i of lane l is the unscaled group sum
//   P[i] = sum_{k in group 4 ks + l / 16} u[k, n] * x[4 h + i, k],  n = l % 16,
// of that lane's own scale group, for activation rows 4 h + i. So the
// weight operand is the plain 6-bit quant minus 32 (an int8, no scale
// folded in, no digit split) and each lane applies its own group scale with
// one integer multiply-add per result: S[h][i] += sc * P[i]. One MFMA per
// K-step, n tile and 4 activation rows (h = 0 .. NH - 1, NH = ceil(M / 4)).
// A lane's sums cover its own groups only; the 4 lane groups are added
// (lane shuffles in a fixed order) after the last super-block.
//
// Launch: a workgroup per 32 weight rows whose KW waves split the
// super-blocks (wave w takes c = w, w + KW, ...), the next super-block's
// weights and activation fragments in flight while one computes; the
// waves' partial tiles meet in LDS at the end (as gemm2s.h).
#pragma once

#include "gemm2.h"
#include "unit.h"

namespace sihip {

// ---- weight copy (GGUF size) ------------------------------------------------
//
// Per block of 32 weight rows and super-block c, one chunk of 6720 bytes
// (32 x 210, the GGUF bytes):
//   [0, 4096):     low nibbles, K-step ks at 1024 ks, lane l at 16 l: rows
//                  16 nt + l % 16 (nt = 0, 1) in bytes 8 nt .. 8 nt + 7, the
//                  16 elements 64 ks + 16 (l / 16) + slot as two words:
//                  byte b of w0 = lo(slot b) | lo(slot 8 + b) << 4, of w1 =
//                  lo(slot 4 + b) | lo(slot 12 + b) << 4
//   [4096, 6144):  high 2-bit fields, lane l at 4096 + 32 l, K-step ks at
//                  + 8 ks, n tile nt at + 4 nt: byte b = hi(slot b) |
//                  hi(slot 4 + b) << 2 | hi(slot 8 + b) << 4 | hi(slot 12 + b) << 6
//   [6144, 6656):  per row, the 16 int8 group scales
//   [6656, 6720):  per row, f16 d
constexpr int kG6SChunk = 6720;
constexpr int kG6SHi = 4096, kG6SSc = 6144, kG6SD = 6656;

__host__ __device__ inline int64_t gemm6s_layout_bytes(int64_t nblk32, int64_t nb) {
    return nblk32 * nb * kG6SChunk;
}

// One thread per 16-byte piece of a chunk (420 per chunk); rows past n_out
// are zero.
__global__ __launch_bounds__(256) void gemm6s_layout_q6k(Layout L, const uint8_t *planes,
                                                         uint8_t *out, int64_t nblk32) {
    const int64_t nb = L.n_in / 256;
    constexpr int per = kG6SChunk / 16;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nblk32 * nb * per) return;
    const int64_t chunk = i / per;
    const int p = (int)(i % per);
    const int64_t blk = chunk / nb, c = chunk % nb;
    uint32_t v[4] = {0, 0, 0, 0};
    // the 16 quants (0..63) of lane l's slots at K-step ks for n tile nt
    auto quants = [&](int ks, int l, int nt, uint32_t qv[16]) -> bool {
        const int64_t row = blk * 32 + 16 * nt + (l & 15);
        if (row >= L.n_out) return false;
        const int g = l >> 4;
        const int k = 2 * ks + (g >> 1), half = g & 1;  // unit, half of it
        const int64_t u = c * 8 + k;
        const U4 ql = ldp<U4>(planes + unit_off(L, 0, row, u));
        const U2 qh = ldp<U2>(planes + unit_off(L, 1, row, u));
        uint32_t q[8];
        nib_split(ql, q);
        two8_split(qh.x, qh.y, q, 4, true);
        for (int e = 0; e < 16; e++) {
            const int idx = 16 * half + e;
            qv[e] = (q[idx >> 2] >> (8 * (idx & 3))) & 0xffu;
        }
        return true;
    };
    if (p < kG6SHi / 16) {  // low nibbles: K-step p / 64, lane p % 64
        const int ks = p >> 6, l = p & 63;
        for (int nt = 0; nt < 2; nt++) {
            uint32_t qv[16];
            if (!quants(ks, l, nt, qv)) continue;
            uint32_t w0 = 0, w1 = 0;
            for (int b = 0; b < 4; b++) {
                w0 |= ((qv[b] & 15u) | ((qv[8 + b] & 15u) << 4)) << (8 * b);
                w1 |= ((qv[4 + b] & 15u) | ((qv[12 + b] & 15u) << 4)) << (8 * b);
            }
            v[2 * nt] = w0;
            v[2 * nt + 1] = w1;
        }
    } else if (p < kG6SSc / 16) {  // high fields of lane l, K-steps 2 h2, 2 h2 + 1
        const int q16 = p - kG6SHi / 16, l = q16 >> 1, h2 = q16 & 1;
        for (int kk = 0; kk < 2; kk++)
            for (int nt = 0; nt < 2; nt++) {
                uint32_t qv[16];
                if (!quants(2 * h2 + kk, l, nt, qv)) continue;
                uint32_t w = 0;
                for (int b = 0; b < 4; b++)
                    w |= ((qv[b] >> 4) | ((qv[4 + b] >> 4) << 2) | ((qv[8 + b] >> 4) << 4) |
                          ((qv[12 + b] >> 4) << 6))
                         << (8 * b);
                v[2 * kk + nt] = w;
            }
    } else if (p < kG6SD / 16) {  // the 16 group scales of one row
        const int64_t row = blk * 32 + (p - kG6SSc / 16);
        if (row < L.n_out) {
            const U4 m = ldp<U4>(planes + block_off(L, 2, row, c * 8));
            v[0] = m.x; v[1] = m.y; v[2] = m.z; v[3] = m.w;
        }
    } else {  // f16 d of rows 8 k .. 8 k + 7
        const int k = p - kG6SD / 16;
        for (int t = 0; t < 8; t++) {
            const int64_t row = blk * 32 + 8 * k + t;
            if (row < L.n_out)
                v[t >> 1] |= (uint32_t)ldp<uint16_t>(planes + block_off(L, 3, row, c * 8)) << (16 * (t & 1));
        }
    }
    *reinterpret_cast<uint4 *>(out + i * 16) = make_uint4(v[0], v[1], v[2], v[3]);
}

// ---- the GEMM -----------------------------------------------------------------

struct G6SArgs {
    const uint8_t *w;     // chunks [nblk32][nb]
    const uint8_t *x;     // activation records of one 16-row block [nb] (g2_rec_bytes(16))
    float *y;             // Y[m * ldy + n]
    int64_t ldy;
    int64_t n_out, M;
    int nb;
};

// NH: 4-row activation groups (M <= 4 NH); KW: waves per workgroup, which
// split the super-blocks of its 32 rows.
template <int NH, int KW>
__global__ __launch_bounds__(64 * KW)
__attribute__((amdgpu_waves_per_eu(2))) void gemm6s_q6k_kernel(G6SArgs A) {
    constexpr int BM = 16;
    constexpr int kRec = g2_rec_bytes(BM);
    __shared__ __attribute__((aligned(16))) float red[KW - 1][NH][2][4][64];
    const int blk = blockIdx.x;  // 32-row block
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, r16 = lane & 15;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(A.w + (int64_t)blk * A.nb * kG6SChunk), (short)0, A.nb * kG6SChunk, 0x00020000);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)A.x, (short)0, A.nb * kRec, 0x00020000);
    // masked activation operand: output row 4 j + i sees lane group j only,
    // so lane l carries row 4 h + (l % 4) of K group l / 16 when l % 16 / 4
    // == l / 16, else zeros; its source is lane 16 g + 4 h + l % 4 of the
    // record fragment. The other lanes load from past the end of the buffer
    // resource, which returns zeros without a memory access.
    const bool keep = (r16 >> 2) == g;
    const int a_off = keep ? 0 : 0x40000000;
    struct Stage {
        uint4 nib[4];   // K-step ks: n tile 0 in x, y; 1 in z, w
        uint4 hi[2];    // K-steps 2 j, 2 j + 1: x, y = ks 2 j (nt 0, 1); z, w = ks 2 j + 1
        uint4 sc[2];    // n tile: the row's 16 group scales
        uint32_t d;     // f16 d of rows r16 (low half) and 16 + r16 (high half)
        uint4 a[NH][4]; // activation fragments
        float4 dx[NH];  // block scales of rows 4 h .. 4 h + 3
    };
    auto ld4 = [&](__amdgpu_buffer_rsrc_t r, int voff, int soff) {
        return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
    };
    auto load = [&](int c, Stage &s) {
        // c is wave-uniform; readfirstlane keeps the offsets scalar (a loop
        // counter the compiler holds in a VGPR would make every buffer load
        // a waterfall loop over lanes)
        const int cu = __builtin_amdgcn_readfirstlane(c);
        const int so = cu * kG6SChunk, xo = cu * kRec;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) s.nib[ks] = ld4(wr, ks * 1024 + lane * 16, so);
#pragma unroll
        for (int j = 0; j < 2; j++) s.hi[j] = ld4(wr, kG6SHi + lane * 32 + j * 16, so);
#pragma unroll
        for (int nt = 0; nt < 2; nt++) s.sc[nt] = ld4(wr, kG6SSc + (16 * nt + r16) * 16, so);
        const uint32_t d0 = __builtin_amdgcn_raw_buffer_load_b32(wr, kG6SD + (r16 >> 1) * 4, so, 0);
        const uint32_t d1 = __builtin_amdgcn_raw_buffer_load_b32(wr, kG6SD + 32 + (r16 >> 1) * 4, so, 0);
        s.d = ((d0 >> (16 * (r16 & 1))) & 0xffffu) | (((d1 >> (16 * (r16 & 1))) & 0xffffu) << 16);
#pragma unroll
        for (int h = 0; h < NH; h++) {
            const int src = 16 * g + 4 * h + (lane & 3);
#pragma unroll
            for (int ks = 0; ks < 4; ks++) s.a[h][ks] = ld4(xr, a_off + ks * 1024 + src * 16, xo);
            s.dx[h] = __builtin_bit_cast(float4, ld4(xr, g2_rec_dx(BM) + 16 * h, xo));
        }
    };
    v4f2_t y[NH][2];
#pragma unroll
    for (int h = 0; h < NH; h++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++) y[h][nt] = (v4f2_t){0.0f, 0.0f, 0.0f, 0.0f};
    auto compute = [&](const Stage &s) {
        v4i2_t S[NH][2];
#pragma unroll
        for (int h = 0; h < NH; h++)
#pragma unroll
            for (int nt = 0; nt < 2; nt++) S[h][nt] = (v4i2_t){0, 0, 0, 0};
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            v4i2_t am[NH];
#pragma unroll
            for (int h = 0; h < NH; h++) am[h] = __builtin_bit_cast(v4i2_t, s.a[h][ks]);
#pragma unroll
            for (int nt = 0; nt < 2; nt++) {
                const uint32_t w0 = nt ? s.nib[ks].z : s.nib[ks].x;
                const uint32_t w1 = nt ? s.nib[ks].w : s.nib[ks].y;
                const uint4 hv = s.hi[ks >> 1];
                const uint32_t H = (ks & 1) ? (nt ? hv.w : hv.z) : (nt ? hv.y : hv.x);
                const uint32_t m4 = 0x0F0F0F0Fu, m2 = 0x30303030u;
                const uint32_t q0 = (w0 & m4) | ((H << 4) & m2);
                const uint32_t q1 = (w1 & m4) | ((H << 2) & m2);
                const uint32_t q2 = ((w0 >> 4) & m4) | (H & m2);
                const uint32_t q3 = ((w1 >> 4) & m4) | ((H >> 2) & m2);
                // q - 32 per byte: q + 96 stays below 256 (no carries), and
                // flipping bit 7 gives the int8 of q - 32
                const uint32_t k60 = 0x60606060u, k80 = 0x80808080u;
                const v4i2_t b = {(int)((q0 + k60) ^ k80), (int)((q1 + k60) ^ k80),
                                  (int)((q2 + k60) ^ k80), (int)((q3 + k60) ^ k80)};
                // this lane's group scale: group 4 ks + g of its row
                const uint32_t scw = ks == 0 ? s.sc[nt].x : ks == 1 ? s.sc[nt].y : ks == 2 ? s.sc[nt].z : s.sc[nt].w;
                const int sc = sbfe8(scw, 8u * (uint32_t)g);
#pragma unroll
                for (int h = 0; h < NH; h++) {
                    const v4i2_t z = {0, 0, 0, 0};
                    const v4i2_t P = __builtin_amdgcn_mfma_i32_16x16x64_i8(am[h], b, z, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; i++) S[h][nt][i] += __mul24(sc, P[i]);  // |P| < 2^17
                }
            }
        }
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const float dw = half_to_float((s.d >> (16 * nt)) & 0xffffu);
#pragma unroll
            for (int h = 0; h < NH; h++) {
                const float dxv[4] = {s.dx[h].x, s.dx[h].y, s.dx[h].z, s.dx[h].w};
#pragma unroll
                for (int i = 0; i < 4; i++) y[h][nt][i] = fma_f32(dxv[i] * dw, (float)S[h][nt][i], y[h][nt][i]);
            }
        }
    };
    Stage s0, s1;
    int c = wave;
    if (c < A.nb) load(c, s0);
    while (c < A.nb) {
        if (c + KW < A.nb) load(c + KW, s1);
        compute(s0);
        c += KW;
        if (c >= A.nb) break;
        if (c + KW < A.nb) load(c + KW, s0);
        compute(s1);
        c += KW;
    }
    // add the 4 lane groups (each holds the sums over its own scale groups):
    // partners l ^ 16, then l ^ 32, the same order in every lane
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
