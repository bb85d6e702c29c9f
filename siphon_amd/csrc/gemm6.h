// Prefill GEMM for Q6_K weights on v_mfma_i32_16x16x64_i8 (gfx950):
// Y[M x n_out] = X[M x n_in] * W^T with X quantized per row to Q8_K by the
// bit-exact quantizer (reference kernels.c:561-595), each output within
// the tolerance of the reference dot (reference kernels.c:480-523).
//
// Arithmetic per super-block c, weight row n, activation row m (the
// reference dot restated):
//   S[m,n] = sum_j sc_j[n] * sum_{k in group j} (q[n,k] - 32) * x[m,k]   (exact int)
//   y[m,n] += dx[m,c] * d[n,c] * S
// with 16 groups j of 16 elements, int8 scales sc_j and 6-bit quants q.
// Each weight value v = (q - 32) * sc lies in [-4096, 4064]; the weight
// copy stores it as two int8 digits, v = 128 hi + lo with lo in [-64, 63]
// and hi in [-32, 32], so two MFMAs per K-step (H against the hi digits,
// L against the lo digits) give S = 128 H + L exactly in int32 (|S| <
// 256 * 4096 * 127 < 2^28). The decode of the 6-bit quants and the scale
// products happen once, when the copy is built, so the loop issues no
// operand arithmetic: per super-block and 16 x 16 output tile, 8 MFMAs and
// a 4-instruction epilogue per accumulator register (combine, convert,
// scale by d, FMA with dx).
//
// Tiles and activation records are those of the Q4_K 16x16 GEMM (gemm2.h):
// a workgroup of 4 waves computes BM = 16 MT activation rows against 128
// weight rows, wave w owning rows 32 w .. 32 w + 31 (two 16-column n
// tiles); the activation record of a super-block is copied to LDS by DMA,
// double buffered. A wave's digit operands of a super-block (64 VGPRs) are
// reloaded K-step by K-step for the next super-block as soon as each
// K-step's MFMAs are issued. K slices
// (S > 1) split the super-blocks of a tile over S workgroups whose partial
// sums are added in slice order (g2_slices_finish), for shapes whose output
// tiles alone would leave CUs idle.
#pragma once

#include "agent.h"
#include "formats.h"
#include "gemm2.h"
#include "unit.h"

namespace sihip {

// ---- weight copy in the order of this kernel ----------------------------------
//
// Per block of 32 weight rows and super-block c, one chunk of 16512 bytes:
//   [0, 16384):     16 operand pieces of 64 lanes x 16 bytes, piece
//                   (2 ks + nt) * 2 + digit (0: hi, 1: lo): lane l holds
//                   row 16 nt + l % 16, elements 64 ks + 16 (l / 16) .. + 15
//                   (scale group 4 ks + l / 16), the operand order of the
//                   activation fragments
//   [16384, 16512): per row, f32 d
constexpr int kG6Chunk = 16512;
constexpr int kG6D = 16384;

__host__ __device__ inline int64_t gemm6_layout_bytes(int64_t nblk32, int64_t nb) {
    return nblk32 * nb * kG6Chunk;
}

// One thread per 16-byte piece of a chunk (1032 per chunk); rows past n_out
// are zero.
__global__ __launch_bounds__(256) void gemm6_layout_q6k(Layout L, const uint8_t *planes,
                                                        uint8_t *out, int64_t nblk32) {
    const int64_t nb = L.n_in / 256;
    constexpr int per = kG6Chunk / 16;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nblk32 * nb * per) return;
    const int64_t chunk = i / per;
    const int p = (int)(i % per);
    const int64_t blk = chunk / nb, c = chunk % nb;
    uint32_t v[4] = {0, 0, 0, 0};
    if (p < kG6D / 16) {
        const int piece = p >> 6, l = p & 63;
        const int ks = piece >> 2, nt = (piece >> 1) & 1, digit = piece & 1;
        const int g = l >> 4;
        const int64_t row = blk * 32 + 16 * nt + (l & 15);
        if (row < L.n_out) {
            // unit 2 ks + g / 2 of the super-block, its elements 16 (g % 2) .. + 15
            const int k = 2 * ks + (g >> 1), half = g & 1;
            const int64_t u = c * 8 + k;
            const U4 ql = ldp<U4>(planes + unit_off(L, 0, row, u));
            const U2 qh = ldp<U2>(planes + unit_off(L, 1, row, u));
            uint32_t q[8];
            nib_split(ql, q);
            two8_split(qh.x, qh.y, q, 4, true);
            const U4 m = ldp<U4>(planes + block_off(L, 2, row, u));
            const int sc = sbfe8(u4_word(m, k >> 1), 16 * (k & 1) + 8 * half);
            for (int e = 0; e < 16; e++) {
                const int idx = 16 * half + e;
                const int val = ((int)((q[idx >> 2] >> (8 * (idx & 3))) & 0xffu) - 32) * sc;
                const int hi = (val + 64) >> 7;  // floor: lo = val - 128 hi in [-64, 63]
                const int dv = digit ? val - 128 * hi : hi;
                v[e >> 2] |= (uint32_t)(dv & 0xff) << (8 * (e & 3));
            }
        }
    } else {  // d of rows 4 k .. 4 k + 3
        const int k = p - kG6D / 16;
        for (int t = 0; t < 4; t++) {
            const int64_t row = blk * 32 + 4 * k + t;
            if (row < L.n_out) {
                const uint32_t dd = ldp<uint16_t>(planes + block_off(L, 3, row, c * 8));
                v[t] = __float_as_uint(half_to_float(dd));
            }
        }
    }
    *reinterpret_cast<uint4 *>(out + i * 16) = make_uint4(v[0], v[1], v[2], v[3]);
}

// ---- the GEMM -----------------------------------------------------------------

struct G6Args {
    const uint8_t *w;     // weight chunks [nblk32][nb]
    const uint8_t *x;     // activation records [MB][nb] (gemm2_quantize_x)
    float *y;             // Y[m * ldy + n]
    int64_t ldy;
    int64_t n_out, M, Mp;
    int nb, MB, NB;       // super-blocks; m blocks of BM rows; n blocks of 128 rows
    // K slices: S == 1, one workgroup per output tile; S > 1, slice s covers
    // super-blocks [s SBK, (s + 1) SBK) and its partial sums go to
    // part[(s Mp + m) * NB * 128 + n], the tile's arrivals to
    // cnt[mblk * NB + nblk] (zero between launches)
    int S, SBK;
    float *part;
    uint32_t *cnt;
};

// At least two waves per SIMD (256 registers each at most), no upper
// bound: 116 VGPRs at MT = 1 and 160 at MT = 2 leave room for three or
// four waves per SIMD, 232 at MT = 4 for two.
template <int MT>
__global__ __launch_bounds__(kG2Threads)
__attribute__((amdgpu_waves_per_eu(2))) void gemm6_q6k_kernel(G6Args A) {
    constexpr int BM = 16 * MT;
    constexpr int kRec = g2_rec_bytes(BM);
    constexpr int kXP = kRec / 16;                           // 16-byte pieces of a record
    constexpr int kXPT = (kXP + kG2Threads - 1) / kG2Threads;  // per thread
    __shared__ __attribute__((aligned(16))) uint8_t sx0[kRec];
    __shared__ __attribute__((aligned(16))) uint8_t sx1[kRec];
    // XCD-aware order: workgroups go round-robin over the 8 XCDs, so the m
    // blocks and slices of one n block (which read the same weights) are
    // consecutive workgroups of one XCD and share its L2
    const int b = blockIdx.x;
    const int xcd = b & 7, t = b >> 3;
    const int per = A.MB * A.S;
    const int nblk = (t / per) * 8 + xcd, rest = t % per;
    const int slice = rest / A.MB, mblk = rest % A.MB;
    if (nblk >= A.NB) return;
    const int c0 = slice * A.SBK;
    const int c1 = c0 + A.SBK < A.nb ? c0 + A.SBK : A.nb;  // this slice's super-blocks
    // wave index as a scalar: the buffer resources below derive from it
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, r16 = lane & 15;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(A.w + (int64_t)(nblk * 4 + wave) * A.nb * kG6Chunk), (short)0, A.nb * kG6Chunk,
        0x00020000);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(A.x + (int64_t)mblk * A.nb * kRec), (short)0, A.nb * kRec, 0x00020000);
    const int v_op = lane * 16, v_d = kG6D + r16 * 4;

    // the activation record of a super-block: each thread loads its pieces
    // into registers at the start of a step and writes them to the other LDS
    // buffer at its end, so the loads have the whole step to arrive (an LDS
    // DMA would make the compiler wait for it before every later LDS read)
    uint4 xs[kXPT];
    auto load_x = [&](int c) {
#pragma unroll
        for (int k = 0; k < kXPT; k++) {
            const int i = (int)threadIdx.x + kG2Threads * k;
            if (kXP % kG2Threads == 0 || i < kXP)
                xs[k] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      xr, (int)threadIdx.x * 16, c * kRec + 4096 * k, 0));
        }
    };
    auto store_x = [&](uint8_t *dst) {
#pragma unroll
        for (int k = 0; k < kXPT; k++) {
            const int i = (int)threadIdx.x + kG2Threads * k;
            if (kXP % kG2Threads == 0 || i < kXP) *reinterpret_cast<uint4 *>(dst + i * 16) = xs[k];
        }
    };
    struct Ops {
        v4i2_t b[4][2][2];  // [ks][nt][hi, lo]
        float d[2];
    };
    auto load_w = [&](int c, Ops &o) {
        const int so = c * kG6Chunk;
#pragma unroll
        for (int ks = 0; ks < 4; ks++)
#pragma unroll
            for (int nt = 0; nt < 2; nt++)
#pragma unroll
                for (int dg = 0; dg < 2; dg++)
                    o.b[ks][nt][dg] = __builtin_bit_cast(
                        v4i2_t, __builtin_amdgcn_raw_buffer_load_b128(
                                    wr, v_op, so + ((2 * ks + nt) * 2 + dg) * 1024, 0));
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
            o.d[nt] = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(wr, v_d, so + nt * 64, 0));
    };

    v4f2_t y[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++) y[mt][nt] = (v4f2_t){0.0f, 0.0f, 0.0f, 0.0f};

    // One super-block c on the operands in o and the record in X. K-step ks
    // of every m tile runs before K-step ks + 1, and the next super-block's
    // operands of K-step ks are loaded into o as soon as its MFMAs have been
    // issued, three quarters of a step ahead of their use (all m tiles'
    // accumulators stay live instead of a second operand set; loading a
    // whole second set a step ahead spills at MT = 4, and MT = 4 ffn_down
    // 4096 x 14336 at M = 512 took 114 us that way, 101 us this way). The
    // next record is loaded at the start and written to xn at the end;
    // loads are unconditional (the last super-block of the slice loads
    // itself again).
    auto step = [&](int c, Ops &o, const uint8_t *X, uint8_t *xn) {
        __syncthreads();
        const int cn = c + 1 < c1 ? c + 1 : c;
        load_x(cn);
        v4i2_t h[MT][2], l[MT][2];
        const int so = cn * kG6Chunk;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const v4i2_t a = *reinterpret_cast<const v4i2_t *>(X + (4 * mt + ks) * 1024 + lane * 16);
                const v4i2_t z = {0, 0, 0, 0};
#pragma unroll
                for (int nt = 0; nt < 2; nt++) {
                    h[mt][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, o.b[ks][nt][0], ks ? h[mt][nt] : z, 0, 0, 0);
                    l[mt][nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, o.b[ks][nt][1], ks ? l[mt][nt] : z, 0, 0, 0);
                }
            }
#pragma unroll
            for (int nt = 0; nt < 2; nt++)
#pragma unroll
                for (int dg = 0; dg < 2; dg++)
                    o.b[ks][nt][dg] = __builtin_bit_cast(
                        v4i2_t, __builtin_amdgcn_raw_buffer_load_b128(
                                    wr, v_op, so + ((2 * ks + nt) * 2 + dg) * 1024, 0));
            __builtin_amdgcn_sched_barrier(0);
        }
        const float d0 = o.d[0], d1 = o.d[1];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const float4 dx = *reinterpret_cast<const float4 *>(X + g2_rec_dx(BM) + (16 * mt + 4 * g) * 4);
            const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float u0 = d0 * (float)(128 * h[mt][0][i] + l[mt][0][i]);
                const float u1 = d1 * (float)(128 * h[mt][1][i] + l[mt][1][i]);
                y[mt][0][i] = fma_f32(dxv[i], u0, y[mt][0][i]);
                y[mt][1][i] = fma_f32(dxv[i], u1, y[mt][1][i]);
            }
        }
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
            o.d[nt] = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(wr, v_d, so + nt * 64, 0));
        store_x(xn);
    };

    Ops o;
    load_x(c0);
    load_w(c0, o);
    store_x(sx0);
    for (int c = c0; c < c1; c += 2) {
        step(c, o, sx0, sx1);
        if (c + 1 < c1) step(c + 1, o, sx1, sx0);
    }

    // result register i of lane l: row 4 (l / 16) + i of the m tile,
    // column l % 16 of the n tile
    const int64_t n0 = (int64_t)nblk * kG2BN + 32 * wave;
    const int64_t m0 = (int64_t)mblk * BM;
    if (A.S == 1) {
        // whole tiles inside M and n_out store without per-element tests
        const bool full = n0 + 32 <= A.n_out && m0 + BM <= A.M;
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const int64_t n = n0 + 16 * nt + r16;
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int64_t m = m0 + 16 * mt + 4 * g + i;
                    if (full || (m < A.M && n < A.n_out)) A.y[m * A.ldy + n] = y[mt][nt][i];
                }
        }
        return;
    }
    // K slices: the partial tile in register order through agent-scope
    // stores (they write through and are read past the per-XCD L2s), then
    // the tile's arrival and the last workgroup's slice-order sum
    const int64_t per_slice = (int64_t)A.MB * A.NB * (BM * kG2BN);
    float *const pt = A.part + ((int64_t)mblk * A.NB + nblk) * (BM * kG2BN);  // slice 0
    g2_store_partial<MT>(pt + slice * per_slice, wave, threadIdx.x & 63, y, 1.0f, A.M - m0);
    g2_slices_finish<MT>(pt, per_slice, A.cnt + (int64_t)mblk * A.NB + nblk, A.S, m0, A.M,
                         (int64_t)nblk * kG2BN, A.n_out, A.y, A.ldy);
}

}  // namespace sihip
