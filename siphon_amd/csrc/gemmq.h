// Batch and prefill GEMM for the formats that pair with Q8_0 activations
// (Q4_0, Q5_0, Q8_0) on v_mfma_i32_16x16x32_i8 (gfx950): one MFMA K-step
// is one 32-element block. Per block b, weight row n, activation row m (the
// reference dots, kernels.c:197-247, restated):
//   S[m,n] = sum_{k in b} u[n,k] * xq[m,k] - bias * sx[m,b]  (exact int)
//   y[m,n] += S * (d[n,b] * dx[m,b])
// with u the stored quant (Q4_0: 0..15, bias 8; Q5_0: 0..31, bias 16; Q8_0:
// -128..127, bias 0) and sx the sum of the block's activation quants. The
// quantizer stores -bias * sx per row, and the MFMA takes it as its C input,
// so the bias costs nothing per output. The activation is quantized per row
// by the bit-exact Q8_0 quantizer of the matvec path (reference
// kernels_avx2.c:594-645).
//
// Tiles follow the 16x16 K-quant GEMMs: a workgroup of 4 waves computes
// BM = 16 MT activation rows against 128 weight rows, wave w owning rows
// 32 w .. 32 w + 31 (two 16-column n tiles). A step covers 128 elements
// (4 blocks). The weights and the activation record of a workgroup's
// steps stream through a ring of gq_depth(MT) register sets (22 VGPRs each
// for Q5_0 at MT = 1), up to 3 steps ahead of the MFMAs, so a short K
// slice has most of its loads in flight at once. The record rides in the
// ring rather than being loaded a step ahead: loads retire in issue order,
// so waiting for a record loaded at the start of the previous step would
// also wait for every weight load issued before it. A step's record is
// copied from its ring slot into LDS at the end of the step before; where a
// K slice's records fit 64 KB (16- and 32-row m blocks), all of them are
// copied into LDS before the first step instead, and the ring carries only
// weights. K slices split a tile's steps over several workgroups when the
// output tiles alone would leave the chip idle.
#pragma once

#include "agent.h"
#include "formats.h"
#include "gemm2.h"
#include "quant.h"
#include "unit.h"

namespace sihip {

typedef int v4iq_t __attribute__((ext_vector_type(4)));

// ---- activation records ----------------------------------------------------
//
// One record per (block of BM rows, step c of 128 elements):
//   [0, 128 BM):        quants, fragment (m tile mt, block j) at 512 (4 mt + j):
//                       lane l holds row 16 mt + l % 16, elements
//                       128 c + 32 j + 8 (l / 16) .. + 7
//   [128 BM, 144 BM):   f32 dx, [j][row]
//   [144 BM, 160 BM):   int32 -BIAS times the sum of the block's quants,
//                       [j][row] (the MFMA's C input)
__host__ __device__ constexpr int gq_rec_bytes(int BM) { return 160 * BM; }
__host__ __device__ constexpr int gq_rec_dx(int BM) { return 128 * BM; }
__host__ __device__ constexpr int gq_rec_bs(int BM) { return 144 * BM; }

// Block j of a step, row mr of its m block, into the step's record R.
template <int BM, int BIAS>
__device__ inline void gq_put_block(uint8_t *R, int mr, int j, const Q80Block &q) {
    // lane group g of the fragment takes elements 8 g .. 8 g + 7 (words 2g, 2g+1)
    uint8_t *frag = R + (4 * (mr >> 4) + j) * 512;
#pragma unroll
    for (int g = 0; g < 4; g++)
        *reinterpret_cast<uint64_t *>(frag + (16 * g + (mr & 15)) * 8) =
            (uint64_t)q.q[2 * g] | ((uint64_t)q.q[2 * g + 1] << 32);
    reinterpret_cast<float *>(R + gq_rec_dx(BM))[j * BM + mr] = q.d;
    reinterpret_cast<int *>(R + gq_rec_bs(BM))[j * BM + mr] = -BIAS * q.sum;
}

// Q8_0 block i (row m = i / (n_in / 32), block kb) of X into its record;
// rows M..Mp-1 are zero.
template <int BM, int BIAS>
__device__ inline void gq_quantize_one(const float *x, int64_t ldx, int64_t M, int64_t n_in,
                                       uint8_t *rec, int64_t i, int scalar) {
    const int64_t nbl = n_in / 32;
    const int64_t m = i / nbl, kb = i % nbl;
    const int64_t c = kb / 4;
    const int j = (int)(kb % 4);
    Q80Block q;
    if (m < M) {
        q = q80_block_sel(x + m * ldx + kb * 32, scalar);
    } else {
        q.d = 0.0f;
        q.sum = 0;
        for (int t = 0; t < 8; t++) q.q[t] = 0;
    }
    const int64_t mb = m / BM;
    const int mr = (int)(m % BM);
    gq_put_block<BM, BIAS>(rec + (mb * (n_in / 128) + c) * gq_rec_bytes(BM), mr, j, q);
}

// One thread per Q8_0 block (row m, block kb); rows M..Mp-1 are zero.
// Consecutive threads take consecutive rows of one block column (Mp is a
// multiple of 16), so the record stores of 16 threads fill whole lines
// (16 rows x 8 bytes per fragment piece, 16 rows' scales and sums).
template <int BM, int BIAS>
__global__ __launch_bounds__(256) void gemmq_quantize_x(const float *x, int64_t ldx, int64_t M,
                                                        int64_t Mp, int64_t n_in, uint8_t *rec,
                                                        int scalar) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= Mp * (n_in / 32)) return;
    gq_quantize_one<BM, BIAS>(x, ldx, M, n_in, rec, (i % Mp) * (n_in / 32) + i / Mp, scalar);
}

// ---- weight copy in the order of this kernel ----------------------------------
//
// Per block of 32 weight rows and step c (4 blocks), one chunk, in the
// order [block / 4][c][block % 4]: the four waves of a workgroup read one
// contiguous run per step (12 KB for Q5_0) instead of four streams apart
// (with 3 KB runs per wave and stream, more workgroups made the GEMM slower
// past about 4 TB/s). Each chunk holds:
//   Q8_0 (4608 B): quants, piece (j, nt) at 512 (2 j + nt), lane l: row
//                  16 nt + l % 16, elements 32 j + 8 (l / 16) .. + 7 (8 bytes);
//                  then f32 d, 16 bytes per row (its 4 blocks) at 4096
//   Q4_0 (2560 B): quants, piece nt at 1024 nt, lane l: row 16 nt + l % 16,
//                  one word per block j (16 bytes): the nibbles of elements
//                  32 j + 8 (l / 16) + e, e = 0..3 in the low nibbles of
//                  bytes e, e = 4..7 in the high nibbles of bytes e - 4;
//                  then f32 d at 2048
//   Q5_0 (3072 B): Q4_0's quants and d (at 2048), then the fifth bits,
//                  piece nt at 2560 + 256 nt, one word per lane l: the bit
//                  of element 32 j + 8 (l / 16) + e at 8 e + 4 + j (e < 4)
//                  or 8 (e - 4) + j (e >= 4), so that a shift by j (right
//                  for elements 0..3, left by 4 - j for 4..7) and one mask
//                  put the bits of block j at bit 4 of each operand byte
template <uint32_t FMT>
__host__ __device__ constexpr int gq_chunk() {
    return FMT == T_Q8_0 ? 4608 : FMT == T_Q4_0 ? 2560 : 3072;
}
template <uint32_t FMT>
__host__ __device__ constexpr int gq_d_off() {
    return FMT == T_Q8_0 ? 4096 : 2048;
}
constexpr int kGQHigh = 2560;

template <uint32_t FMT>
__host__ __device__ inline int64_t gemmq_layout_bytes(int64_t nblk32, int64_t nk) {
    return nblk32 * nk * gq_chunk<FMT>();
}

// The quants u of unit (row, block) as 8 dwords, byte k of q[t] = element
// 4 t + k, and its f32 scale.
template <uint32_t FMT>
__device__ inline void gq_unit(const Layout &L, const uint8_t *planes, int64_t row, int64_t kb,
                               uint32_t q[8], float &d) {
    Planes P;
#pragma unroll
    for (int p = 0; p < 4; p++) P.p[p] = planes + L.plane_off[p];
    Raw w;
    load_unit<FMT>(P, (uint32_t)col_rec(L, row, kb), w);
    if constexpr (FMT == T_Q8_0) {
        q[0] = w.a.x; q[1] = w.a.y; q[2] = w.a.z; q[3] = w.a.w;
        q[4] = w.b.x; q[5] = w.b.y; q[6] = w.b.z; q[7] = w.b.w;
    } else {
        nib_split(w.a, q);
        if constexpr (FMT == T_Q5_0) add_bit4(q, w.f, 4);
    }
    d = half_to_float(w.e & 0xffffu);
}

// One thread per (32-row block, step, row r, block j... ) piece: threads
// cover the chunk in 16-byte pieces; rows past n_out are zero.
template <uint32_t FMT>
__global__ __launch_bounds__(256) void gemmq_layout(Layout L, const uint8_t *planes, uint8_t *out,
                                                    int64_t nblk32) {
    const int64_t nk = L.n_in / 128;
    constexpr int per = gq_chunk<FMT>() / 16;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nblk32 * nk * per) return;
    const int64_t chunk = i / per;
    const int p = (int)(i % per);
    const int64_t rem = chunk % (4 * nk);
    const int64_t blk = chunk / (4 * nk) * 4 + rem % 4, c = rem / 4;
    uint32_t v[4] = {0, 0, 0, 0};
    const int off = p * 16;
    if (off < gq_d_off<FMT>()) {
        if constexpr (FMT == T_Q8_0) {
            // two lanes per piece: piece (j, nt) lane pair
            const int piece = off / 512, lp = (off % 512) / 8;  // first lane of the pair
            const int j = piece >> 1, nt = piece & 1;
            for (int h = 0; h < 2; h++) {
                const int l = lp + h;
                const int64_t row = blk * 32 + 16 * nt + (l & 15);
                if (row >= L.n_out) continue;
                uint32_t q[8];
                float d;
                gq_unit<FMT>(L, planes, row, 4 * c + j, q, d);
                const int g = l >> 4;
                v[2 * h] = q[2 * g];
                v[2 * h + 1] = q[2 * g + 1];
            }
        } else {
            const int nt = off / 1024, l = (off % 1024) / 16;
            const int64_t row = blk * 32 + 16 * nt + (l & 15);
            if (row < L.n_out) {
                const int g = l >> 4;
                for (int j = 0; j < 4; j++) {
                    uint32_t q[8];
                    float d;
                    gq_unit<FMT>(L, planes, row, 4 * c + j, q, d);
                    // elements 8 g .. 8 g + 7: q[2g] bytes e, q[2g + 1] bytes e - 4
                    const uint32_t lo = q[2 * g] & 0x0F0F0F0Fu, hi = q[2 * g + 1] & 0x0F0F0F0Fu;
                    v[j] = lo | (hi << 4);
                }
            }
        }
    } else if (FMT != T_Q5_0 || off < kGQHigh) {  // d of rows (off - doff) / 16
        const int r = (off - gq_d_off<FMT>()) / 16;
        const int64_t row = blk * 32 + r;
        if (row < L.n_out)
            for (int j = 0; j < 4; j++) {
                uint32_t q[8];
                float d;
                gq_unit<FMT>(L, planes, row, 4 * c + j, q, d);
                v[j] = __float_as_uint(d);
            }
    } else {  // Q5_0 fifth bits: 4 lanes per piece
        const int q0 = (off - kGQHigh) / 4;  // first (nt, lane) index of the piece
        for (int h = 0; h < 4; h++) {
            const int idx = q0 + h, nt = idx >> 6, l = idx & 63;
            const int64_t row = blk * 32 + 16 * nt + (l & 15);
            if (row >= L.n_out) continue;
            const int g = l >> 4;
            uint32_t word = 0;
            for (int j = 0; j < 4; j++) {
                uint32_t q[8];
                float d;
                gq_unit<FMT>(L, planes, row, 4 * c + j, q, d);
                for (int e = 0; e < 8; e++) {
                    const uint32_t bit = (q[2 * g + (e >> 2)] >> (8 * (e & 3) + 4)) & 1u;
                    word |= bit << (e < 4 ? 8 * e + 4 + j : 8 * (e - 4) + j);
                }
            }
            v[h] = word;
        }
    }
    *reinterpret_cast<uint4 *>(out + i * 16) = make_uint4(v[0], v[1], v[2], v[3]);
}

// ---- the GEMM -----------------------------------------------------------------

struct GQArgs {
    const uint8_t *w;     // weight chunks [nblk32 / 4][nk][4]
    const uint8_t *x;     // activation records [MB][nk]
    float *y;             // Y[m * ldy + n]
    int64_t ldy;
    int64_t n_out, M, Mp;
    int nk, MB, NB;
    int S, SBK;           // K slices over steps
    float *part;
    uint32_t *cnt;
    int q80s;             // the scalar Q8_0 quantizer (q80_block_sel)
    const float *xf;      // XM 2: X[m * ldx + k], f32, quantized by the launch itself
    int64_t ldx;
};

// steps in flight per wave: a ring of gq_depth(MT) register sets (two at
// MT = 4, whose accumulators leave no room for four)
__host__ __device__ constexpr int gq_depth(int MT) { return MT >= 4 ? 2 : 4; }

// Dynamic LDS of gemmq_kernel<.., XM = 1>: the records of sbk steps in
// whole KiBs. That mode runs where it is at most kGQSliceLds.
__host__ __device__ constexpr int64_t gq_lds_bytes(int BM, int64_t sbk) {
    return (sbk * gq_rec_bytes(BM) + 1023) / 1024 * 1024;
}
constexpr int64_t kGQSliceLds = 64 * 1024;

// At least two waves per SIMD (256 registers each at most); no upper bound,
// so the register count sets the occupancy: 124 VGPRs at MT = 1, 168 at
// MT = 2, 134 at MT = 4 (three or four waves per SIMD), where an upper
// bound of two would make the compiler reserve registers for two.
//
// XM, where a workgroup's activation records come from:
//   0: through the register ring into two LDS buffers, a step ahead;
//   1: all records of its K slice copied into LDS (dynamic, gq_lds_bytes)
//      before the first step, so the steps read LDS only, with no record
//      loads, LDS stores or barriers between them;
//   2: as 1, but the workgroup quantizes its K slice of X (f32, A.xf) into
//      the same LDS image itself, one Q8_0 block per thread and pass (the
//      quantizer of the separate launch, so the records are the same
//      bytes), and no quantization launch runs before it. Each thread's
//      first block of X is requested before the ring's first weights, so
//      the quantization waits only for X (loads retire in issue order).
template <uint32_t FMT, int MT, int XM>
__global__ __launch_bounds__(kG2Threads)
__attribute__((amdgpu_waves_per_eu(2))) void gemmq_kernel(GQArgs A) {
    static_assert(XM == 0 || XM == 1 || XM == 2, "record modes 0, 1 and 2");
    constexpr int BM = 16 * MT;
    constexpr int kRec = gq_rec_bytes(BM);
    constexpr int kXP = kRec / 16;
    constexpr int kXPT = (kXP + kG2Threads - 1) / kG2Threads;
    constexpr int kChunk = gq_chunk<FMT>();
    constexpr int kD = gq_depth(MT);
    constexpr int bias = FMT == T_Q4_0 ? 8 : FMT == T_Q5_0 ? 16 : 0;
    // whole 4 KiB rounds, so every thread loads and stores each round: a
    // conditional last round splits the step into blocks, and the compiler
    // then sinks the epilogues below it, keeping every MFMA result live
    constexpr int kSx = kXPT * 4096;
    __shared__ __attribute__((aligned(16))) uint8_t sx0[XM == 0 ? kSx : 16];
    __shared__ __attribute__((aligned(16))) uint8_t sx1[XM == 0 ? kSx : 16];
    extern __shared__ __attribute__((aligned(16))) uint8_t gq_slice[];
    const int b = (int)blockIdx.x;
    const int xcd = b & 7, t = b >> 3;
    const int per = A.MB * A.S;
    const int nblk = (t / per) * 8 + xcd, rest = t % per;
    const int slice = rest / A.MB, mblk = rest % A.MB;
    if (nblk >= A.NB) return;
    const int c0 = slice * A.SBK;
    const int c1 = c0 + A.SBK < A.nk ? c0 + A.SBK : A.nk;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, r16 = lane & 15;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(A.w + (int64_t)nblk * A.nk * 4 * kChunk), (short)0, A.nk * 4 * kChunk,
        0x00020000);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(A.x + (int64_t)mblk * A.nk * kRec), (short)0, A.nk * kRec, 0x00020000);

    // this lane's weights of one step and this thread's pieces of its
    // activation record
    struct Ops {
        uint2 q8[4][2];   // Q8_0: [block][nt]
        uint4 nib[2];     // Q4_0/Q5_0: [nt], word per block
        uint32_t hb[2];   // Q5_0: [nt], the fifth bits of the 4 blocks
        float4 d[2];      // [nt], f32 d of the lane's row for the 4 blocks
        uint4 xs[kXPT];   // record pieces tid + 256 k
    };
    // pieces past the record read the next record (or zero past the buffer
    // end) into the padding of the LDS copy, which nothing reads
    auto store_x = [&](const Ops &o, uint8_t *dst) {
#pragma unroll
        for (int k = 0; k < kXPT; k++)
            *reinterpret_cast<uint4 *>(dst + ((int)threadIdx.x + kG2Threads * k) * 16) = o.xs[k];
    };
    auto load_x = [&](int c, Ops &o) {
#pragma unroll
        for (int k = 0; k < kXPT; k++)
            o.xs[k] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                    xr, (int)threadIdx.x * 16, c * kRec + 4096 * k, 0));
    };
    auto load_wt = [&](int c, Ops &o) {
        const int so = (c * 4 + wave) * kChunk;
        if constexpr (FMT == T_Q8_0) {
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int nt = 0; nt < 2; nt++)
                    o.q8[j][nt] = __builtin_bit_cast(
                        uint2, __builtin_amdgcn_raw_buffer_load_b64(wr, lane * 8, so + (2 * j + nt) * 512, 0));
        } else {
#pragma unroll
            for (int nt = 0; nt < 2; nt++)
                o.nib[nt] = __builtin_bit_cast(
                    uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, lane * 16, so + nt * 1024, 0));
            if constexpr (FMT == T_Q5_0) {
#pragma unroll
                for (int nt = 0; nt < 2; nt++)
                    o.hb[nt] = __builtin_amdgcn_raw_buffer_load_b32(wr, lane * 4, so + kGQHigh + nt * 256, 0);
            }
        }
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
            o.d[nt] = __builtin_bit_cast(
                float4, __builtin_amdgcn_raw_buffer_load_b128(wr, r16 * 16, so + gq_d_off<FMT>() + nt * 256, 0));
    };
    auto load_w = [&](int c, Ops &o) {
        load_x(c, o);
        load_wt(c, o);
    };
    // the MFMA operand (8 quants) of block j, n tile nt
    auto operand = [&](const Ops &o, int j, int nt) -> long {
        if constexpr (FMT == T_Q8_0) {
            return __builtin_bit_cast(long, o.q8[j][nt]);
        } else {
            const uint32_t w = j == 0 ? o.nib[nt].x : j == 1 ? o.nib[nt].y : j == 2 ? o.nib[nt].z : o.nib[nt].w;
            uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
            if constexpr (FMT == T_Q5_0) {
                lo |= (o.hb[nt] >> j) & 0x10101010u;
                hi |= (o.hb[nt] << (4 - j)) & 0x10101010u;
            }
            return __builtin_bit_cast(long, make_uint2(lo, hi));
        }
    };

    v4f2_t y[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++) y[mt][nt] = (v4f2_t){0.0f, 0.0f, 0.0f, 0.0f};

    // step c: the record in X, the weights in cur; step c + kD - 1
    // goes into the ring slot the previous step freed, and the record of
    // step c + 1 (in slot nxt) into the other LDS buffer
    auto step = [&](int c, const Ops &cur, Ops &ahead, const Ops &nxt, const uint8_t *X,
                    uint8_t *xn) {
        __syncthreads();
        const int ca = c + kD - 1 < c1 ? c + kD - 1 : c1 - 1;
        load_w(ca, ahead);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const long b0 = operand(cur, j, 0), b1 = operand(cur, j, 1);
            const float dw0 = j == 0 ? cur.d[0].x : j == 1 ? cur.d[0].y : j == 2 ? cur.d[0].z : cur.d[0].w;
            const float dw1 = j == 0 ? cur.d[1].x : j == 1 ? cur.d[1].y : j == 2 ? cur.d[1].z : cur.d[1].w;
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const long a = *reinterpret_cast<const long *>(X + (4 * mt + j) * 512 + lane * 8);
                const int off = (j * BM + 16 * mt + 4 * g) * 4;
                v4iq_t cb = {0, 0, 0, 0};
                if constexpr (bias != 0) cb = *reinterpret_cast<const v4iq_t *>(X + gq_rec_bs(BM) + off);
                const v4iq_t s0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b0, cb, 0, 0, 0);
                const v4iq_t s1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b1, cb, 0, 0, 0);
                const float4 dx = *reinterpret_cast<const float4 *>(X + gq_rec_dx(BM) + off);
                const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    y[mt][0][i] = fma_f32((float)s0[i], dw0 * dxv[i], y[mt][0][i]);
                    y[mt][1][i] = fma_f32((float)s1[i], dw1 * dxv[i], y[mt][1][i]);
                }
            }
        }
        store_x(nxt, xn);
    };
    // XM 1: step c with the slice's records in LDS and only the weights
    // in the ring
    auto step_lds = [&](int c, const Ops &cur, Ops &ahead) {
        const int ca = c + kD - 1 < c1 ? c + kD - 1 : c1 - 1;
        load_wt(ca, ahead);
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t *X = gq_slice + (c - c0) * kRec;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const long b0 = operand(cur, j, 0), b1 = operand(cur, j, 1);
            const float dw0 = j == 0 ? cur.d[0].x : j == 1 ? cur.d[0].y : j == 2 ? cur.d[0].z : cur.d[0].w;
            const float dw1 = j == 0 ? cur.d[1].x : j == 1 ? cur.d[1].y : j == 2 ? cur.d[1].z : cur.d[1].w;
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const long a = *reinterpret_cast<const long *>(X + (4 * mt + j) * 512 + lane * 8);
                const int off = (j * BM + 16 * mt + 4 * g) * 4;
                v4iq_t cb = {0, 0, 0, 0};
                if constexpr (bias != 0) cb = *reinterpret_cast<const v4iq_t *>(X + gq_rec_bs(BM) + off);
                const v4iq_t s0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b0, cb, 0, 0, 0);
                const v4iq_t s1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b1, cb, 0, 0, 0);
                const float4 dx = *reinterpret_cast<const float4 *>(X + gq_rec_dx(BM) + off);
                const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    y[mt][0][i] = fma_f32((float)s0[i], dw0 * dxv[i], y[mt][0][i]);
                    y[mt][1][i] = fma_f32((float)s1[i], dw1 * dxv[i], y[mt][1][i]);
                }
            }
        }
    };

    Ops o[kD];
    if constexpr (XM == 0) {
        // kD (even) steps per round, so the LDS buffer of step c is sx0 for
        // c - c0 even and sx1 for c - c0 odd
        static_assert(kD % 2 == 0, "LDS buffers alternate by step");
#pragma unroll
        for (int u = 0; u + 1 < kD; u++) load_w(c0 + u < c1 ? c0 + u : c1 - 1, o[u]);
        store_x(o[0], sx0);
        // whole rounds of kD steps without conditions, then the last
        // partial round: a condition inside the round splits it into blocks,
        // and the compiler's wait counts at the joins assume the loads of a
        // skipped step were never issued, so every step waited for the
        // ring's later slots too (the ring then bought no depth)
        int c = c0;
        for (; c + kD <= c1; c += kD) {
#pragma unroll
            for (int u = 0; u < kD; u++)
                step(c + u, o[u], o[(u + kD - 1) % kD], o[(u + 1) % kD], (u & 1) ? sx1 : sx0,
                     (u & 1) ? sx0 : sx1);
        }
#pragma unroll
        for (int u = 0; u < kD; u++)
            if (c + u < c1)
                step(c + u, o[u], o[(u + kD - 1) % kD], o[(u + 1) % kD], (u & 1) ? sx1 : sx0,
                     (u & 1) ? sx0 : sx1);
    } else if constexpr (XM == 1) {
        // the first weights go out first
#pragma unroll
        for (int u = 0; u + 1 < kD; u++) load_wt(c0 + u < c1 ? c0 + u : c1 - 1, o[u]);
        // the slice's records, 1 KiB per wave instruction straight into LDS
        // (whole KiBs: the last may read into the next record, or zero past
        // the buffer, into LDS that no step reads)
        const int kib = ((c1 - c0) * kRec + 1023) / 1024;
        for (int i = wave; i < kib; i += kG2Threads / 64)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xr, (__attribute__((address_space(3))) void *)(gq_slice + i * 1024), 16, lane * 16,
                c0 * kRec + i * 1024, 0, 0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        for (int c = c0; c < c1; c += kD) {
#pragma unroll
            for (int u = 0; u < kD; u++)
                if (c + u < c1) step_lds(c + u, o[u], o[(u + kD - 1) % kD]);
        }
    } else {
        // the slice's blocks: nq = BM rows x 4 per step, block i = row i / nb4,
        // block i % nb4 of the slice; rows past M are zero
        const int nb4 = 4 * (c1 - c0), nq = BM * nb4;
        const int64_t m0q = (int64_t)mblk * BM;
        auto src = [&](int i, int &mr, int &kb) -> const float * {
            mr = i / nb4;
            kb = i - mr * nb4;
            return A.xf + (m0q + mr) * A.ldx + (int64_t)c0 * 128 + 32 * kb;
        };
        auto put = [&](int mr, int kb, const Q80Block &q) {
            gq_put_block<BM, bias>(gq_slice + (kb >> 2) * kRec, mr, kb & 3, q);
        };
        // this thread's first block before the weights
        const int i0 = (int)threadIdx.x;
        int mr0 = 0, kb0 = 0;
        const float *s0 = i0 < nq ? src(i0, mr0, kb0) : A.xf;
        const bool live0 = i0 < nq && m0q + mr0 < A.M;
        float v0[32];
        if (live0) q80_load(s0, v0);
#pragma unroll
        for (int u = 0; u + 1 < kD; u++) load_wt(c0 + u < c1 ? c0 + u : c1 - 1, o[u]);
        if (i0 < nq) {
            Q80Block q;
            if (live0) {
                q = q80_block_sel_v(v0, A.q80s);
            } else {
                q.d = 0.0f;
                q.sum = 0;
                for (int t = 0; t < 8; t++) q.q[t] = 0;
            }
            put(mr0, kb0, q);
        }
        for (int i = i0 + kG2Threads; i < nq; i += kG2Threads) {
            int mr, kb;
            const float *sx = src(i, mr, kb);
            Q80Block q;
            if (m0q + mr < A.M) {
                q = q80_block_sel(sx, A.q80s);
            } else {
                q.d = 0.0f;
                q.sum = 0;
                for (int t = 0; t < 8; t++) q.q[t] = 0;
            }
            put(mr, kb, q);
        }
        __syncthreads();
        for (int c = c0; c < c1; c += kD) {
#pragma unroll
            for (int u = 0; u < kD; u++)
                if (c + u < c1) step_lds(c + u, o[u], o[(u + kD - 1) % kD]);
        }
    }

    const int64_t n0 = (int64_t)nblk * kG2BN + 32 * wave;
    const int64_t m0 = (int64_t)mblk * BM;
    if (A.S == 1) {
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
