// Fused small-M GEMM for the K-quant weights (Q2_K .. Q6_K, M <= 8
// activation rows: the batched decode step), one launch per group of
// matrices that share X: Y_i[M x n_out_i] = X[M x n_in] * W_i^T, each output
// within the tolerance of the reference dot (reference kernels.c:249-523;
// the per-super-block arithmetic and the weight copy are gemmks.h's).
//
// Against gemmks_kernel (a separate quantization launch, one launch per
// matrix, a workgroup per 32 rows whose waves split that block's
// super-blocks) this launch
//   - quantizes X itself: each workgroup converts the M rows of its K slice
//     to Q8_K (the bit-exact 16-lane quantizer of quant.h, reference
//     kernels.c:561-595) straight into LDS, in the masked-operand order the
//     MFMAs read, while the first weights of every wave are in flight; no
//     activation records go through memory and no second launch is needed;
//   - covers several matrices (segments, up to two weight formats F0, F1)
//     with one flat grid;
//   - cuts the K dimension into slices when the row blocks alone would not
//     fill the chip: a workgroup owns a tile of kKFWaves 32-row blocks and
//     one slice of SBK super-blocks, each wave one block of the tile and
//     every super-block of the slice (a ring of SW super-blocks of weights
//     in registers), so each wave streams a contiguous run of its block's
//     chunks and no partial sums meet inside the workgroup. With S > 1
//     slices the slices' partial tiles go through agent-scope stores and
//     the last workgroup of a tile adds them in slice order
//     (kf_finish), so the result does not depend on arrival order.
#pragma once

#include "agent.h"
#include "gemmks.h"

namespace sihip {

constexpr int kKFWaves = 4;                   // waves per workgroup = 32-row blocks per tile
constexpr int kKFThreads = 64 * kKFWaves;
constexpr int kKFRows = 32 * kKFWaves;        // weight rows per tile
constexpr int kKFMaxSegs = 4;
constexpr int kKFMaxSBK = 24;                 // super-blocks of a K slice
constexpr int kKFRec = 2304 + 32;             // LDS bytes per super-block
constexpr int kKFMp = 8;                      // activation rows of the partial sums
constexpr int kKFMaxM = 8;

// LDS image of one super-block of the slice: the quants of rows 0..7 as
// [K-step ks][lane group g][row][16 bytes] (the 16 elements 64 ks + 16 g ..
// + 15 of the super-block), each (ks, g) run padded to 9 rows so that the 4
// lane groups of a wave's reads, and the 16 lanes of a quantizer's stores,
// start on different banks; then the 8 block scales dx.
__host__ __device__ constexpr int kf_q_off(int ks, int g, int row) {
    return ((ks * 4 + g) * 9 + row) * 16;
}
constexpr int kKFDx = 2304;

struct GKFSeg {
    const uint8_t *w;   // gemmks.h chunks [nblk][nb]
    float *y;           // Y[m * ldy + n]
    int64_t ldy, n_out;
    float *part;        // S > 1: partial sums [S][ntile][kKFMp * kKFRows], register order (kf_finish)
    uint32_t *cnt;      // S > 1: arrival counters [ntile], zero between launches
    uint32_t type;
    int nblk;           // 32-row blocks
    int ntile;          // tiles of kKFWaves blocks
    int S, SBK;         // K slices, super-blocks per slice
    int wg0;            // first workgroup of the segment
};

struct GKFArgs {
    const float *x;
    int64_t ldx, M;
    int nb;             // super-blocks per row (n_in / 256)
    int nseg;
    GKFSeg seg[kKFMaxSegs];
};

// The prologue: rows 0..M-1 of X over super-blocks c0 .. c0 + nc - 1 are
// quantized into the LDS images, 16 lanes per 256-element block,
// kKFThreads / 16 blocks per pass (a 16-lane group enters or leaves a pass
// whole). The X values of the first kKFPre passes are requested before the
// first weights (kf_x_first), so the quantization waits only for them: the
// memory counter retires loads in order, and X requested after the weights
// would wait for the weights' HBM latency too. Loads past the last block
// read block 0 again (nothing stores them), so every load is unconditional.
constexpr int kKFPre = 4;
struct KFXFirst {
    float4 t[kKFPre][4];
};

__device__ inline const float4 *kf_x_src(const GKFArgs &A, int c0, int idx) {
    const int M = (int)A.M;
    const int cl = idx / M, m = idx - cl * M;
    return reinterpret_cast<const float4 *>(A.x + (int64_t)m * A.ldx + (int64_t)(c0 + cl) * 256 +
                                            (threadIdx.x & 15) * 16);
}

__device__ inline void kf_x_first(const GKFArgs &A, int c0, int nc, KFXFirst &xf) {
    const int nq = (int)A.M * nc;
#pragma unroll
    for (int p = 0; p < kKFPre; p++) {
        const int idx = p * (kKFThreads / 16) + (int)(threadIdx.x >> 4);
        const float4 *src = kf_x_src(A, c0, idx < nq ? idx : 0);
#pragma unroll
        for (int i = 0; i < 4; i++) xf.t[p][i] = src[i];
    }
}

__device__ inline void kf_quantize_one(const GKFArgs &A, int idx, const float4 (&t)[4],
                                       uint8_t *lds) {
    const int M = (int)A.M;
    const int lane16 = threadIdx.x & 15;
    const int cl = idx / M, m = idx - cl * M;
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[4 * i] = t[i].x; v[4 * i + 1] = t[i].y; v[4 * i + 2] = t[i].z; v[4 * i + 3] = t[i].w;
    }
    const Q8KRow r = q8k_block_row16(v, lane16);
    uint8_t *R = lds + cl * kKFRec;
    *reinterpret_cast<uint4 *>(R + kf_q_off(lane16 >> 2, lane16 & 3, m)) = r.q;
    if (lane16 == 0) reinterpret_cast<float *>(R + kKFDx)[m] = r.d;
}

// The rest of the prologue after kf_x_first: quantizes its passes, then the
// remaining ones (load, quantize), and zeroes rows M .. ROWS - 1, which the
// MFMAs read.
template <int ROWS>
__device__ inline void kf_prologue(const GKFArgs &A, int c0, int nc, const KFXFirst &xf,
                                   uint8_t *lds) {
    const int M = (int)A.M;
    const int nq = M * nc;
#pragma unroll
    for (int p = 0; p < kKFPre; p++) {
        const int idx = p * (kKFThreads / 16) + (int)(threadIdx.x >> 4);
        if (idx < nq) kf_quantize_one(A, idx, xf.t[p], lds);
    }
    for (int base = kKFPre * (kKFThreads / 16); base < nq; base += kKFThreads / 16) {
        const int idx = base + (int)(threadIdx.x >> 4);
        if (idx < nq) {
            const float4 *src = kf_x_src(A, c0, idx);
            float4 t[4];
#pragma unroll
            for (int i = 0; i < 4; i++) t[i] = src[i];
            kf_quantize_one(A, idx, t, lds);
        }
    }
    constexpr int rows = ROWS;
    if (M < rows) {
        const int nz = nc * (rows - M) * 17;  // 16 quant pieces and a scale per row
        for (int e = threadIdx.x; e < nz; e += kKFThreads) {
            const int cl = e / ((rows - M) * 17), rem = e - cl * ((rows - M) * 17);
            const int row = M + rem / 17, k = rem % 17;
            uint8_t *R = lds + cl * kKFRec;
            if (k < 16)
                *reinterpret_cast<uint4 *>(R + kf_q_off(k >> 2, k & 3, row)) = make_uint4(0, 0, 0, 0);
            else
                reinterpret_cast<float *>(R + kKFDx)[row] = 0.0f;
        }
    }
}

// One super-block for the formats with a scale and min per 32-element unit
// (Q4_K, Q5_K): the activation operand is masked two ways, so one MFMA per
// K-step and n tile covers all 8 activation rows. A row r of the operand
// holds x[r % 8] in the K slots of lane groups 2 (r / 8), + 1 (one unit)
// and zeros elsewhere, so result register i of lane l (lane group g) is
// the unscaled sum over unit 2 ks + g / 2 for activation row 4 (g % 2) + i,
// which is the unit whose scale and min the lane holds (gemmks.h's copy):
//   S[i] += s * P[i]  (an integer multiply-add per result)
// and the mins run on the matrix core against the lane's min in all 16 of
// its slots, accumulated over the K-steps in the MFMA itself:
//   T = sum_ks MFMA(x_ks, m_ks)  (exact: |T| < 2^21)
// y[nt][i] += dx_i * (d * S - dmin * T); lanes g and g ^ 2 (the two units
// of a K-step) are added after the last super-block.
template <uint32_t FMT>
__device__ inline void kf_compute_u2(const KSWStage<FMT> &s, const uint4 (&a)[4], float4 dx,
                                     int r16, v4f2_t (&y)[2]) {
    static_assert(KS<FMT>::unit32, "unit-scale formats only");
    v4i2_t S[2], T[2];
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        S[nt] = (v4i2_t){0, 0, 0, 0};
        T[nt] = (v4i2_t){0, 0, 0, 0};
    }
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        const v4i2_t am = __builtin_bit_cast(v4i2_t, a[ks]);
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const v4i2_t b = ks_operand<FMT>(s, ks, nt);
            const int sv = (int)((s.sc[nt][0] >> (8 * ks)) & 0xffu);
            // the unit's min (byte ks) in every byte
            const int mb = (int)__builtin_amdgcn_perm(s.sc[nt][1], s.sc[nt][1], 0x01010101u * ks);
            const v4i2_t z = {0, 0, 0, 0};
            const v4i2_t P = __builtin_amdgcn_mfma_i32_16x16x64_i8(am, b, z, 0, 0, 0);
            T[nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(am, (v4i2_t){mb, mb, mb, mb}, T[nt], 0, 0, 0);
            // |P| < 2^17 and s <= 63: 24-bit operands, products below 2^23
#pragma unroll
            for (int i = 0; i < 4; i++) S[nt][i] += __mul24(sv, P[i]);
        }
    }
    const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        const uint32_t dword = s.d[nt];  // d in the low, dmin in the high half
        const float dw = half_to_float(dword & 0xffffu);
        const float ndm = -half_to_float(dword >> 16);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float u = fma_f32(dw, (float)S[nt][i], ndm * (float)T[nt][i]);
            y[nt][i] = fma_f32(dxv[i], u, y[nt][i]);
        }
    }
}

// One super-block for Q2_K, whose 2-bit quant times its 4-bit group scale
// fits an int8 (q s <= 45): the scale is folded into the weight operand
// (one 32-bit multiply per operand dword: bytes below 256, no carries) and
// the activation operand is not masked, so the MFMAs accumulate the scaled
// sums over the whole super-block themselves, for up to 16 activation rows:
//   S = sum_ks MFMA(x_ks, q s),  T = sum_ks MFMA(x_ks, m)   (exact integers)
// with m the lane's group min in all 16 of its slots. Result register i of
// lane l is complete for activation row 4 (l / 16) + i; rows 8..15 are
// zeros here (M <= 8). y[nt][i] += dx_i * (d * S - dmin * T).
__device__ inline void kf_compute_fold(const KSWStage<T_Q2_K> &s, const uint4 (&a)[4], float4 dx,
                                       v4f2_t (&y)[2]) {
    v4i2_t S[2], T[2];
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        S[nt] = (v4i2_t){0, 0, 0, 0};
        T[nt] = (v4i2_t){0, 0, 0, 0};
    }
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        const v4i2_t am = __builtin_bit_cast(v4i2_t, a[ks]);
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const v4i2_t q = ks_operand<T_Q2_K>(s, ks, nt);
            // group 4 ks + g at byte ks: the scale in the low, the min in
            // the high nibble
            const uint32_t b = (s.sc[nt][0] >> (8 * ks)) & 0xffu;
            const uint32_t sv = b & 15u;
            const int mb = (int)((b >> 4) * 0x01010101u);
            const v4i2_t qs = {(int)((uint32_t)q[0] * sv), (int)((uint32_t)q[1] * sv),
                               (int)((uint32_t)q[2] * sv), (int)((uint32_t)q[3] * sv)};
            S[nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(am, qs, S[nt], 0, 0, 0);
            T[nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(am, (v4i2_t){mb, mb, mb, mb}, T[nt], 0, 0, 0);
        }
    }
    const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        const uint32_t dword = s.d[nt];  // d in the low, dmin in the high half
        const float dw = half_to_float(dword & 0xffffu);
        const float ndm = -half_to_float(dword >> 16);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float u = fma_f32(dw, (float)S[nt][i], ndm * (float)T[nt][i]);
            y[nt][i] = fma_f32(dxv[i], u, y[nt][i]);
        }
    }
}

// End of a K-sliced tile after each wave has issued the agent-scope stores
// of its slice's partial sums in the registers' order: the 1024 floats of
// slice s at pt + s * per_slice, float 256 w + 32 (4 nt + i) + l holding
// result register i of lane l (< 32) of wave w's n tile nt, which is
// activation row 4 (l / 16) + i, column 32 w + 16 nt + l % 16 of the tile.
// Stored that way each store instruction writes whole 128-byte lines and
// the last workgroup reads a slice with one 16-byte load per thread (the
// same partial sums scattered row by row as 64-byte pieces took 1.8 us more
// per launch at M = 8). Counting and ordering as slices_finish (agent.h):
// each wave's stores complete before the barrier that precedes the count,
// the last of the S workgroups adds the slices in slice order and resets
// the counter.
__device__ inline void kf_finish(const float *pt, int64_t per_slice, uint32_t *cnt, int S,
                                 int64_t M, int64_t n0, int64_t n_out, float *y, int64_t ldy) {
    static_assert(kKFThreads * 4 == kKFWaves * 256, "one float4 of a slice per thread");
    __shared__ uint32_t last_flag;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (threadIdx.x == 0)
        last_flag = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                    (uint32_t)S - 1;
    __syncthreads();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (!last_flag) return;
    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(pt), (short)0, (int)(((int64_t)(S - 1) * per_slice + kKFWaves * 256) * 4),
        0x00020000);
    const uint32_t t4 = threadIdx.x * 16u;  // this thread's 16 bytes of a slice
    // slices in groups of 8 whose loads are issued together (each group
    // costs one round trip: agent-scope loads miss the XCD's L2), added in
    // slice order
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < S; s0 += 8) {
        uint4 pv[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int s = s0 + k < S ? s0 + k : S - 1;
            pv[k] = __builtin_bit_cast(
                uint4, __builtin_amdgcn_raw_buffer_load_b128(pr, (int)((int64_t)s * per_slice * 4 + t4), 0, 16));
        }
#pragma unroll
        for (int k = 0; k < 8; k++)
            if (s0 + k < S) {
                v[0] += __uint_as_float(pv[k].x);
                v[1] += __uint_as_float(pv[k].y);
                v[2] += __uint_as_float(pv[k].z);
                v[3] += __uint_as_float(pv[k].w);
            }
    }
    // floats 4 t .. 4 t + 3: wave w, register (nt, i), lanes l .. l + 3 (one
    // lane group): row 4 (l / 16) + i, columns 32 w + 16 nt + l % 16 + j
    const int k = 4 * (int)threadIdx.x;
    const int w = k >> 8, r = k & 255;
    const int nt = r >> 7, i = (r >> 5) & 3, l = r & 31;
    const int64_t m = 4 * (l >> 4) + i;
    const int64_t n = n0 + 32 * w + 16 * nt + (l & 15);
    if (m < M) {
        float *const dst = y + m * ldy + n;
        if (n + 3 < n_out && ((uintptr_t)dst & 15) == 0) {
            *reinterpret_cast<float4 *>(dst) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++)
                if (n + j < n_out) dst[j] = v[j];
        }
    }
    if (threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The workgroup's share of segment sg: tile t % ntile, slice t / ntile.
template <uint32_t FMT, int NH>
__device__ inline void kf_body(const GKFArgs &A, const GKFSeg &sg, int t, uint8_t *lds) {
    using F = KS<FMT>;
    constexpr int SW = gemmks_sw<FMT, NH>();
    const int tile = t % sg.ntile, slice = t / sg.ntile;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, r16 = lane & 15;
    const int blk = tile * kKFWaves + wave;
    const bool has = blk < sg.nblk;  // wave-uniform; a wave past the last block only stages
    const int c0 = slice * sg.SBK;
    const int c1 = c0 + sg.SBK < A.nb ? c0 + sg.SBK : A.nb;
    const int bw = has ? blk : sg.nblk - 1;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(sg.w + (int64_t)bw * A.nb * F::chunk), (short)0, A.nb * F::chunk, 0x00020000);
    // the ring: super-block c uses weight set (c - c0) % SW; loads past the
    // slice read its last super-block again (nothing computes them), so
    // every load is unconditional and the compiler's wait counts stay exact
    auto cl = [&](int c) { return c < c1 - 1 ? c : c1 - 1; };
    KFXFirst xf;
    kf_x_first(A, c0, c1 - c0, xf);
    KSWStage<FMT> ws[SW];
#pragma unroll
    for (int k = 0; k < SW - 1; k++) ks_load_w<FMT>(wr, cl(c0 + k), lane, ws[k]);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    // unit-scale formats: the two-way masked operand of all 8 rows (one
    // result tile per n tile); Q2_K: the unmasked operand (scales folded
    // into the weights); the others: gemmks.h's four-way masked operand of
    // 4 rows per MFMA, NH of them
    constexpr bool U2 = F::unit32;
    constexpr bool FOLD = FMT == T_Q2_K;
    constexpr int YH = U2 || FOLD ? 1 : NH;
    kf_prologue<U2 || FOLD ? 8 : 4 * NH>(A, c0, c1 - c0, xf, lds);
    __syncthreads();

    v4f2_t y[YH][2];
#pragma unroll
    for (int h = 0; h < YH; h++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++) y[h][nt] = (v4f2_t){0.0f, 0.0f, 0.0f, 0.0f};
    // four-way (gemmks.h): lane l carries row 4 h + l % 4 of lane group
    // l / 16's K slots when l % 16 / 4 == l / 16, else zeros; two-way: row
    // l % 8 when l % 16 / 8 == l / 32, else zeros; unmasked: row l % 16
    // (zeros past row 7)
    const bool own = FOLD ? r16 < 8 : U2 ? (r16 >> 3) == (g >> 1) : (r16 >> 2) == g;
    auto load_x = [&](int c, KSXStage<NH> &x) {
        const uint8_t *R = lds + (c - c0) * kKFRec;
#pragma unroll
        for (int h = 0; h < NH; h++) {
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                const uint4 v = *reinterpret_cast<const uint4 *>(R + kf_q_off(ks, g, 4 * h + (lane & 3)));
                x.a[h][ks] = own ? v : make_uint4(0, 0, 0, 0);
            }
            x.dx[h] = *reinterpret_cast<const float4 *>(R + kKFDx + 16 * h);
        }
    };
    auto load_x2 = [&](int c, uint4 (&a)[4], float4 &dx) {
        const uint8_t *R = lds + (c - c0) * kKFRec;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const uint4 v = *reinterpret_cast<const uint4 *>(R + kf_q_off(ks, g, r16 & 7));
            a[ks] = own ? v : make_uint4(0, 0, 0, 0);
        }
        dx = *reinterpret_cast<const float4 *>(R + kKFDx + 16 * (g & 1));
    };
    auto load_x1 = [&](int c, uint4 (&a)[4], float4 &dx) {
        const uint8_t *R = lds + (c - c0) * kKFRec;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const uint4 v = *reinterpret_cast<const uint4 *>(R + kf_q_off(ks, g, r16 & 7));
            a[ks] = own ? v : make_uint4(0, 0, 0, 0);
        }
        // rows 4 g .. 4 g + 3 (lane groups 2 and 3 hold padding rows)
        dx = *reinterpret_cast<const float4 *>(R + kKFDx + 16 * (g & 1));
    };
    if (has) {
        for (int cb = c0; cb < c1; cb += SW) {
#pragma unroll
            for (int j = 0; j < SW; j++) {
                const int c = cb + j;
                ks_load_w<FMT>(wr, cl(c + SW - 1), lane, ws[(j + SW - 1) % SW]);
                asm volatile("" ::: "memory");
                __builtin_amdgcn_sched_barrier(0);
                if (c < c1) {
                    if constexpr (FOLD) {
                        uint4 a[4];
                        float4 dx;
                        load_x1(c, a, dx);
                        kf_compute_fold(ws[j % SW], a, dx, y[0]);
                    } else if constexpr (U2) {
                        uint4 a[4];
                        float4 dx;
                        load_x2(c, a, dx);
                        kf_compute_u2<FMT>(ws[j % SW], a, dx, r16, y[0]);
                    } else {
                        KSXStage<NH> x;
                        load_x(c, x);
                        ks_compute<FMT, NH>(ws[j % SW], x, r16, y);
                    }
                }
            }
        }
        if constexpr (FOLD) {
            // complete in every lane
        } else if constexpr (U2) {  // the two units of a K-step: lanes l and l ^ 32
#pragma unroll
            for (int nt = 0; nt < 2; nt++)
#pragma unroll
                for (int i = 0; i < 4; i++) y[0][nt][i] += __shfl_xor(y[0][nt][i], 32, 64);
        } else {
            ks_add_groups<NH>(y);
        }
    }
    // activation row of result i of y[h]: four-way, lane group h holds rows
    // 4 h .. 4 h + 3 (every lane group has them after the additions);
    // two-way and unmasked, lane groups 0 and 1 hold rows 0..3 and 4..7
    const int64_t n0 = (int64_t)blk * 32;
    auto holds = [&](int h) { return U2 || FOLD ? g < 2 : g == h; };
    auto row_of = [&](int h, int i) { return U2 || FOLD ? 4 * (g & 1) + i : 4 * h + i; };
    if (sg.S == 1) {
        if (has) {
#pragma unroll
            for (int h = 0; h < YH; h++) {
                if (!holds(h)) continue;
#pragma unroll
                for (int nt = 0; nt < 2; nt++) {
                    const int64_t n = n0 + 16 * nt + r16;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int64_t m = row_of(h, i);
                        if (m < A.M && n < sg.n_out) sg.y[m * sg.ldy + n] = y[h][nt][i];
                    }
                }
            }
        }
        return;
    }
    // K slices: the partial tile in the registers' order (kf_finish), lanes
    // 0..31 of each result register one 128-byte line; lane group g (< 2)
    // holds activation rows 4 g .. 4 g + 3 (four-way: of y[g])
    const int64_t per_slice = (int64_t)sg.ntile * kKFWaves * 256;
    float *const pt = sg.part + (int64_t)tile * (kKFWaves * 256);
    if (has && lane < 32) {
        float *const pw = pt + slice * per_slice + wave * 256 + lane;
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float v = YH == 1 || g == 0 ? y[0][nt][i] : y[YH - 1][nt][i];
                __hip_atomic_store(pw + (nt * 4 + i) * 32, v, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
    }
    kf_finish(pt, per_slice, sg.cnt + tile, sg.S, A.M, (int64_t)tile * kKFRows, sg.n_out, sg.y,
              sg.ldy);
}

// Grid: sum over segments of ntile * S workgroups of kKFThreads; dynamic
// LDS: kKFRec bytes per super-block of the largest slice.
template <uint32_t F0, uint32_t F1, int NH>
__global__ __launch_bounds__(kKFThreads)
__attribute__((amdgpu_waves_per_eu(2))) void gemmkf_kernel(GKFArgs A) {
    extern __shared__ __attribute__((aligned(16))) uint8_t kf_lds[];
    const int b = blockIdx.x;
    int i = 0;
#pragma unroll
    for (int k = 1; k < kKFMaxSegs; k++)
        if (k < A.nseg && b >= A.seg[k].wg0) i = k;
    const GKFSeg &sg = A.seg[i];
    if constexpr (F0 == F1) {
        kf_body<F0, NH>(A, sg, b - sg.wg0, kf_lds);
    } else {
        if (sg.type == F0)
            kf_body<F0, NH>(A, sg, b - sg.wg0, kf_lds);
        else
            kf_body<F1, NH>(A, sg, b - sg.wg0, kf_lds);
    }
}

}  // namespace sihip
