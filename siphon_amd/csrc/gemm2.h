// Prefill GEMM for Q4_K weights on v_mfma_i32_16x16x64_i8 (gfx950):
// Y[M x n_out] = X[M x n_in] * W^T with X quantized per row to Q8_K by the
// bit-exact quantizer (reference kernels.c:561-595), each output within
// the tolerance of the reference dot (reference kernels.c:349-410).
//
// Arithmetic per super-block c, weight row n, activation row m (the
// reference dot restated):
//   S[m,n] = sum_j sc_j[n] * sum_{k in unit j} q[n,k] * x[m,k]    (exact int)
//   T[m,n] = sum_g mn_{g/2}[n] * bsum_g[m]                          (exact)
//   y[m,n] += dx[m,c] * (d[n,c] * S - dmin[n,c] * T)
// The 6-bit unit scale is split as sc = 8 sh + sl (sh, sl in 0..7), so both
// weight operands sh * q and sl * q fit in int8 (<= 105); two accumulators
// H and L give S = 8 H + L exactly. The min term runs on one
// v_mfma_f32_16x16x32_f16 whose 32 k-slots hold the 16 group sums twice,
// against hi and lo halves of -dmin * mn * 2^E: dmin * mn has at most
// 17 significant bits, so hi + lo (two f16) is exact and the products with
// the group sums (at most 11 bits) are exact in f32. With d' = d * 2^E
// (exact) the epilogue is two FMAs per output,
//   u = d' * S + T',  yacc += dx * u,
// and the result is yacc * 2^-E at the end. E is chosen per weight so that
// hi stays far inside the f16 range (at most 2^15).
//
// Tiles. A workgroup of 4 waves computes BM = 16 * MT activation rows
// against 128 weight rows; wave w owns weight rows 32 w .. 32 w + 31 (two
// 16-column n tiles). Per super-block each wave decodes its weights once
// (the split operands of 4 K-steps x 2 n tiles: 64 VGPRs) and applies them
// to its MT m tiles one after the other, so the decode is shared by MT m
// tiles while only one m tile's accumulators are live. The activation
// record of the super-block (quants in MFMA operand order, group sums and
// scales of the BM rows) is copied to LDS by DMA, double buffered.
//
// Operand layout of the 16x16 MFMAs (checked on the device): A lane l holds
// row l % 16 at k = KG * (l / 16) + slot (KG = 16 for i8 x64, 8 for f16
// x32); B lane l holds column l % 16 at the same k; result register i of
// lane l is D[4 (l / 16) + i][l % 16]. K-step ks of a super-block covers its
// elements 64 ks .. 64 ks + 63; lane group g takes 64 ks + 16 g + slot,
// which is unit 2 ks + g / 2, elements 16 (g % 2) + slot of the unit.
#pragma once

#include "agent.h"
#include "formats.h"
#include "quant.h"
#include "unit.h"

namespace sihip {

typedef int v4i2_t __attribute__((ext_vector_type(4)));
typedef float v4f2_t __attribute__((ext_vector_type(4)));
typedef _Float16 v8h2_t __attribute__((ext_vector_type(8)));
typedef unsigned short u16x2b_t __attribute__((ext_vector_type(2)));

constexpr int kG2Threads = 256;
constexpr int kG2BN = 128;  // weight rows per workgroup

// ---- activation records ----------------------------------------------------
//
// One record per (m block of BM rows, super-block c), KiB aligned so it is
// copied to LDS in whole 1 KiB DMA pieces:
//   [0, 256 BM):        quants, fragment (mt, ks) at 1024 (4 mt + ks); its
//                       lane l holds 16 bytes: row 16 mt + l % 16, elements
//                       64 ks + 16 (l / 16) .. + 15 of the super-block
//   [256 BM, 288 BM):   f16 group sums, 32 bytes per row
//   [288 BM, 292 BM):   f32 block scale dx per row
__host__ __device__ constexpr int g2_rec_bytes(int BM) { return (BM * 292 + 1023) / 1024 * 1024; }
__host__ __device__ constexpr int g2_rec_bsum(int BM) { return 256 * BM; }
__host__ __device__ constexpr int g2_rec_dx(int BM) { return 288 * BM; }

// One 16-lane row per Q8_K block (row m, super-block c) of X; rows M..Mp-1
// are zero. Grid: gemm2_quantize_grid(Mp * nb) workgroups of 256. (A wave
// per block, 4 elements per lane, measured no faster at M = 512 and slower
// at M = 2048, 14.8 against 13.1 us: its 4-byte record stores.)
constexpr int kG2QBlocks = kG2Threads / 16;  // blocks per workgroup
__host__ __device__ inline int64_t gemm2_quantize_grid(int64_t blocks) {
    return (blocks + kG2QBlocks - 1) / kG2QBlocks;
}

template <int BM>
__global__ __launch_bounds__(kG2Threads) void gemm2_quantize_x(const float *x, int64_t ldx,
                                                               int64_t M, int64_t Mp, int64_t nb,
                                                               uint8_t *rec) {
    const int lane16 = threadIdx.x & 15;
    const int64_t blk = (int64_t)blockIdx.x * (kG2Threads / 16) + (threadIdx.x >> 4);
    if (blk >= Mp * nb) return;  // whole 16-lane rows leave together
    // a workgroup takes 16 consecutive rows of one super-block column (Mp is
    // a multiple of 16), so its record stores fill whole cache lines (16 rows
    // x 16 bytes per piece) instead of 16-byte pieces of lines that other
    // workgroups complete
    const int64_t m = blk % Mp, c = blk / Mp;
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
    const int64_t mb = m / BM;
    const int mr = (int)(m % BM);
    uint8_t *R = rec + (mb * nb + c) * g2_rec_bytes(BM);
    // elements 16 lane16 .. + 15: K-step lane16 / 4, lane group lane16 % 4
    const int mt = mr >> 4, ks = lane16 >> 2, g = lane16 & 3;
    *reinterpret_cast<uint4 *>(R + (4 * mt + ks) * 1024 + (16 * g + (mr & 15)) * 16) = r.q;
    reinterpret_cast<_Float16 *>(R + g2_rec_bsum(BM) + mr * 32)[lane16] = (_Float16)(float)r.gsum;
    if (lane16 == 0) reinterpret_cast<float *>(R + g2_rec_dx(BM))[mr] = r.d;
}

// ---- weight copy in the order of this kernel (Q4_K) ---------------------------
//
// Per block of 32 weight rows and super-block c, one chunk of 6784 bytes:
//   [0, 4096):     quants, 4 pieces (ks) of 64 lanes x 16 bytes: lane l, rows
//                  16 nt + l % 16 for nt = 0, 1 in bytes 8 nt .. 8 nt + 7:
//                  the 16 nibbles of lane group l / 16 as two words w0, w1,
//                  byte b of w0 = slot b | slot 8 + b << 4, of w1 = slot
//                  4 + b | slot 12 + b << 4 (masks and one shift decode them)
//   [4096, 4608):  per row, sh_0..sh_7 then sl_0..sl_7 (sc_j = 8 sh_j + sl_j)
//   [4608, 4736):  per row, f32 d * 2^E
//   [4736, 6784):  min operand, 2 n tiles x 64 lanes x 8 f16: lane l, row
//                  16 nt + l % 16, groups 8 (l / 16 % 2) .. + 7: hi (l < 32)
//                  or lo (l >= 32) half of -dmin * mn_{group / 2} * 2^E
constexpr int kG2ChunkQ4K = 6784;
constexpr int kG2Scl = 4096, kG2D = 4608, kG2Min = 4736;

__host__ __device__ inline int64_t gemm2_layout_bytes(int64_t nblk32, int64_t nb) {
    return nblk32 * nb * kG2ChunkQ4K;
}

// One thread per 16-byte piece of a chunk (424 per chunk); rows past n_out
// are zero.
__global__ __launch_bounds__(256) void gemm2_layout_q4k(Layout L, const uint8_t *planes,
                                                        uint8_t *out, int64_t nblk32, float e2) {
    const int64_t nb = L.n_in / 256;
    constexpr int per = kG2ChunkQ4K / 16;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nblk32 * nb * per) return;
    const int64_t chunk = i / per;
    const int p = (int)(i % per);
    const int64_t blk = chunk / nb, c = chunk % nb;
    uint32_t v[4] = {0, 0, 0, 0};
    if (p < kG2Scl / 16) {  // quants: K-step p / 64, lane p % 64
        const int ks = p >> 6, l = p & 63, g = l >> 4;
        const int h = g & 1;
        for (int nt = 0; nt < 2; nt++) {
            const int64_t row = blk * 32 + 16 * nt + (l & 15);
            if (row >= L.n_out) continue;
            const uint8_t *rec = planes + unit_off(L, 0, row, c * 8 + 2 * ks + (g >> 1));
            auto slot = [&](int s) -> uint32_t {
                const uint32_t byte = rec[s];
                return h ? byte >> 4 : byte & 15u;
            };
            uint32_t w0 = 0, w1 = 0;
            for (int b = 0; b < 4; b++) {
                w0 |= (slot(b) | (slot(8 + b) << 4)) << (8 * b);
                w1 |= (slot(4 + b) | (slot(12 + b) << 4)) << (8 * b);
            }
            v[2 * nt] = w0;
            v[2 * nt + 1] = w1;
        }
    } else if (p < kG2D / 16) {  // split scales of one row
        const int64_t row = blk * 32 + (p - kG2Scl / 16);
        if (row < L.n_out) {
            const U4 m = ldp<U4>(planes + block_off(L, 1, row, c * 8));
            for (int j = 0; j < 8; j++) {
                int sc, mn;
                k4_scale_min(m, j, sc, mn);
                v[j >> 2] |= (uint32_t)(sc >> 3) << (8 * (j & 3));
                v[2 + (j >> 2)] |= (uint32_t)(sc & 7) << (8 * (j & 3));
            }
        }
    } else if (p < kG2Min / 16) {  // d * 2^E of rows 4 k .. 4 k + 3
        const int k = p - kG2D / 16;
        for (int t = 0; t < 4; t++) {
            const int64_t row = blk * 32 + 4 * k + t;
            if (row < L.n_out) {
                const uint32_t dd = ldp<U4>(planes + block_off(L, 1, row, c * 8)).x;
                v[t] = __float_as_uint(half_to_float(dd & 0xffffu) * e2);
            }
        }
    } else {  // min operand of one lane
        const int q = p - kG2Min / 16, nt = q >> 6, l = q & 63;
        const int64_t row = blk * 32 + 16 * nt + (l & 15);
        if (row < L.n_out) {
            const U4 m = ldp<U4>(planes + block_off(L, 1, row, c * 8));
            const float dmin = half_to_float(m.x >> 16);
            const bool lo = l >= 32;
            for (int s = 0; s < 8; s++) {
                const int grp = 8 * ((l >> 4) & 1) + s;
                int sc, mn;
                k4_scale_min(m, grp >> 1, sc, mn);
                const float val = -dmin * (float)mn * e2;  // exact: 17 significant bits
                const _Float16 hi = (_Float16)val;
                const _Float16 part = lo ? (_Float16)(val - (float)hi) : hi;
                v[s >> 1] |= (uint32_t)__builtin_bit_cast(uint16_t, part) << (16 * (s & 1));
            }
        }
    }
    *reinterpret_cast<uint4 *>(out + i * 16) = make_uint4(v[0], v[1], v[2], v[3]);
}

// ---- the GEMM -----------------------------------------------------------------

// One matrix of a launch: several Q4_K matrices over one X (q and k, gate
// and up) share a grid, their n blocks one after another.
constexpr int kG2MaxSegs = 4;
struct G2Seg {
    const uint8_t *w;     // weight chunks [nblk32][nb]
    float *y;             // Y[m * ldy + n]
    int64_t ldy, n_out;
    float yscale;         // 2^-E
    int nb0;              // the segment's first n block in the grid
};

struct G2Args {
    const uint8_t *x;     // activation records [MB][nb]
    int64_t M, Mp;
    int nb, MB, NB;       // super-blocks; m blocks of BM rows; n blocks of 128 rows (all segments)
    // K slices: S == 1, one workgroup per output tile; S > 1, slice s covers
    // super-blocks [s SBK, (s + 1) SBK) and its partial sums (already scaled
    // by 2^-E) go to part[(s Mp + m) * NB * 128 + 128 nblk + n % 128], the
    // tile's arrivals to cnt[mblk * NB + nblk] (zero between launches)
    int S, SBK;
    float *part;
    uint32_t *cnt;
    int nseg;
    G2Seg seg[kG2MaxSegs];
};

// ---- K slices of the 16x16-tile GEMMs (this file, gemm6.h, gemmh.h, gemmq.h)
//
// A workgroup of 4 waves computes a BM x 128 output tile: wave w columns
// 32 w .. 32 w + 31 as two 16-column n tiles, MT = BM / 16 m tiles; result
// register i of lane l of tile (mt, nt) is row 16 mt + 4 (l / 16) + i,
// column 32 w + 16 nt + l % 16. A K slice's partial tile is stored in that
// register order, float ((w MT + mt) 2 + nt) 256 + 64 i + l of the tile's
// BM * 128 floats (at part + ((slice MB + mblk) NB + nblk) BM 128), so each
// store instruction writes 256 contiguous bytes and the last workgroup
// reads a slice with 16-byte loads. Stored row by row (four 64-byte pieces
// per instruction) the partial sums cost the Llama-3-8B prefill at M = 512
// 2.3-3.5 us per sliced call (a timing copy without them). In 16-row tiles
// (MT = 1) rows at or past M (rows >= `rows` of the tile) are neither
// stored nor read: at M = 8 that halves the hand-off's traffic. (Taller
// tiles store and read them: the extra predicates made the MT = 8 kernels
// spill.)
template <int MT>
__device__ inline void g2_store_partial(float *pt, int wave, int lane, const v4f2_t (&y)[MT][2],
                                        float scale, int64_t rows) {
    float *const pw = pt + wave * (MT * 512) + lane;
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (MT > 1 || 4 * (lane >> 4) + i < rows)
                    __hip_atomic_store(pw + ((mt * 2 + nt) * 4 + i) * 64, y[mt][nt][i] * scale,
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// End of a K-sliced tile after every wave has issued g2_store_partial for
// its slice (pt: the tile's partial in slice 0, per_slice floats between
// slices): the arrival count and ordering of slices_finish (agent.h); the
// last of the S workgroups adds the slices in slice order into y[m * ldy + n]
// for rows m0 + r below M and columns n0 + c below n_out, and resets the
// counter.
template <int MT>
__device__ inline void g2_slices_finish(const float *pt, int64_t per_slice, uint32_t *cnt, int S,
                                        int64_t m0, int64_t M, int64_t n0, int64_t n_out, float *y,
                                        int64_t ldy) {
    constexpr int kQ = MT * 2;  // float4s per thread of a slice's tile (256 threads)
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
        const_cast<float *>(pt), (short)0,
        (int)(((int64_t)(S - 1) * per_slice + MT * 2048) * 4), 0x00020000);
    // floats 4 (q 256 + tid) .. + 3 of a slice's tile: wave w, tile
    // (mt, nt), register i, lanes l .. l + 3, all of one row m; with MT = 1
    // rows at or past M were not stored
    // (recomputed where used: kept in arrays they spilled at MT = 8)
    auto row_of = [&](int q) -> int64_t {
        const int rem = ((q * 256 + (int)threadIdx.x) * 4) % (MT * 512);
        return m0 + 16 * (rem >> 9) + 4 * ((rem & 63) >> 4) + ((rem >> 6) & 3);
    };
    auto col_of = [&](int q) -> int64_t {
        const int k = (q * 256 + (int)threadIdx.x) * 4;
        const int w = k / (MT * 512), rem = k % (MT * 512);
        return n0 + 32 * w + 16 * ((rem >> 8) & 1) + (rem & 15);
    };
    float v[kQ][4];
#pragma unroll
    for (int q = 0; q < kQ; q++) v[q][0] = v[q][1] = v[q][2] = v[q][3] = 0.0f;
    // the loads of kU slices issued together (agent-scope loads miss the
    // XCD's L2: each group is one round trip), the slices added in slice
    // order
    constexpr int kU = kQ >= 8 ? 1 : 8 / kQ;
    auto load = [&](int s, int q) {
        return MT > 1 || row_of(q) < M ? __builtin_bit_cast(
                              uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                         pr, (int)(((int64_t)s * per_slice + (q * 256 + (int)threadIdx.x) * 4) * 4),
                                         0, 16))
                        : make_uint4(0, 0, 0, 0);
    };
    auto add = [&](int q, uint4 p) {
        v[q][0] += __uint_as_float(p.x);
        v[q][1] += __uint_as_float(p.y);
        v[q][2] += __uint_as_float(p.z);
        v[q][3] += __uint_as_float(p.w);
    };
    int s = 0;
    for (; s + kU <= S; s += kU) {
        uint4 pv[kU][kQ];
#pragma unroll
        for (int u = 0; u < kU; u++)
#pragma unroll
            for (int q = 0; q < kQ; q++) pv[u][q] = load(s + u, q);
#pragma unroll
        for (int u = 0; u < kU; u++)
#pragma unroll
            for (int q = 0; q < kQ; q++) add(q, pv[u][q]);
    }
    if constexpr (kU > 1) {
        for (; s < S; s++) {
            uint4 pv[kQ];
#pragma unroll
            for (int q = 0; q < kQ; q++) pv[q] = load(s, q);
#pragma unroll
            for (int q = 0; q < kQ; q++) add(q, pv[q]);
        }
    }
#pragma unroll
    for (int q = 0; q < kQ; q++) {
        const int64_t m = row_of(q);
        if (m < M) {
            const int64_t n_ = col_of(q);
            float *const dst = y + m * ldy + n_;
            if (n_ + 3 < n_out && ((uintptr_t)dst & 15) == 0) {
                *reinterpret_cast<float4 *>(dst) = make_float4(v[q][0], v[q][1], v[q][2], v[q][3]);
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++)
                    if (n_ + j < n_out) dst[j] = v[q][j];
            }
        }
    }
    if (threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// q * f bytewise for bytes and products below 256 (no carries between
// bytes); f2 holds the factor in both 16-bit halves.
__device__ inline uint32_t g2_bytes_times(uint32_t q, uint32_t f2) {
    const u16x2b_t a = __builtin_bit_cast(u16x2b_t, q);
    const u16x2b_t b = __builtin_bit_cast(u16x2b_t, f2);
    return __builtin_bit_cast(uint32_t, (u16x2b_t)(a * b));
}

// W: waves per SIMD the kernel is built for (2: 256 registers each, two
// workgroups per CU; 1: 512, one workgroup per CU).
template <int MT, int W>
__global__ __launch_bounds__(kG2Threads)
__attribute__((amdgpu_waves_per_eu(W, W))) void gemm2_q4k_kernel(G2Args A) {
    constexpr int BM = 16 * MT;
    constexpr int kRec = g2_rec_bytes(BM);
    constexpr int kPieces = kRec / 1024;
    // two LDS objects, not one array indexed by the step's parity: each
    // step reads one and copies the next record into the other, and only
    // distinct objects let the compiler see that the step's LDS reads do
    // not depend on the copy in flight (it otherwise waits for the copy
    // before the first read, which exposes its whole latency)
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
    // the tile's segment, its fields read with constant indices (wave-
    // uniform selects; a reference into the argument array at a computed
    // index made the compiler keep the arguments in scratch memory, and
    // the main loop spilled)
    G2Seg sg = A.seg[0];
#pragma unroll
    for (int k = 1; k < kG2MaxSegs; k++)
        if (k < A.nseg && nblk >= A.seg[k].nb0) sg = A.seg[k];
    const int lblk = nblk - sg.nb0;  // n block within the segment's matrix
    const int c0 = slice * A.SBK;
    const int c1 = c0 + A.SBK < A.nb ? c0 + A.SBK : A.nb;  // this slice's super-blocks
    // wave index as a scalar: the buffer resources below derive from it
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, r16 = lane & 15;
    // buffer resources over this wave's weight chunks and this block's
    // activation records: per-lane offsets are constants, the super-block
    // moves the scalar offset, so no address arithmetic runs on the VALU
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(sg.w + (int64_t)(lblk * 4 + wave) * A.nb * kG2ChunkQ4K), (short)0,
        A.nb * kG2ChunkQ4K, 0x00020000);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(A.x + (int64_t)mblk * A.nb * kRec), (short)0, A.nb * kRec, 0x00020000);
    const int v_nib = lane * 16, v_scl = kG2Scl + r16 * 16, v_d = kG2D + r16 * 4;
    const int v_min = kG2Min + lane * 16;

    // this wave's share of the 1 KiB pieces of a record; every wave issues
    // the same number of copies (a wave past the last piece copies the last
    // piece again: the same bytes to the same place), so the copies are
    // straight-line code with a fixed count
    auto dma = [&](int c, uint8_t *dst) {
#pragma unroll
        for (int k = 0; k < (kPieces + 3) / 4; k++) {
            const int i = wave + 4 * k < kPieces ? wave + 4 * k : kPieces - 1;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xr, (__attribute__((address_space(3))) void *)(dst + i * 1024), 16, v_nib,
                c * kRec + i * 1024, 0, 0);
        }
    };
    struct Raw {
        uint4 nib[4];  // K-step ks: nt 0 in x, y; nt 1 in z, w
        uint4 scl[2];
        float d[2];
        uint4 mn[2];
    };
    auto ld4 = [&](int voff, int soff, int imm) {
        return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wr, voff + imm, soff, 0));
    };
    auto load_w = [&](int c, Raw &r) {
        const int so = c * kG2ChunkQ4K;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) r.nib[ks] = ld4(v_nib, so, ks * 1024);
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            r.scl[nt] = ld4(v_scl, so, nt * 256);
            r.d[nt] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wr, v_d + nt * 64, so, 0));
            r.mn[nt] = ld4(v_min, so, nt * 1024);
        }
    };
    // byte selector of this lane's unit (2 ks + g / 2) in both 16-bit halves
    uint32_t sel[4];
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        const uint32_t u = (uint32_t)(2 * ks + (g >> 1));
        sel[ks] = u | (0x0cu << 8) | (u << 16) | (0x0cu << 24);
    }

    v4f2_t y[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++) y[mt][nt] = (v4f2_t){0.0f, 0.0f, 0.0f, 0.0f};

    Raw raw;
    dma(c0, sx0);
    load_w(c0, raw);
    // one super-block: X holds its record, the next one is copied to Xn
    auto step = [&](int c, const uint8_t *X, uint8_t *Xn) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        // decode this super-block's operands
        v4i2_t bh[4][2], bl[4][2];
#pragma unroll
        for (int ks = 0; ks < 4; ks++)
#pragma unroll
            for (int nt = 0; nt < 2; nt++) {
                const uint32_t w0 = nt ? raw.nib[ks].z : raw.nib[ks].x;
                const uint32_t w1 = nt ? raw.nib[ks].w : raw.nib[ks].y;
                const uint32_t q0 = w0 & 0x0F0F0F0Fu, q1 = w1 & 0x0F0F0F0Fu;
                const uint32_t q2 = (w0 >> 4) & 0x0F0F0F0Fu, q3 = (w1 >> 4) & 0x0F0F0F0Fu;
                const uint32_t sh = __builtin_amdgcn_perm(raw.scl[nt].y, raw.scl[nt].x, sel[ks]);
                const uint32_t sl = __builtin_amdgcn_perm(raw.scl[nt].w, raw.scl[nt].z, sel[ks]);
                bh[ks][nt] = (v4i2_t){(int)g2_bytes_times(q0, sh), (int)g2_bytes_times(q1, sh),
                                      (int)g2_bytes_times(q2, sh), (int)g2_bytes_times(q3, sh)};
                bl[ks][nt] = (v4i2_t){(int)g2_bytes_times(q0, sl), (int)g2_bytes_times(q1, sl),
                                      (int)g2_bytes_times(q2, sl), (int)g2_bytes_times(q3, sl)};
            }
        const float dw[2] = {raw.d[0], raw.d[1]};
        const v8h2_t bm[2] = {__builtin_bit_cast(v8h2_t, raw.mn[0]), __builtin_bit_cast(v8h2_t, raw.mn[1])};
        // the next super-block's record and weights, a whole super-block
        // ahead; unconditional (the last super-block loads itself again), so
        // the registers of the prefetch are the ones decoded next
        const int cn = c + 1 < c1 ? c + 1 : c;
        dma(cn, Xn);
        load_w(cn, raw);
        // keep the copies and loads here, ahead of the tiles' LDS reads
        __builtin_amdgcn_sched_barrier(0);
        // quants of m tile mt + 1 are read while mt computes (ping-pong by
        // the parity of the unrolled tile index); group sums and scales at
        // the start of their own tile, in time for its epilogue
        v4i2_t a[2][4];
        auto lds_q = [&](int mt, v4i2_t (&aa)[4]) {
#pragma unroll
            for (int ks = 0; ks < 4; ks++)
                aa[ks] = *reinterpret_cast<const v4i2_t *>(X + (4 * mt + ks) * 1024 + lane * 16);
        };
        lds_q(0, a[0]);
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            if (mt + 1 < MT) lds_q(mt + 1, a[(mt + 1) & 1]);
            const v8h2_t bs = *reinterpret_cast<const v8h2_t *>(X + g2_rec_bsum(BM) + (16 * mt + r16) * 32 + (g & 1) * 16);
            const float4 dx = *reinterpret_cast<const float4 *>(X + g2_rec_dx(BM) + (16 * mt + 4 * g) * 4);
            const v4i2_t(&am)[4] = a[mt & 1];
            const v4f2_t z = {0.0f, 0.0f, 0.0f, 0.0f};
            const v4f2_t t0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(bs, bm[0], z, 0, 0, 0);
            const v4f2_t t1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(bs, bm[1], z, 0, 0, 0);
            v4i2_t h0 = {0, 0, 0, 0}, h1 = {0, 0, 0, 0}, l0 = {0, 0, 0, 0}, l1 = {0, 0, 0, 0};
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                h0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(am[ks], bh[ks][0], h0, 0, 0, 0);
                l0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(am[ks], bl[ks][0], l0, 0, 0, 0);
                h1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(am[ks], bh[ks][1], h1, 0, 0, 0);
                l1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(am[ks], bl[ks][1], l1, 0, 0, 0);
            }
            const float dxv[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float u0 = fma_f32(dw[0], (float)(8 * h0[i] + l0[i]), t0[i]);
                const float u1 = fma_f32(dw[1], (float)(8 * h1[i] + l1[i]), t1[i]);
                y[mt][0][i] = fma_f32(dxv[i], u0, y[mt][0][i]);
                y[mt][1][i] = fma_f32(dxv[i], u1, y[mt][1][i]);
            }
        }
    };
    int c = c0;
    for (; c + 1 < c1; c += 2) {
        step(c, sx0, sx1);
        step(c + 1, sx1, sx0);
    }
    if (c < c1) step(c, sx0, sx1);
    // result register i of lane l: row 4 (l / 16) + i of the m tile,
    // column l % 16 of the n tile; whole tiles inside M and n_out store
    // without per-element tests
    const int64_t n0 = (int64_t)lblk * kG2BN + 32 * wave;  // within the segment's matrix
    const int64_t m0 = (int64_t)mblk * BM;
    if (A.S == 1) {
        const bool full = n0 + 32 <= sg.n_out && m0 + BM <= A.M;
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            const int64_t n = n0 + 16 * nt + r16;
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int64_t m = m0 + 16 * mt + 4 * g + i;
                    if (full || (m < A.M && n < sg.n_out)) sg.y[m * sg.ldy + n] = y[mt][nt][i] * sg.yscale;
                }
        }
        return;
    }
    // K slices: the partial tile (already scaled by 2^-E) in register order
    // through agent-scope stores (they write through and are read past the
    // per-XCD L2s), then the tile's arrival and the last workgroup's
    // slice-order sum into the segment's columns
    const int64_t per_slice = (int64_t)A.MB * A.NB * (BM * kG2BN);
    float *const pt = A.part + ((int64_t)mblk * A.NB + nblk) * (BM * kG2BN);  // slice 0
    g2_store_partial<MT>(pt + slice * per_slice, wave, lane, y, sg.yscale, A.M - m0);
    g2_slices_finish<MT>(pt, per_slice, A.cnt + (int64_t)mblk * A.NB + nblk, A.S, m0, A.M,
                         (int64_t)lblk * kG2BN, sg.n_out, sg.y, sg.ldy);
}

}  // namespace sihip
