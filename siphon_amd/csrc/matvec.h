// Batch-1 / small-M quantized matvec on gfx950 over the planar layout of
// formats.h.
//
// One workgroup = 4 wavefronts. Each wave owns row tiles of R rows; lane
// (r, g) streams units g, g+G, g+2G, ... of row r, so every load instruction
// of a wave reads one contiguous 64 * P byte span of a plane (coalesced
// 16-byte loads for the quant planes). Weight data arrives in batches of
// kBatch steps, double buffered: while one batch is decoded the next one is
// in flight, and the first batch is requested before the prologue so its
// HBM latency overlaps the activation quantization.
//
// Prologue: the workgroup converts the f32 activation column(s) into the
// weight type's pair format directly into LDS with the bit-exact quantizers
// of quant.h (or copies an already quantized column), so no separate
// quantization launch is needed.
//
// Decode and dot products are in unit.h: quants become 8 dwords of int8 and
// meet the activation bytes (read from LDS, broadcast across the R rows of
// the tile) in v_dot4_i32_i8; integer sums are exact and each unit's float
// epilogue applies the block scales. The G partial sums of a row are
// combined with lane shuffles in a fixed order, so results are deterministic
// and need no atomics.
//
// Per-unit arithmetic restates the reference dots (reference
// src/kernels.c:197-523, src/kernels_avx2.c:150-590):
//   Q4_0/Q5_0/Q8_0: d_w*d_x*sum(q*x), with the -8/-16 bias folded as
//                   sum(u*x) - bias*sum(x)
//   Q2_K/Q4_K/Q5_K: d*d_x*sum_j sc_j*sum(q*x) - dmin*d_x*sum_j m_j*bsum_j
//   Q3_K/Q6_K:      d*d_x*sum_g sc_g*(sum(u*x) - bias*bsum_g)
//   F16:            sum f16(w)*f16(x) with f32 accumulation (v_dot2)
#pragma once

#include "agent.h"
#include "formats.h"
#include "quant.h"
#include "unit.h"

namespace sihip {

constexpr int kWaves = 4;             // wavefronts per workgroup
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxCols = 8;           // activation columns per launch
#ifndef SIHIP_BATCH
#define SIHIP_BATCH 4
#endif
constexpr int kBatch = SIHIP_BATCH;   // steps per weight batch

// LDS bytes of one activation column in pair format.
__host__ __device__ inline int64_t lds_col_bytes(uint32_t pair, int64_t n_in) {
    if (pair == T_Q8_K) return n_in + (n_in / 256) * (4 + 32);
    if (pair == T_Q8_0) return n_in + (n_in / 32) * 8;
    return n_in * 2;  // F16
}

// One weight matrix of a launch, described by what the kernel reads (the
// layout's plane bases and tile geometry, with the host computing whatever
// it can). Several matrices that share the activation (QKV, gate+up) run in
// one launch: matrix i takes the workgroups of grid row blockIdx.y == i
// (the surplus of a row wider than its nwg exits at once), and all of them
// stage the same activation into LDS. A launch of one matrix reads seg[0]
// at a fixed offset, so the first kernel-argument loads of its waves go out
// together; selecting the matrix by a loaded value first would add a round
// trip (measured: about 0.4 us per launch).
constexpr int kMaxSegs = 4;
// Segments of one launch: a matrix of a launch of several may be cut into
// consecutive ranges of its row tiles, each a segment of its own, so that
// every segment has the same workgroup count and the grid (the widest
// segment's workgroups x the segments) has no surplus (run_matvec_multi).
constexpr int kMaxLaunchSegs = 8;

struct MVSeg {
    const uint8_t *plane[4];  // plane bases
    float *y;                 // outputs, column c at y + c * ldy
    int64_t ldy;
    // Column slices. split == 1: a workgroup computes whole rows (spr == S).
    // split > 1: workgroup i computes rounds [spr * (i % split), +spr) of
    // the kWaves tiles of group i / split, one tile per wave, and stores its
    // partial sums in part[(slice * NC + c) * ntiles * R + row]; the last
    // workgroup of a group to arrive (counted in cnt[group], which is zero
    // between launches) adds the slices in slice order and writes y.
    float *part;
    uint32_t *cnt;
    uint32_t split, spr;
    uint32_t type;
    uint32_t n_out;           // rows to compute (<= the layout's rows)
    uint32_t ntiles;          // ceil(n_out / R)
    uint32_t nwg;             // workgroups of this matrix
    uint32_t G, logG, R;      // wave tile: G columns x R rows
    uint32_t S;               // rounds per tile
    uint32_t ncols;           // columns per row
};

struct MVArgs {
    MVSeg seg[kMaxLaunchSegs];
    int nseg;
    int64_t n_in;
    const float *x;       // f32 activations, column c at x + c * ldx (or null)
    const uint8_t *xq;    // pair-format activations, column c at xq + c * ldxq
    int64_t ldx, ldxq;
    int nc;               // activation columns staged (== the kernel's NC)
    int64_t col_bytes;    // LDS bytes per column
    int q80s;             // Q8_0 pair from f32: the scalar quantizer (q80_block_sel)
};

// ---- prologue: activations -> LDS ----------------------------------------
//
// Q8_K from f32 is split in two so the caller can issue its first weight
// batch in between, from wave-uniform control flow: stage_q8k_first loads
// the x values of the first XP passes (16 blocks per pass; memory counters
// drain in order, so x loaded after the weights could only be waited for
// together with them), stage_activations quantizes them and stages the
// remaining passes. XP > 1 is used for long rows (n_in > 4096) by kernels
// whose register budget has room for the extra values.

// Passes of 64 Q8_0 blocks whose x values a thread loads together.
constexpr int kQ80Passes = 4;

// float4s of an F16 activation a thread loads together.
constexpr int kF16Vecs = 8;

template <int XP>
struct XFirst {
    float4 t[XP][4];            // Q8_K: the first XP passes
    float2 h[kQ80Passes][4];    // Q8_0 (4 lanes per block): the first passes
    float4 f[kF16Vecs];         // F16: the first group
};

// 16 lanes quantize one block: thread tid owns block (tid >> 4) + 16 p of
// pass p (counted from block b0 of the row, nbl blocks staged), elements
// 16 * (tid & 15) .. +15 of it.
template <int XP>
__device__ inline void stage_q8k_first(const MVArgs &a, XFirst<XP> &xf, int64_t b0, int64_t nbl) {
    const int tid = threadIdx.x;
    if (!a.x) return;
#pragma unroll
    for (int p = 0; p < XP; p++) {
        if (16 * p < nbl) {  // wave-uniform
            int64_t b = (tid >> 4) + 16 * p;
            b = b < nbl ? b : nbl - 1;  // clamped: the load stays in the range
            const float4 *src = reinterpret_cast<const float4 *>(a.x + (b0 + b) * 256 + (tid & 15) * 16);
#pragma unroll
            for (int i = 0; i < 4; i++) xf.t[p][i] = src[i];
        }
    }
}

// Q8_0 from f32 with the SIMD quantizer: a quad of lanes quantizes one
// block (q80_quad_v); thread tid owns block (tid >> 2) + 64 p of pass p,
// and loads the x values of kQ80Passes passes together. The first ones are
// loaded here, before the first weight batch, as for Q8_K.
__device__ inline void q80_load_passes(const float *xc, int64_t p0, int64_t nbl,
                                       float2 (&t)[kQ80Passes][4]) {
#pragma unroll
    for (int p = 0; p < kQ80Passes; p++) {
        if (p0 + 64 * p < nbl) {  // wave-uniform
            int64_t b = p0 + 64 * p + (threadIdx.x >> 2);
            b = b < nbl ? b : nbl - 1;  // clamped: the load stays in the range
            q80_quad_load(xc + b * 32, threadIdx.x & 3, t[p]);
        }
    }
}

template <int XP>
__device__ inline void stage_q80_first(const MVArgs &a, XFirst<XP> &xf, int64_t b0, int64_t nbl) {
    if (!a.x || a.q80s) return;
    q80_load_passes(a.x + b0 * 32, 0, nbl, xf.h);
}

// F16 from f32: thread tid converts float4s tid + kThreads v of each group
// of kThreads * kF16Vecs, whose loads it issues together; the first group
// is loaded before the first weight batch.
__device__ inline void f16_load_group(const float *xc, int64_t v0, int64_t nvec,
                                      float4 (&f)[kF16Vecs]) {
#pragma unroll
    for (int v = 0; v < kF16Vecs; v++) {
        if (v0 + kThreads * v < nvec) {  // wave-uniform
            int64_t i = v0 + kThreads * v + threadIdx.x;
            i = i < nvec ? i : nvec - 1;  // clamped: the load stays in the range
            f[v] = reinterpret_cast<const float4 *>(xc)[i];
        }
    }
}

template <int XP>
__device__ inline void stage_f16_first(const MVArgs &a, XFirst<XP> &xf, int64_t b0, int64_t nbl) {
    if (!a.x) return;
    f16_load_group(a.x + b0 * 32, 0, nbl * 8, xf.f);
}

__device__ inline void q8k_stage_block(uint8_t *col, int64_t n, int64_t b, int lane16,
                                       const float4 t4[4]) {
    const int64_t nb = n / 256;
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[4 * i] = t4[i].x; v[4 * i + 1] = t4[i].y; v[4 * i + 2] = t4[i].z; v[4 * i + 3] = t4[i].w;
    }
    const Q8KRow r = q8k_block_row16(v, lane16);
    *reinterpret_cast<uint4 *>(col + q8k_lds_unit((uint32_t)nb, (uint32_t)b, lane16 >> 1) +
                               16 * (lane16 & 1)) = r.q;
    reinterpret_cast<int16_t *>(col + n + nb * 4)[b * 16 + lane16] = (int16_t)r.gsum;
    if (lane16 == 0) reinterpret_cast<float *>(col + n)[b] = r.d;
}

// Stages pair blocks [b0, b0 + nbl) of each column (32-element units for
// F16) as the LDS image of a row of n = nbl blocks' elements: a launch of
// whole rows stages its row (b0 = 0), a column slice only its slice, so its
// LDS holds a slice rather than a row.
template <uint32_t PAIR, int XP>
__device__ inline void stage_activations(const MVArgs &a, uint8_t *lds, const XFirst<XP> &xf,
                                         int64_t b0, int64_t nbl, int64_t n) {
    const int tid = threadIdx.x;
    for (int c = 0; c < a.nc; c++) {
        uint8_t *col = lds + c * a.col_bytes;
        if constexpr (PAIR == T_Q8_K) {
            const int64_t nb = n / 256;
            float *dcol = reinterpret_cast<float *>(col + n);
            int16_t *bcol = reinterpret_cast<int16_t *>(col + n + nb * 4);
            if (a.x) {
                const float *xc = a.x + c * a.ldx + b0 * 256;
                const int lane16 = tid & 15;
                int64_t bt = tid >> 4;
                if (c == 0) {  // the passes loaded up front
#pragma unroll
                    for (int p = 0; p < XP; p++)
                        if (bt + 16 * p < nbl) q8k_stage_block(col, n, bt + 16 * p, lane16, xf.t[p]);
                    bt += 16 * XP;
                }
                for (int64_t b = bt; b < nbl; b += kThreads / 16) {
                    const float4 *src = reinterpret_cast<const float4 *>(xc + b * 256 + lane16 * 16);
                    float4 t4[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) t4[i] = src[i];
                    q8k_stage_block(col, n, b, lane16, t4);
                }
            } else {
                const uint8_t *src = a.xq + c * a.ldxq + b0 * 292;
                for (int64_t i = tid; i < nbl * 73; i += kThreads) {
                    const int64_t b = i / 73, w = i % 73;  // 73 dwords per 292-byte block
                    const uint32_t v = reinterpret_cast<const uint32_t *>(src + b * 292)[w];
                    if (w == 0) dcol[b] = __uint_as_float(v);
                    else if (w < 65)
                        *reinterpret_cast<uint32_t *>(
                            col + q8k_lds_unit((uint32_t)nb, (uint32_t)b, (uint32_t)(w - 1) >> 3) +
                            4 * ((w - 1) & 7)) = v;
                    else reinterpret_cast<uint32_t *>(bcol + b * 16)[w - 65] = v;
                }
            }
        } else if constexpr (PAIR == T_Q8_0) {
            const int64_t nb = n / 32;
            float *dcol = reinterpret_cast<float *>(col + n);
            int *scol = reinterpret_cast<int *>(col + n + nb * 4);
            if (a.x && !a.q80s) {
                // every lane runs every pass (the quads exchange values), lanes
                // past the last block on a clamped copy whose results are not
                // stored
                const int j = tid & 3;
                const float *xc = a.x + c * a.ldx + b0 * 32;
                for (int64_t p0 = 0; p0 < nbl; p0 += 64 * kQ80Passes) {
                    float2 t[kQ80Passes][4];
                    if (c == 0 && p0 == 0) {
#pragma unroll
                        for (int p = 0; p < kQ80Passes; p++)
#pragma unroll
                            for (int i = 0; i < 4; i++) t[p][i] = xf.h[p][i];
                    } else {
                        q80_load_passes(xc, p0, nbl, t);
                    }
#pragma unroll
                    for (int p = 0; p < kQ80Passes; p++) {
                        if (p0 + 64 * p < nbl) {  // wave-uniform
                            const int64_t b = p0 + 64 * p + (tid >> 2);
                            const Q80Quad r = q80_quad_v(t[p]);
                            if (b < nbl) {
                                uint16_t *q16 = reinterpret_cast<uint16_t *>(col + b * 32);
#pragma unroll
                                for (int i = 0; i < 4; i++) q16[4 * i + j] = (uint16_t)r.q2[i];
                                if (j == 0) {
                                    dcol[b] = r.d;
                                    scol[b] = r.sum;
                                }
                            }
                        }
                    }
                }
                continue;
            }
            for (int64_t b = tid; b < nbl; b += kThreads) {
                uint32_t q[8];
                float d;
                int sum;
                if (a.x) {
                    const Q80Block r = q80_block_sel(a.x + c * a.ldx + (b0 + b) * 32, a.q80s);
                    for (int t = 0; t < 8; t++) q[t] = r.q[t];
                    d = r.d;
                    sum = r.sum;
                } else {
                    const uint8_t *src = a.xq + c * a.ldxq + (b0 + b) * 34;
                    d = f16_bits_to_f32((uint32_t)src[0] | ((uint32_t)src[1] << 8));
                    sum = 0;
                    for (int t = 0; t < 8; t++) {
                        uint32_t w = 0;
                        for (int k = 0; k < 4; k++) {
                            const uint8_t byte = src[2 + 4 * t + k];
                            sum += (int8_t)byte;
                            w |= (uint32_t)byte << (8 * k);
                        }
                        q[t] = w;
                    }
                }
                uint4 *dst = reinterpret_cast<uint4 *>(col + b * 32);
                dst[0] = make_uint4(q[0], q[1], q[2], q[3]);
                dst[1] = make_uint4(q[4], q[5], q[6], q[7]);
                dcol[b] = d;
                scol[b] = sum;
            }
        } else {  // F16
            uint16_t *h = reinterpret_cast<uint16_t *>(col);
            if (a.x) {
                const float *xc = a.x + c * a.ldx + b0 * 32;
                const int64_t nvec = nbl * 8;
                for (int64_t v0 = 0; v0 < nvec; v0 += kThreads * kF16Vecs) {
                    float4 f[kF16Vecs];
                    if (c == 0 && v0 == 0) {
#pragma unroll
                        for (int v = 0; v < kF16Vecs; v++) f[v] = xf.f[v];
                    } else {
                        f16_load_group(xc, v0, nvec, f);
                    }
#pragma unroll
                    for (int v = 0; v < kF16Vecs; v++) {
                        const int64_t i = v0 + kThreads * v + tid;
                        if (v0 + kThreads * v < nvec && i < nvec) {
                            const uint32_t lo =
                                (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f[v].x) |
                                ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f[v].y) << 16);
                            const uint32_t hi =
                                (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f[v].z) |
                                ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f[v].w) << 16);
                            *reinterpret_cast<uint2 *>(h + 4 * i) = make_uint2(lo, hi);
                        }
                    }
                }
            } else {
                const uint16_t *src = reinterpret_cast<const uint16_t *>(a.xq + c * a.ldxq) + b0 * 32;
                for (int64_t i = tid; i < nbl * 32; i += kThreads) h[i] = src[i];
            }
        }
    }
}

// ---- the kernel -------------------------------------------------------------
//
// Each wave walks a flat sequence of rounds (tile, s): tiles wave0,
// wave0 + nwaves, ... and S rounds per tile. One round is one super-block per
// lane for the K-quants and kBatch units per lane otherwise. All control
// flow in the loop is wave-uniform (scalar); loads are never predicated per
// lane: rows past n_out in the last tile read the zero-filled padding that
// the upload allocates (their results are not stored), and padding slots
// past the end of a row re-read a real column and are discarded.

struct Item {
    uint32_t tile, s, rec;  // rec = (tile * S + s) * 64
};

__device__ inline float dpp_f32(float v, int ctrl) {
    return __uint_as_float(dpp_u32(__float_as_uint(v), ctrl));
}

// Sum over the G lanes of a group in the order of reduce_partner (unit.h).
__device__ inline float group_sum(float v, int G) {
    if (G > 1) v += dpp_f32(v, kDppXor1);
    if (G > 2) v += dpp_f32(v, kDppXor2);
    if (G > 4) v += dpp_f32(v, kDppHalfMirror);
    if (G > 8) v += dpp_f32(v, kDppMirror);
    if (G > 16) v += __shfl_xor(v, 16, 64);
    if (G > 32) v += __shfl_xor(v, 32, 64);
    return v;
}

template <uint32_t FMT>
struct Buf {
    static constexpr bool kq = is_kquant(FMT);
    static constexpr int items = kq ? 1 : kBatch;  // rounds per buffer
    KRaw k;
    Raw u[kBatch];
};

// End of a column-sliced workgroup: count its arrival in its tile group and,
// if it is the group's last, add the partial sums of the group's rows over
// the slices in slice order (the same order whichever workgroup is last)
// and reset the counter for the next launch. Nothing waits on another
// workgroup.
//
// Partial sums travel through agent-scope atomic stores and loads, which
// write through / read past the per-XCD L2 caches, so no L2 write-back or
// invalidation (what an agent-scope release / acquire fence costs on gfx950:
// a 7x slower launch) is needed: each wave waits until its partial stores
// have completed before the workgroup counts its arrival, and the last
// workgroup reads the partials only after its arrival has returned.
//
// `last` is a word of LDS past the staged activations (the launch of a sliced
// matrix allocates it; a static LDS variable would add to every launch's LDS
// and cost occupancy where the activations fill it exactly).
template <int NC>
__device__ inline void split_reduce(const MVSeg &sg, uint32_t grp, uint32_t ldp, uint32_t *last) {
    // The signal fences keep the compiler from moving memory operations
    // across the completion wait, the count and the loads after it (they
    // emit no instruction); the hardware order is the wait and the barriers.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (threadIdx.x == 0)
        *last = __hip_atomic_fetch_add(sg.cnt + grp, 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT) == sg.split - 1;
    __syncthreads();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (!*last) return;
    const uint32_t rows = kWaves * sg.R;
    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
        sg.part, (short)0, (int)(sg.split * NC * ldp * 4), 0x00020000);
    for (uint32_t i = threadIdx.x; i < rows * NC; i += kThreads) {
        const uint32_t c = i / rows;
        const int64_t row = (int64_t)grp * rows + (i - c * rows);
        if (row < (int64_t)sg.n_out) {
            // slices in groups of 8 whose loads are issued together, added in
            // slice order
            float v = 0.0f;
            for (uint32_t p0 = 0; p0 < sg.split; p0 += 8) {
                float pv[8];
#pragma unroll
                for (uint32_t k = 0; k < 8; k++) {
                    const uint32_t p = p0 + k < sg.split ? p0 + k : sg.split - 1;
                    pv[k] = load_agent_f32(pr, (uint32_t)(((int64_t)(p * NC + c) * ldp + row) * 4));
                }
#pragma unroll
                for (uint32_t k = 0; k < 8; k++)
                    if (p0 + k < sg.split) v += pv[k];
            }
            sg.y[c * sg.ldy + row] = v;
        }
    }
    if (threadIdx.x == 0)
        __hip_atomic_store(sg.cnt + grp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The matvec of one matrix (segment sg) by the workgroups of its range.
// SPLIT: compiled with the column-slice paths (a launch with a sliced
// matrix); without them a launch of whole rows keeps the shorter code.
template <uint32_t FMT, int NC, int XP, bool SPLIT>
__device__ inline void matvec_body(const MVArgs &A, const MVSeg &sg, uint8_t *lds) {
    constexpr bool KQ = is_kquant(FMT);
    constexpr uint32_t PAIR = (FMT == T_F16) ? T_F16
                              : (FMT == T_Q4_0 || FMT == T_Q5_0 || FMT == T_Q8_0) ? T_Q8_0
                                                                                   : T_Q8_K;
    constexpr int ITEMS = Buf<FMT>::items;
    const int lane = threadIdx.x & 63;
    const int G = (int)sg.G;
    const int g = lane & (G - 1);
    const int r = lane >> sg.logG;
    Planes P;
#pragma unroll
    for (int p = 0; p < 4; p++) P.p[p] = sg.plane[p];
    const uint32_t S = sg.S;
    const uint32_t n_in = (uint32_t)A.n_in;
    const uint32_t last_col = sg.ncols - 1;
    // When G does not divide the columns, the last round of a tile has
    // padding slots (column s * G + g past the row). Their lanes load the
    // row's last real column of that round instead, which the same load
    // instruction fetches anyway, so padding costs no memory traffic; their
    // contribution is discarded.
    const uint32_t glast = last_col - (S - 1) * (uint32_t)G;
    const uint32_t lane_last = (uint32_t)(r * G) + ((uint32_t)g < glast ? (uint32_t)g : glast);
    const uint32_t col_bytes = (uint32_t)A.col_bytes;
    const uint32_t ntiles = sg.ntiles;
    const uint32_t R = sg.R;
    // wave-uniform: keep the whole walk in scalar registers
    const uint32_t wv = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const uint32_t wgi = blockIdx.x;
    const bool split = SPLIT && sg.split > 1;
    const uint32_t grp = split ? wgi / sg.split : 0u;
    const uint32_t slice = split ? wgi - grp * sg.split : 0u;
    // rounds [s_begin, s_end) of each tile
    const uint32_t s_begin = SPLIT ? slice * sg.spr : 0u;
    const uint32_t s_end = !SPLIT ? S : s_begin + sg.spr < S ? s_begin + sg.spr : S;
    const uint32_t wave0 = (split ? grp : wgi) * kWaves + wv;
    const uint32_t nwaves = split ? ntiles : sg.nwg * kWaves;  // split: one tile per wave
    const uint32_t my_tiles = wave0 < ntiles ? (ntiles - 1 - wave0) / nwaves + 1 : 0;
    const uint32_t total = my_tiles * (s_end - s_begin);  // rounds of this wave
    // activation blocks of the columns this workgroup's rounds read; a
    // slice's LDS image is a row of its own (n_loc elements, columns from
    // cbase)
    const int64_t b0 = (int64_t)s_begin * G;
    const int64_t b1 = (int64_t)s_end * G < sg.ncols ? (int64_t)s_end * G : (int64_t)sg.ncols;
    constexpr uint32_t kColElems = KQ ? 256u : 32u;
    const uint32_t n_loc = SPLIT ? (uint32_t)(b1 - b0) * kColElems : n_in;
    const uint32_t cbase = SPLIT ? (uint32_t)b0 : 0u;

    // finished rows go to y, or (sliced) to this slice's partial sums, rows
    // of the last tile included; agent-scope stores, which partial sums need
    // (split_reduce) and which cost y nothing
    float *const out = split ? sg.part + (int64_t)slice * NC * ntiles * R : sg.y;
    const int64_t out_ld = split ? (int64_t)ntiles * R : sg.ldy;
    const int64_t out_rows = split ? (int64_t)ntiles * R : (int64_t)sg.n_out;

    auto step = [&](Item &it) {
        if (++it.s == s_end) {
            it.s = s_begin;
            it.tile += nwaves;
            it.rec = (it.tile * S + s_begin) * 64u;
        } else {
            it.rec += 64u;
        }
    };
    // issue the loads of the next ITEMS rounds; rounds past the end repeat
    // the last round (in bounds, results unused)
    // a wave without rows (only in the last workgroup) still loads, from
    // tile 0, so that the loads before the barrier are unconditional
    const uint32_t t0 = total ? wave0 : 0u;
    Item in_it{t0, s_begin, (t0 * S + s_begin) * 64u};
    uint32_t issued = 0;
    auto issue = [&](Buf<FMT> &b) {
#pragma unroll
        for (int i = 0; i < ITEMS; i++) {
            const uint32_t ln = in_it.s == S - 1 ? lane_last : (uint32_t)lane;
            if constexpr (KQ)
                load_kblock<FMT>(P, in_it.rec * 8u + ln, in_it.rec + ln, b.k);
            else
                load_unit<FMT>(P, in_it.rec + ln, b.u[i]);
            if (issued < total) {
                issued++;
                if (issued < total) step(in_it);
            }
        }
    };
    Item c_it{wave0, s_begin, (wave0 * S + s_begin) * 64u};
    uint32_t c_k = 0;
    float acc[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) acc[c] = 0.0f;
    auto consume = [&](const Buf<FMT> &b) {
#pragma unroll
        for (int i = 0; i < ITEMS; i++) {
            if (c_k < total) {
                uint32_t col = c_it.s * (uint32_t)G + (uint32_t)g;
                const bool pad = col > last_col;
                col = pad ? last_col : col;  // padding slots read a valid LDS column
                float keep[NC];
#pragma unroll
                for (int c = 0; c < NC; c++) keep[c] = acc[c];
                if constexpr (KQ)
                    compute_kblock<FMT, NC>(lds, col_bytes, n_loc, col - cbase, b.k, acc);
                else
                    compute_unit<FMT, NC>(lds, col_bytes, n_loc, col - cbase, b.u[i], acc);
#pragma unroll
                for (int c = 0; c < NC; c++) acc[c] = pad ? keep[c] : acc[c];
                if (c_it.s == s_end - 1) {
                    const int64_t row = (int64_t)c_it.tile * R + r;
#pragma unroll
                    for (int c = 0; c < NC; c++) {
                        const float v = group_sum(acc[c], G);
                        if (g == 0 && row < out_rows)
                            __hip_atomic_store(out + c * out_ld + row, v, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
                        acc[c] = 0.0f;
                    }
                }
                step(c_it);
                c_k++;
            }
        }
    };

    Buf<FMT> bufA, bufB;
    XFirst<XP> xf;
    if constexpr (PAIR == T_Q8_K) stage_q8k_first<XP>(A, xf, b0, b1 - b0);
    if constexpr (PAIR == T_Q8_0) stage_q80_first<XP>(A, xf, b0, b1 - b0);
    if constexpr (PAIR == T_F16) stage_f16_first<XP>(A, xf, b0, b1 - b0);
    issue(bufA);
    stage_activations<PAIR, XP>(A, lds, xf, b0, b1 - b0, n_loc);
    if (total == 1) {  // one round: no second buffer (it would reload the same round)
        __syncthreads();
        consume(bufA);
    } else {
        issue(bufB);
        __syncthreads();
        // a wave without rows (total == 0) only helped to stage
        if (total != 0) {
            // Two buffers in flight: each buffer is refilled right after it
            // has been decoded, so a refill never overwrites registers with a
            // load pending and every wait covers one buffer only. The
            // steady-state loop has one exit at the top and unconditional
            // refills, so the memory counters always hold the two buffers in
            // the same order and each wait is for the older one alone. The
            // last 1-3 buffers drain without redundant refills.
            const uint32_t nbuf = (total + ITEMS - 1) / ITEMS;
            uint32_t i = 0;  // next buffer to decode; A holds it, B the one after
            while (i + 4 <= nbuf) {
                consume(bufA);
                issue(bufA);
                consume(bufB);
                issue(bufB);
                i += 2;
            }
            const uint32_t left = nbuf - i;  // 1..3
            consume(bufA);
            if (left == 3) issue(bufA);
            if (left >= 2) consume(bufB);
            if (left == 3) consume(bufA);
        }
    }
    if constexpr (SPLIT)
        if (split) split_reduce<NC>(sg, grp, ntiles * R,
                         reinterpret_cast<uint32_t *>(lds + (int64_t)A.nc * A.col_bytes));
}

// Requests every kernel argument a wave uses before its first branch, so
// that they arrive in one round trip of scalar loads (the compiler would
// otherwise load some after the first test and pay a second one).
__device__ inline void request_args(const MVArgs &A, const MVSeg &sg) {
    asm volatile("" ::"s"(sg.plane[0]), "s"(sg.plane[1]), "s"(sg.plane[2]), "s"(sg.plane[3]),
                 "s"(sg.y), "s"(sg.ldy), "s"(sg.part), "s"(sg.cnt), "s"(sg.split), "s"(sg.spr),
                 "s"(sg.type), "s"(sg.n_out), "s"(sg.ntiles), "s"(sg.nwg), "s"(sg.G),
                 "s"(sg.logG), "s"(sg.R), "s"(sg.S), "s"(sg.ncols), "s"(A.x), "s"(A.xq),
                 "s"(A.ldx), "s"(A.ldxq), "s"(A.n_in), "s"(A.nc), "s"(A.col_bytes));
}

// MULTI: the matrices of grid row blockIdx.y (a launch of several);
// otherwise the one matrix seg[0], with a grid of exactly its workgroups.
template <uint32_t F0, uint32_t F1, int NC, int XP, bool SPLIT, bool MULTI>
__global__ __launch_bounds__(kThreads) void matvec_kernel(MVArgs A) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    static_assert(pair_of(F0) == pair_of(F1), "one launch stages one activation format");
    static_assert(MULTI || F0 == F1, "formats mix only in launches of several matrices");
    const MVSeg sg = A.seg[MULTI ? blockIdx.y : 0];
    request_args(A, sg);
    if constexpr (MULTI) {
        if (blockIdx.x >= sg.nwg) return;  // the whole workgroup, before any barrier
        if (F0 == F1 || sg.type == F0)
            matvec_body<F0, NC, XP, SPLIT>(A, sg, lds);
        else
            matvec_body<F1, NC, XP, SPLIT>(A, sg, lds);
    } else {
        matvec_body<F0, NC, XP, SPLIT>(A, sg, lds);
    }
}

// ---- standalone quantizers (global output in the reference block layouts) --

// 16 lanes per 256-block, the same code path as the matvec prologue.
__global__ __launch_bounds__(kThreads) void quantize_q8K_kernel(const float *x, uint8_t *out,
                                                                int64_t nb) {
    const int lane16 = threadIdx.x & 15;
    const int64_t b = (int64_t)blockIdx.x * (kThreads / 16) + (threadIdx.x >> 4);
    if (b >= nb) return;  // whole 16-lane rows leave together
    const float4 *src = reinterpret_cast<const float4 *>(x + b * 256 + lane16 * 16);
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 t = src[i];
        v[4 * i] = t.x; v[4 * i + 1] = t.y; v[4 * i + 2] = t.z; v[4 * i + 3] = t.w;
    }
    const Q8KRow r = q8k_block_row16(v, lane16);
    uint8_t *o = out + b * 292;
    uint32_t *qd = reinterpret_cast<uint32_t *>(o + 4 + lane16 * 16);
    qd[0] = r.q.x; qd[1] = r.q.y; qd[2] = r.q.z; qd[3] = r.q.w;
    reinterpret_cast<int16_t *>(o + 260)[lane16] = (int16_t)r.gsum;
    if (lane16 == 0) *reinterpret_cast<float *>(o) = r.d;
}

__global__ __launch_bounds__(kThreads) void quantize_q80_kernel(const float *x, uint8_t *out,
                                                                int64_t nb, int scalar) {
    const int64_t b = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (b >= nb) return;
    const Q80Block r = q80_block_sel(x + b * 32, scalar);
    uint8_t *o = out + b * 34;
    o[0] = (uint8_t)(r.dbits & 0xff);
    o[1] = (uint8_t)(r.dbits >> 8);
    for (int t = 0; t < 8; t++)
        for (int k = 0; k < 4; k++) o[2 + 4 * t + k] = (uint8_t)(r.q[t] >> (8 * k));
}

__global__ __launch_bounds__(kThreads) void convert_f16_kernel(const float *x, uint16_t *out,
                                                               int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < n) out[i] = __builtin_bit_cast(uint16_t, (_Float16)x[i]);
}

// ---- dequantized rows (reference row_to_f32, backend.c:122-131) -------------

// Rows [row0, row0 + nrows) of the matrix into out (row r - row0 at
// out + (r - row0) * ldo): one thread per (row, column), the column's units
// decoded as the dot products decode them (unit.h dequant_*).
template <uint32_t FMT>
__global__ __launch_bounds__(kThreads) void dequant_rows_kernel(Layout L, const uint8_t *w,
                                                                int64_t row0, int64_t nrows,
                                                                float *out, int64_t ldo) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= nrows * L.ncols) return;
    const int64_t rr = i / L.ncols, c = i % L.ncols;
    Planes P;
#pragma unroll
    for (int p = 0; p < 4; p++) P.p[p] = w + L.plane_off[p];
    const uint32_t cr = (uint32_t)col_rec(L, row0 + rr, c);
    float *o = out + rr * ldo;
    float v[32];
    if constexpr (is_kquant(FMT)) {
        KRaw raw;
        load_kblock<FMT>(P, (cr >> 6) * 512u + (cr & 63u), cr, raw);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            dequant_kunit<FMT>(raw, k, v);
            float4 *dst = reinterpret_cast<float4 *>(o + c * 256 + 32 * k);
#pragma unroll
            for (int q = 0; q < 8; q++) dst[q] = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
        }
    } else {
        Raw raw;
        load_unit<FMT>(P, cr, raw);
        dequant_unit<FMT>(raw, v);
        float4 *dst = reinterpret_cast<float4 *>(o + c * 32);
#pragma unroll
        for (int q = 0; q < 8; q++) dst[q] = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
    }
}

// ---- repack: GGUF blocks -> planes ------------------------------------------

__global__ __launch_bounds__(kThreads) void repack_kernel(Layout L, const uint8_t *src,
                                                          uint8_t *dst, int64_t row_bytes,
                                                          int64_t recs_per_row, int64_t rec_bytes) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= L.n_out * recs_per_row) return;
    const int64_t row = i / recs_per_row, k = i % recs_per_row;
    repack_block(L, dst, src + row * row_bytes + k * rec_bytes, row, k);
}

}  // namespace sihip
