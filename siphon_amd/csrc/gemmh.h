// Prefill and batch GEMM for F16 weights on v_mfma_f32_16x16x32_f16
// (gfx950): Y[M x n_out] = X[M x n_in] * W^T with X converted to f16 as the
// reference's F16 pair does (backend.c:19-27), each output within the
// tolerance of the reference dot (reference kernels.c:189-195: f16 weight
// times f16 activation, summed in f32). A product of two f16 values is exact
// in f32; the MFMA sums the products in f32 in its own order.
//
// Tiles follow the 16x16 K-quant GEMMs (gemm2.h, gemm6.h): a workgroup of 4
// waves computes BM = 16 MT activation rows against 128 weight rows, wave w
// owning rows 32 w .. 32 w + 31 (two 16-column n tiles). A step covers 128
// elements of K (4 MFMA K-steps of 32); the operands rotate by K-step as in
// gemm6.h (the next step's weights of K-step ks are loaded as soon as its
// MFMAs are issued), the activation record of a step is staged through
// registers into LDS, and K slices split a tile's steps over several
// workgroups when the output tiles alone would leave the chip idle. There
// is no epilogue: the accumulators are the outputs.
#pragma once

#include "agent.h"
#include "formats.h"
#include "gemm2.h"
#include "unit.h"

namespace sihip {

typedef _Float16 v8hh_t __attribute__((ext_vector_type(8)));

// ---- activation records ----------------------------------------------------
//
// One record per (block of BM rows, step c of 128 elements): fragment
// (m tile mt, K-step ks) at 1024 (4 mt + ks); its lane l holds row
// 16 mt + l % 16, elements 128 c + 32 ks + 8 (l / 16) .. + 7 as f16.
__host__ __device__ constexpr int gh_rec_bytes(int BM) { return 256 * BM; }

// One thread per 8 elements (16 bytes of a fragment); rows M..Mp-1 are
// zero. Grid: ceil(Mp * n_in / 8 / 256) workgroups of 256. Groups of 16
// consecutive threads take 16 consecutive rows (Mp is a multiple of 16) of
// one 8-element piece, so their stores fill 256 contiguous bytes.
template <int BM>
__global__ __launch_bounds__(256) void gemmh_convert_x(const float *x, int64_t ldx, int64_t M,
                                                       int64_t Mp, int64_t n_in, uint8_t *rec) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t per_row = n_in / 8;
    if (i >= Mp * per_row) return;
    const int64_t grp = i >> 4;  // (row group of 16, piece)
    const int64_t m = (grp / per_row) * 16 + (i & 15), k8 = grp % per_row;
    const int64_t k = k8 * 8;
    const int64_t c = k / 128;
    const int ks = (int)((k % 128) / 32), g = (int)((k % 32) / 8);
    v8hh_t v;
    if (m < M) {
        const float4 a = *reinterpret_cast<const float4 *>(x + m * ldx + k);
        const float4 b = *reinterpret_cast<const float4 *>(x + m * ldx + k + 4);
        v = (v8hh_t){(_Float16)a.x, (_Float16)a.y, (_Float16)a.z, (_Float16)a.w,
                     (_Float16)b.x, (_Float16)b.y, (_Float16)b.z, (_Float16)b.w};
    } else {
        v = (v8hh_t){0, 0, 0, 0, 0, 0, 0, 0};
    }
    const int64_t mb = m / BM;
    const int mr = (int)(m % BM);
    uint8_t *R = rec + (mb * (n_in / 128) + c) * gh_rec_bytes(BM);
    *reinterpret_cast<v8hh_t *>(R + (4 * (mr >> 4) + ks) * 1024 + (16 * g + (mr & 15)) * 16) = v;
}

// ---- weight copy in the order of this kernel ----------------------------------
//
// Per block of 32 weight rows and step c, one chunk of 8192 bytes: piece
// (ks, nt) at 1024 (2 ks + nt), lane l holding row 16 nt + l % 16, elements
// 128 c + 32 ks + 8 (l / 16) .. + 7 (16 bytes of f16).
constexpr int kGHChunk = 8192;

__host__ __device__ inline int64_t gemmh_layout_bytes(int64_t nblk32, int64_t nk) {
    return nblk32 * nk * kGHChunk;
}

// One thread per 16-byte piece (512 per chunk); rows past n_out are zero.
__global__ __launch_bounds__(256) void gemmh_layout_f16(Layout L, const uint8_t *planes,
                                                        uint8_t *out, int64_t nblk32) {
    const int64_t nk = L.n_in / 128;
    constexpr int per = kGHChunk / 16;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nblk32 * nk * per) return;
    const int64_t chunk = i / per;
    const int p = (int)(i % per);
    const int64_t blk = chunk / nk, c = chunk % nk;
    const int ks = p >> 7, nt = (p >> 6) & 1, l = p & 63;
    const int64_t row = blk * 32 + 16 * nt + (l & 15);
    uint4 v = make_uint4(0, 0, 0, 0);
    if (row < L.n_out) {
        // unit 4 c + ks of the row (32 elements, 64 bytes), bytes 16 (l / 16) ..
        const uint8_t *u = planes + unit_off(L, 0, row, 4 * c + ks);
        v = *reinterpret_cast<const uint4 *>(u + 16 * (l >> 4));
    }
    *reinterpret_cast<uint4 *>(out + i * 16) = v;
}

// ---- the GEMM -----------------------------------------------------------------

struct GHArgs {
    const uint8_t *w;     // weight chunks [nblk32][nk]
    const uint8_t *x;     // activation records [MB][nk]
    float *y;             // Y[m * ldy + n]
    int64_t ldy;
    int64_t n_out, M, Mp;
    int nk, MB, NB;       // steps of 128; m blocks of BM rows; n blocks of 128 rows
    int S, SBK;           // K slices: slice s covers steps [s SBK, (s + 1) SBK)
    float *part;          // part[(s Mp + m) * NB * 128 + n]
    uint32_t *cnt;        // cnt[mblk * NB + nblk], zero between launches
    const float *xf;      // XF: X itself, f32, X[m * ldx + k]
    int64_t ldx;
};

// At least two waves per SIMD, no upper bound: the register count (80
// VGPRs at MT = 1 to 248 at MT = 8) sets the occupancy.
//
// XF: the workgroup converts its own steps of X (A.xf) into the records as
// it stages them, with gemmh_convert_x's conversion and placement, instead
// of reading records that a conversion launch wrote (A.x).
template <int MT, bool XF>
__global__ __launch_bounds__(kG2Threads)
__attribute__((amdgpu_waves_per_eu(2))) void gemmh_f16_kernel(GHArgs A) {
    constexpr int BM = 16 * MT;
    constexpr int kRec = gh_rec_bytes(BM);
    constexpr int kXP = kRec / 16;
    constexpr int kXPT = (kXP + kG2Threads - 1) / kG2Threads;
    __shared__ __attribute__((aligned(16))) uint8_t sx0[kRec];
    __shared__ __attribute__((aligned(16))) uint8_t sx1[kRec];
    // XCD-aware order, as in gemm6.h
    const int b = blockIdx.x;
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
        (void *)(A.w + (int64_t)(nblk * 4 + wave) * A.nk * kGHChunk), (short)0, A.nk * kGHChunk,
        0x00020000);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(A.x + (int64_t)mblk * A.nk * kRec), (short)0, A.nk * kRec, 0x00020000);
    const int v_op = lane * 16;

    uint4 xs[kXPT];
    float4 xv[kXPT][2];  // XF
    auto load_x = [&](int c) {
#pragma unroll
        for (int k = 0; k < kXPT; k++) {
            const int i = (int)threadIdx.x + kG2Threads * k;
            if (kXP % kG2Threads == 0 || i < kXP) {
                if constexpr (XF) {
                    // piece i of the record: fragment (mt, ks) = i / 64, lane
                    // i % 64 (row 16 mt + l % 16, elements 32 ks + 8 (l / 16)
                    // of the step); rows past M stay zero
                    const int fr = i >> 6, l = i & 63;
                    const int64_t m = (int64_t)mblk * BM + 16 * (fr >> 2) + (l & 15);
                    xv[k][0] = xv[k][1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    if (m < A.M) {
                        const float *src = A.xf + m * A.ldx + 128 * c + 32 * (fr & 3) + 8 * (l >> 4);
                        xv[k][0] = reinterpret_cast<const float4 *>(src)[0];
                        xv[k][1] = reinterpret_cast<const float4 *>(src)[1];
                    }
                } else {
                    xs[k] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                          xr, (int)threadIdx.x * 16, c * kRec + 4096 * k, 0));
                }
            }
        }
    };
    auto store_x = [&](uint8_t *dst) {
#pragma unroll
        for (int k = 0; k < kXPT; k++) {
            const int i = (int)threadIdx.x + kG2Threads * k;
            if (kXP % kG2Threads == 0 || i < kXP) {
                if constexpr (XF) {
                    const float4 a = xv[k][0], b = xv[k][1];
                    *reinterpret_cast<v8hh_t *>(dst + i * 16) =
                        (v8hh_t){(_Float16)a.x, (_Float16)a.y, (_Float16)a.z, (_Float16)a.w,
                                 (_Float16)b.x, (_Float16)b.y, (_Float16)b.z, (_Float16)b.w};
                } else {
                    *reinterpret_cast<uint4 *>(dst + i * 16) = xs[k];
                }
            }
        }
    };
    v8hh_t bw[4][2];
    auto load_ks = [&](int c, int ks) {
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
            bw[ks][nt] = __builtin_bit_cast(
                v8hh_t, __builtin_amdgcn_raw_buffer_load_b128(wr, v_op, c * kGHChunk + (2 * ks + nt) * 1024, 0));
    };

    v4f2_t y[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++) y[mt][nt] = (v4f2_t){0.0f, 0.0f, 0.0f, 0.0f};

    // step c: the record in X, the operands in bw; K-step ks of every m
    // tile, then the next step's operands of ks into the same registers
    auto step = [&](int c, const uint8_t *X, uint8_t *xn) {
        __syncthreads();
        const int cn = c + 1 < c1 ? c + 1 : c;
        load_x(cn);
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const v8hh_t a = *reinterpret_cast<const v8hh_t *>(X + (4 * mt + ks) * 1024 + lane * 16);
#pragma unroll
                for (int nt = 0; nt < 2; nt++)
                    y[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bw[ks][nt], y[mt][nt], 0, 0, 0);
            }
            load_ks(cn, ks);
            __builtin_amdgcn_sched_barrier(0);
        }
        store_x(xn);
    };

    load_x(c0);
#pragma unroll
    for (int ks = 0; ks < 4; ks++) load_ks(c0, ks);
    store_x(sx0);
    for (int c = c0; c < c1; c += 2) {
        step(c, sx0, sx1);
        if (c + 1 < c1) step(c + 1, sx1, sx0);
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
