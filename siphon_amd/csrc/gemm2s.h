// Small-M GEMM for Q4_K weights (M <= 16 activation rows, the batched
// decode step) on v_mfma_i32_16x16x64_i8: the arithmetic, weight copy and
// activation records of the 16x16 Q4_K GEMM (gemm2.h) with a launch shaped
// for few rows.
//
// At M <= 16 one 16-row m tile covers every activation row, so the work is
// the weight stream: each weight byte is read once and meets all M rows in
// the MFMAs. The launch is shaped like a matvec rather than a GEMM:
//   - a workgroup owns one 32-row block of the weight (one GEMM-copy chunk
//     column) and its KW waves split the super-blocks of the row among
//     themselves (wave w takes c = w, w + KW, ...), so every wave streams
//     its own chunks and n_out / 32 workgroups cover the matrix without K
//     slices across workgroups;
//   - a wave keeps the next super-block's weights and activation fragments
//     in flight while it computes the current one (two register sets);
//   - the activation fragments (16 bytes per lane and K-step, the record's
//     MFMA operand order) are read straight from the records in global
//     memory, which every workgroup shares through the L2, so no LDS
//     staging and no barrier sit in the loop;
//   - the KW partial 32-row tiles meet in LDS once at the end and wave 0
//     adds them in wave order (deterministic) and stores the M rows.
#pragma once

#include "gemm2.h"

namespace sihip {


struct G2SArgs {
    const uint8_t *w;     // GEMM-copy chunks [nblk32][nb] (gemm2.h)
    const uint8_t *x;     // activation records of one 16-row block [nb] (g2_rec_bytes(16))
    float *y;             // Y[m * ldy + n]
    int64_t ldy;
    int64_t n_out, M;
    int nb;
    float yscale;         // 2^-E
};

// KW: waves per workgroup, which split the super-blocks of its 32 rows.
template <int KW>
__global__ __launch_bounds__(64 * KW)
__attribute__((amdgpu_waves_per_eu(2))) void gemm2s_q4k_kernel(G2SArgs A) {
    constexpr int BM = 16;
    constexpr int kRec = g2_rec_bytes(BM);
    __shared__ __attribute__((aligned(16))) float red[KW - 1][2][4][64];
    const int blk = blockIdx.x;  // 32-row block
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, r16 = lane & 15;
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(A.w + (int64_t)blk * A.nb * kG2ChunkQ4K), (short)0, A.nb * kG2ChunkQ4K, 0x00020000);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void *)A.x, (short)0, A.nb * kRec, 0x00020000);
    const int v_nib = lane * 16, v_scl = kG2Scl + r16 * 16, v_d = kG2D + r16 * 4;
    const int v_min = kG2Min + lane * 16;
    const int v_bs = g2_rec_bsum(BM) + r16 * 32 + (g & 1) * 16, v_dx = g2_rec_dx(BM) + 4 * g * 4;

    struct Stage {
        uint4 nib[4];  // K-step ks: n tile 0 in x, y; 1 in z, w
        uint4 scl[2];
        float d[2];
        uint4 mn[2];
        uint4 a[4];    // activation fragments, K-step ks
        uint4 bs;      // f16 group sums of this lane's row
        float4 dx;     // block scales of rows 4 g .. 4 g + 3
    };
    auto ld4 = [&](__amdgpu_buffer_rsrc_t r, int voff, int soff) {
        return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
    };
    auto load = [&](int c, Stage &s) {
        // c is wave-uniform; readfirstlane keeps the offsets scalar (a loop
        // counter the compiler holds in a VGPR would make every buffer load
        // a waterfall loop over lanes)
        const int cu = __builtin_amdgcn_readfirstlane(c);
        const int so = cu * kG2ChunkQ4K, xo = cu * kRec;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) s.nib[ks] = ld4(wr, v_nib + ks * 1024, so);
#pragma unroll
        for (int nt = 0; nt < 2; nt++) {
            s.scl[nt] = ld4(wr, v_scl + nt * 256, so);
            s.d[nt] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wr, v_d + nt * 64, so, 0));
            s.mn[nt] = ld4(wr, v_min + nt * 1024, so);
        }
#pragma unroll
        for (int ks = 0; ks < 4; ks++) s.a[ks] = ld4(xr, ks * 1024 + lane * 16, xo);
        s.bs = ld4(xr, v_bs, xo);
        s.dx = __builtin_bit_cast(float4, ld4(xr, v_dx, xo));
    };
    uint32_t sel[4];
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        const uint32_t u = (uint32_t)(2 * ks + (g >> 1));
        sel[ks] = u | (0x0cu << 8) | (u << 16) | (0x0cu << 24);
    }
    v4f2_t y[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
    auto compute = [&](const Stage &s) {
        const v4f2_t z = {0.0f, 0.0f, 0.0f, 0.0f};
        const v8h2_t bsv = __builtin_bit_cast(v8h2_t, s.bs);
        v4f2_t t[2];
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
            t[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bsv, __builtin_bit_cast(v8h2_t, s.mn[nt]), z, 0, 0, 0);
        v4i2_t h[2] = {{0, 0, 0, 0}, {0, 0, 0, 0}}, l[2] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const v4i2_t am = __builtin_bit_cast(v4i2_t, s.a[ks]);
#pragma unroll
            for (int nt = 0; nt < 2; nt++) {
                const uint32_t w0 = nt ? s.nib[ks].z : s.nib[ks].x;
                const uint32_t w1 = nt ? s.nib[ks].w : s.nib[ks].y;
                const uint32_t q0 = w0 & 0x0F0F0F0Fu, q1 = w1 & 0x0F0F0F0Fu;
                const uint32_t q2 = (w0 >> 4) & 0x0F0F0F0Fu, q3 = (w1 >> 4) & 0x0F0F0F0Fu;
                const uint32_t sh = __builtin_amdgcn_perm(s.scl[nt].y, s.scl[nt].x, sel[ks]);
                const uint32_t sl = __builtin_amdgcn_perm(s.scl[nt].w, s.scl[nt].z, sel[ks]);
                const v4i2_t bh = {(int)g2_bytes_times(q0, sh), (int)g2_bytes_times(q1, sh),
                                   (int)g2_bytes_times(q2, sh), (int)g2_bytes_times(q3, sh)};
                const v4i2_t bl = {(int)g2_bytes_times(q0, sl), (int)g2_bytes_times(q1, sl),
                                   (int)g2_bytes_times(q2, sl), (int)g2_bytes_times(q3, sl)};
                h[nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(am, bh, h[nt], 0, 0, 0);
                l[nt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(am, bl, l[nt], 0, 0, 0);
            }
        }
        const float dxv[4] = {s.dx.x, s.dx.y, s.dx.z, s.dx.w};
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float u = fma_f32(s.d[nt], (float)(8 * h[nt][i] + l[nt][i]), t[nt][i]);
                y[nt][i] = fma_f32(dxv[i], u, y[nt][i]);
            }
    };
    // super-blocks wave, wave + KW, ...: two register sets alternate, the
    // loads of the next super-block issued before the current one computes.
    // The loop runs over pairs that both exist, so its loads need no
    // condition (the one past the end reads the last super-block again,
    // which nothing computes): a load under a condition makes the compiler
    // count it as possibly missing, and the compute that follows then waits
    // for every load in flight, the prefetch too. The empty asm statement
    // (a memory clobber) after the loads keeps the compiler from sinking
    // them below the compute, and the scheduling barrier keeps the compute
    // from moving above them.
    const int last = A.nb - 1;
    Stage s0, s1;
    int c = wave;
    load(c < last ? c : last, s0);
    for (; c + KW < A.nb; c += 2 * KW) {
        load(c + KW, s1);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        compute(s0);
        load(c + 2 * KW < last ? c + 2 * KW : last, s0);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        compute(s1);
    }
    if (c < A.nb) compute(s0);
    // partial tiles of waves 1..3 to LDS; wave 0 adds them in wave order
    if (wave > 0) {
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
#pragma unroll
            for (int i = 0; i < 4; i++) red[wave - 1][nt][i][lane] = y[nt][i];
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int wv = 0; wv < KW - 1; wv++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
#pragma unroll
            for (int i = 0; i < 4; i++) y[nt][i] += red[wv][nt][i][lane];
    const int64_t n0 = (int64_t)blk * 32;
#pragma unroll
    for (int nt = 0; nt < 2; nt++) {
        const int64_t n = n0 + 16 * nt + r16;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int64_t m = 4 * g + i;
            if (m < A.M && n < A.n_out) A.y[m * A.ldy + n] = y[nt][i] * A.yscale;
        }
    }
}

}  // namespace sihip
