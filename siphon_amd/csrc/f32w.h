// F32 weights (reference pair F32: backend.c:102-103 passes x through
// unconverted; si_dot_f32, kernels.c:180-187, sums the float products in
// double). The device keeps the tensor's rows as they are (row-major f32)
// and streams them once per launch of up to kF32Cols activation columns;
// each wave computes one row: lanes take 16-byte strides of the row, the
// float products accumulate per lane in f32 and the lanes are added in a
// fixed tree, so results are deterministic (within the path's tolerance of
// the reference's double sum).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sihip {

constexpr int kF32Threads = 256;
constexpr int kF32Cols = 4;

template <int NC>
__global__ __launch_bounds__(kF32Threads) void f32_matvec_kernel(const float *W, int64_t n_in,
                                                                 int64_t n_out, const float *x,
                                                                 int64_t ldx, float *y,
                                                                 int64_t ldy) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * (kF32Threads / 64) + (threadIdx.x >> 6);
    if (row >= n_out) return;  // whole waves
    const float *w = W + row * n_in;
    float acc[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) acc[c] = 0.0f;
    // rows and x are 16-byte aligned when n_in % 4 == 0 (the host checks x)
    if ((n_in & 3) == 0) {
        const int64_t n4 = n_in >> 2;
        for (int64_t i = lane; i < n4; i += 64) {
            const float4 wv = reinterpret_cast<const float4 *>(w)[i];
#pragma unroll
            for (int c = 0; c < NC; c++) {
                const float4 xv = reinterpret_cast<const float4 *>(x + c * ldx)[i];
                acc[c] += wv.x * xv.x;
                acc[c] += wv.y * xv.y;
                acc[c] += wv.z * xv.z;
                acc[c] += wv.w * xv.w;
            }
        }
    } else {
        for (int64_t i = lane; i < n_in; i += 64) {
            const float wv = w[i];
#pragma unroll
            for (int c = 0; c < NC; c++) acc[c] += wv * x[c * ldx + i];
        }
    }
#pragma unroll
    for (int c = 0; c < NC; c++) {
        float v = acc[c];
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
        if (lane == 0) y[c * ldy + row] = v;
    }
}

// Rows [row0, row0 + nrows) copied to out (row r - row0 at out + (r - row0) * ldo).
__global__ __launch_bounds__(kF32Threads) void f32_rows_kernel(const float *W, int64_t n_in,
                                                               int64_t row0, int64_t nrows,
                                                               float *out, int64_t ldo) {
    const int64_t i = (int64_t)blockIdx.x * kF32Threads + threadIdx.x;
    if (i >= nrows * n_in) return;
    const int64_t r = i / n_in, k = i % n_in;
    out[r * ldo + k] = W[(row0 + r) * n_in + k];
}

}  // namespace sihip
