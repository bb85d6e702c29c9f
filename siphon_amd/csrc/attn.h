// Decode attention of one layer over an f16 KV cache, bit-identical to the
// reference's x86 path: attn_head (reference engine.c:90-147) with its AVX2
// f16 dot (kernels_avx2.c:118-148), softmax (kernels.c:855-885) and the
// softmax's exp polynomial (kernels.c:820-850).
//
// Three launches on one stream:
//   attn_scores_kernel   sc[h][j] = dot(K[hk][j], f16(q_h)) * kq_scale
//   attn_softmax_kernel  p16[h][j] = f16(softmax(sc[h])[j])
//   attn_values_kernel   out[h][c] = dot(V[hk][c][0..n), p16[h])
//
// The f16 dot is evaluated in the reference's order. Its 32 f32
// accumulators (accumulator a takes elements i with i % 32 == a, by FMA in
// increasing i) are spread over 8 lanes of one row, 4 each: lane L of the
// row holds accumulators 4L..4L+3. The reference reduces them as
// registers r0+r2, r1+r3, then their sum, then lanes l and l+4, then two
// pairwise rounds; with that lane assignment these are the lane-xor steps
// 4, 2, 1 followed by two in-lane additions. Elements past the last
// multiple of 32 are added to the double total one by one, as in the
// reference.
//
// The softmax sums its 8-element group totals in double in a tree rather
// than in the reference's sequential order. The two double totals differ
// by at most n * 2^-53 relative, which changes the float 1/total only when
// that lies within that distance of a float rounding boundary (about 1e-6
// of heads at n = 4096). Tail elements (n % 8) use expf in the reference
// (libm): here exp in double rounded to float, which differs from glibc's
// expf in about 0.07% of arguments by one float ulp, and such a difference
// survives the f16 rounding of its probability only rarely.
#pragma once

#include "quant.h"

namespace sihip {

constexpr int kAttnThreads = 256;
constexpr int kAttnRowLanes = 8;                                // lanes per dot
constexpr int kAttnRows = kAttnThreads / kAttnRowLanes;         // dots per workgroup
constexpr int kAttnHeads = 4;                                   // query heads per pass
constexpr int kAttnMaxHd = 512;

struct AttnArgs {
    const float *q;        // [n_head * hd]
    const uint16_t *k;     // [n_head_kv][n_ctx][hd]
    const uint16_t *v;     // [n_head_kv][hd][n_ctx]
    float *out;            // [n_head * hd]
    float *sc;             // [n_head][ld] scaled scores
    uint16_t *p16;         // [n_head][ld] f16 probabilities
    int64_t n_ctx, ld;
    int n, hd, gqa, n_head;
    float kq_scale;
};

__device__ inline float f16_at(const uint16_t *p, int64_t i) { return f16_bits_to_f32(p[i]); }

// The reference's tree over the 32 accumulators of one row; lane L of the
// row (lane & 7) holds acc[e] = accumulator 4L + e. Every lane of the wave
// takes part; the result is valid in lane L == 0.
__device__ inline float dot_tree(const float acc[4]) {
    float x[4];
#pragma unroll
    for (int e = 0; e < 4; e++) x[e] = acc[e] + __shfl_xor(acc[e], 4);  // r0 + r2, r1 + r3
#pragma unroll
    for (int e = 0; e < 4; e++) x[e] = x[e] + __shfl_xor(x[e], 2);      // (r0+r2) + (r1+r3)
#pragma unroll
    for (int e = 0; e < 4; e++) x[e] = x[e] + __shfl_xor(x[e], 1);      // lanes l + (l + 4)
    return (x[0] + x[1]) + (x[2] + x[3]);
}

// exp of the softmax groups: the polynomial the reference uses there (its
// constants and branch structure kept, since the result is compared bit
// for bit): x = n ln2 + b with n from the 1.5 * 2^23 rounding shift and ln2
// in two parts, a polynomial in b, and 2^n built in the exponent field;
// |n| > 126 scales by two factors, |n| > 192 saturates.
__device__ inline float expf_poly(float x) {
    const float shift = 0x1.8p23f;
    const float z = __builtin_fmaf(x, 0x1.715476p+0f, shift);
    const float n = z - shift;
    const float b = __builtin_fmaf(-n, 0x1.7f7d1cp-20f, __builtin_fmaf(-n, 0x1.62e4p-1f, x));
    const uint32_t e = __float_as_uint(z) << 23;
    const float k = __uint_as_float(e + 0x3f800000u);
    const float u = b * b;
    const float p = __builtin_fmaf(
        __builtin_fmaf(__builtin_fmaf(0x1.0e4020p-7f, b, 0x1.573e2ep-5f), u,
                       __builtin_fmaf(0x1.555e66p-3f, b, 0x1.fffdb6p-2f)),
        u, 0x1.ffffecp-1f * b);
    if (!(__builtin_fabsf(n) > 126.0f)) return __builtin_fmaf(p, k, k);
    const uint32_t g = n <= 0.0f ? 0x82000000u : 0u;
    const float s1 = __uint_as_float(g + 0x7f000000u);
    if (__builtin_fabsf(n) > 192.0f) return s1 * s1;
    const float s2 = __uint_as_float(e - g);
    return __builtin_fmaf(s2, p, s2) * s1;
}

// Grid (ceil(n / kAttnRows), n_head_kv * ceil(gqa / kAttnHeads)): each
// workgroup scores kAttnRows cached positions against up to kAttnHeads
// query heads of one KV head, holding each key row in registers across
// the heads.
__global__ __launch_bounds__(kAttnThreads) void attn_scores_kernel(AttnArgs A) {
    __shared__ uint16_t q16[kAttnHeads * kAttnMaxHd];
    const int chunks = (A.gqa + kAttnHeads - 1) / kAttnHeads;
    const int hk = blockIdx.y / chunks;
    const int h0 = hk * A.gqa + (blockIdx.y % chunks) * kAttnHeads;
    const int nh = min(kAttnHeads, hk * A.gqa + A.gqa - h0);
    const int hd = A.hd;
    for (int i = threadIdx.x; i < nh * hd; i += kAttnThreads)
        q16[i] = f32_to_f16_bits(A.q[(int64_t)h0 * hd + i]);
    __syncthreads();
    const int L = threadIdx.x & (kAttnRowLanes - 1);
    const int64_t j = (int64_t)blockIdx.x * kAttnRows + threadIdx.x / kAttnRowLanes;
    const int64_t jr = j < A.n ? j : A.n - 1;  // rows past n score row n-1, unstored
    const uint16_t *krow = A.k + ((int64_t)hk * A.n_ctx + jr) * hd;
    const int body = hd & ~31;
    float kv[kAttnMaxHd / 32][4];
#pragma unroll
    for (int t = 0; t < kAttnMaxHd / 32; t++)
        if (32 * t < body)
#pragma unroll
            for (int e = 0; e < 4; e++) kv[t][e] = f16_at(krow, 32 * t + 4 * L + e);
    for (int hh = 0; hh < nh; hh++) {
        const uint16_t *qh = q16 + hh * hd;
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < kAttnMaxHd / 32; t++)
            if (32 * t < body)
#pragma unroll
                for (int e = 0; e < 4; e++)
                    acc[e] = __builtin_fmaf(kv[t][e], f16_bits_to_f32(qh[32 * t + 4 * L + e]), acc[e]);
        const float res = dot_tree(acc);
        if (L == 0 && j < A.n) {
            double total = 0.0;
            total += (double)res;
            for (int i = body; i < hd; i++)
                total += (double)(f16_at(krow, i) * f16_bits_to_f32(qh[i]));
            A.sc[(int64_t)(h0 + hh) * A.ld + j] = (float)total * A.kq_scale;
        }
    }
}

// Block-wide reductions over kAttnThreads threads.
__device__ inline float block_max(float m, float *red) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float t = __shfl_xor(m, o);
        m = t > m ? t : m;
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = m;
    __syncthreads();
    m = red[0];
    for (int i = 1; i < kAttnThreads / 64; i++) m = red[i] > m ? red[i] : m;
    __syncthreads();
    return m;
}

__device__ inline double block_sum(double s, double *red) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = s;
    __syncthreads();
    s = red[0];
    for (int i = 1; i < kAttnThreads / 64; i++) s += red[i];
    return s;
}

// Grid n_head: one workgroup per query head. Exponentials are evaluated
// twice (for the total, then for the probabilities) rather than stored.
__global__ __launch_bounds__(kAttnThreads) void attn_softmax_kernel(AttnArgs A) {
    __shared__ float redf[kAttnThreads / 64];
    __shared__ double redd[kAttnThreads / 64];
    const float *sc = A.sc + (int64_t)blockIdx.x * A.ld;
    uint16_t *p16 = A.p16 + (int64_t)blockIdx.x * A.ld;
    const int n = A.n;
    float m = -__builtin_inff();
    for (int j = threadIdx.x; j < n; j += kAttnThreads) m = sc[j] > m ? sc[j] : m;
    const float mx = block_max(m, redf);
    const int groups = n / 8;
    double part = 0.0;
    for (int g = threadIdx.x; g < groups; g += kAttnThreads) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = expf_poly(sc[8 * g + e] - mx);
        part += (double)(((v[0] + v[4]) + (v[2] + v[6])) + ((v[1] + v[5]) + (v[3] + v[7])));
    }
    if (threadIdx.x == 0)
        for (int j = 8 * groups; j < n; j++) part += (double)(float)exp((double)(sc[j] - mx));
    const double total = block_sum(part, redd);
    const float scale = (float)(1.0 / total);
    for (int j = threadIdx.x; j < n; j += kAttnThreads) {
        const float x = sc[j] - mx;
        const float e = j < 8 * groups ? expf_poly(x) : (float)exp((double)x);
        p16[j] = f32_to_f16_bits(e * scale);
    }
}

// Grid (ceil(hd / kAttnRows), n_head_kv * ceil(gqa / kAttnHeads)): each
// workgroup contracts kAttnRows value rows with up to kAttnHeads
// probability rows of one KV head, each value element read once for all
// of them.
__global__ __launch_bounds__(kAttnThreads) void attn_values_kernel(AttnArgs A) {
    const int chunks = (A.gqa + kAttnHeads - 1) / kAttnHeads;
    const int hk = blockIdx.y / chunks;
    const int h0 = hk * A.gqa + (blockIdx.y % chunks) * kAttnHeads;
    const int nh = min(kAttnHeads, hk * A.gqa + A.gqa - h0);
    const int L = threadIdx.x & (kAttnRowLanes - 1);
    const int c = blockIdx.x * kAttnRows + threadIdx.x / kAttnRowLanes;
    const int cr = c < A.hd ? c : A.hd - 1;
    const uint16_t *vrow = A.v + ((int64_t)hk * A.hd + cr) * A.n_ctx;
    const uint16_t *prow[kAttnHeads];
#pragma unroll
    for (int hh = 0; hh < kAttnHeads; hh++)
        prow[hh] = A.p16 + (int64_t)(h0 + (hh < nh ? hh : nh - 1)) * A.ld;
    const int n = A.n, body = n & ~31;
    float acc[kAttnHeads][4];
#pragma unroll
    for (int hh = 0; hh < kAttnHeads; hh++)
#pragma unroll
        for (int e = 0; e < 4; e++) acc[hh][e] = 0.0f;
#pragma unroll 4
    for (int i0 = 0; i0 < body; i0 += 32) {
        const int i = i0 + 4 * L;
        float vv[4];
#pragma unroll
        for (int e = 0; e < 4; e++) vv[e] = f16_at(vrow, i + e);
#pragma unroll
        for (int hh = 0; hh < kAttnHeads; hh++)
#pragma unroll
            for (int e = 0; e < 4; e++)
                acc[hh][e] = __builtin_fmaf(vv[e], f16_at(prow[hh], i + e), acc[hh][e]);
    }
#pragma unroll
    for (int hh = 0; hh < kAttnHeads; hh++) {
        const float res = dot_tree(acc[hh]);
        if (L == 0 && hh < nh && c < A.hd) {
            double total = 0.0;
            total += (double)res;
            for (int i = body; i < n; i++)
                total += (double)(f16_at(vrow, i) * f16_at(prow[hh], i));
            A.out[(int64_t)(h0 + hh) * A.hd + c] = (float)total;
        }
    }
}

}  // namespace sihip
