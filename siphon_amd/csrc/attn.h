// Decode attention of one layer over an f16 KV cache, bit-identical to the
// reference's x86 path: attn_head (reference engine.c:90-147) with its AVX2
// f16 dot (kernels_avx2.c:118-148), softmax (kernels.c:855-885) and the
// softmax's exp polynomial (kernels.c:820-850).
//
// Three launches on one stream:
//   attn_scores_kernel   sc[h][j] = dot(K[hk][j], f16(q_h)) * kq_scale
//   attn_softmax_kernel  p[h][j] = f16(softmax(sc[h])[j])
//   attn_pv_kernel       out[h][c] = dot(V[hk][c][0..n), p[h])
// or, for n <= kAttnFuseMax, two: attn_scores_kernel, then attn_pv_kernel
// with NG > 0, each of whose waves computes the softmax of its query head
// itself (wave_softmax) into LDS instead of loading probabilities.
//
// The f16 dot is evaluated in the reference's order. Its 32 f32
// accumulators (accumulator a takes elements i with i % 32 == a, by FMA in
// increasing i) are spread over 8 lanes of one row, 4 each: lane L of the
// row holds accumulators 4L..4L+3. The reference reduces them as
// registers r0+r2, r1+r3, then their sum, then lanes l and l+4, then two
// pairwise rounds; with that lane assignment these are additions of lanes
// L + 4, L + 2, L + 1 followed by two in-lane additions. Elements past the last
// multiple of 32 are added to the double total one by one, as in the
// reference.
//
// Each accumulator is one chain of n / 32 dependent FMAs over the whole
// context, so the value contraction cannot be split along the positions
// without changing the result. attn_pv_kernel instead stages a whole
// chunk of value rows and probabilities in LDS with every thread's loads in
// flight at once, then runs the chains out of LDS. Workspace rows (scores
// and probabilities) hold lw >= n entries, lw a multiple of kAttnBlock, so
// whole-block loads stay inside the allocation; entries past n are loaded
// but not used.
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
    float *sc;             // [n_head][ld] scaled scores (caller's, optional)
    uint16_t *p16;         // [n_head][ld] f16 probabilities (caller's, optional)
    float *sw;             // [n_head][lw] scaled scores (workspace)
    uint16_t *pw;          // [n_head][lw] f16 probabilities (workspace)
    int64_t n_ctx, ld, lw;
    int n, hd, gqa, n_head;
    float kq_scale;
};

__device__ inline float f16_at(const uint16_t *p, int64_t i) { return f16_bits_to_f32(p[i]); }

// Lane i receives lane i + K of its 16-lane row (a DPP row shift; lanes
// whose source lies past the row receive 0, and are not used below).
template <int K>
__device__ inline float from_lane_up(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x100 + K, 0xf, 0xf, true));
}

// The reference's tree over the 32 accumulators of one row; lane L of the
// row (lane & 7, rows of 8 lanes) holds acc[e] = accumulator 4L + e. Lane
// L adds lane L + 4 (registers r0 + r2 at L = 0, 1; r1 + r3 at L = 2, 3),
// then lane L + 2 (the sum of those), then lane L + 1 (lanes l and l + 4
// of the reference's 8-wide registers); the result is valid in L == 0.
// Every lane of the wave takes part.
__device__ inline float dot_tree(const float acc[4]) {
    float x[4];
#pragma unroll
    for (int e = 0; e < 4; e++) x[e] = acc[e] + from_lane_up<4>(acc[e]);
#pragma unroll
    for (int e = 0; e < 4; e++) x[e] = x[e] + from_lane_up<2>(x[e]);
#pragma unroll
    for (int e = 0; e < 4; e++) x[e] = x[e] + from_lane_up<1>(x[e]);
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

constexpr int kAttnBlock = 4096;  // softmax positions per workgroup pass (16 per thread)

// exp of a tail position's shifted score (positions past the last whole
// 8-group): exp in double, rounded.
__device__ inline float tail_exp(float x) { return (float)exp((double)x); }

// The softmax of query head h's scores by one wave, for n <= 512 NG (the
// value launch of the two-launch path): lane l holds the 8-groups of
// positions 512 g + 8 l .. + 7, g < NG. The max, the exponentials, each
// group's float sum in the reference's 8-lane order, 1 / total and the f16
// probabilities are attn_softmax_kernel's; only the order in which the
// groups' sums are added in double differs (a 64-lane tree instead of a
// 256-thread one, both within n 2^-53 relative of the reference's
// sequential sum). The tail [gend, n) is added, and its probabilities
// written, by the lane whose group holds it, with tail_exp. The
// probabilities go to pdst[0 .. 512 NG) (positions past n hold values
// that are not used), and to the caller's probs16 where p16_out.
constexpr int kAttnFuseMax = 1024;

template <int NG>
__device__ inline void wave_softmax(const AttnArgs &A, int h, int lane, uint16_t *pdst,
                                    bool p16_out) {
    const int n = A.n, gend = n & ~7;
    const float *row = A.sw + (int64_t)h * A.lw;  // lw >= 512 NG entries
    float v[NG][8];
#pragma unroll
    for (int g = 0; g < NG; g++)
        if (512 * g < n) {  // wave-uniform
            const float4 *p = reinterpret_cast<const float4 *>(row + 512 * g + 8 * lane);
            const float4 a = p[0], b = p[1];
            v[g][0] = a.x, v[g][1] = a.y, v[g][2] = a.z, v[g][3] = a.w;
            v[g][4] = b.x, v[g][5] = b.y, v[g][6] = b.z, v[g][7] = b.w;
        }
    float mx = -__builtin_inff();
#pragma unroll
    for (int g = 0; g < NG; g++)
        if (512 * g < n)
#pragma unroll
            for (int e = 0; e < 8; e++)
                if (512 * g + 8 * lane + e < n && v[g][e] > mx) mx = v[g][e];
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float t = __shfl_xor(mx, o);
        mx = t > mx ? t : mx;
    }
    // the tail's scores, before the exponentials replace them
    const bool tail_owner = gend < n && lane == (gend % 512) / 8;
    float tv[8];
#pragma unroll
    for (int g = 0; g < NG; g++)
        if (g == gend / 512)
#pragma unroll
            for (int e = 0; e < 8; e++) tv[e] = v[g][e];
    double part = 0.0;
#pragma unroll
    for (int g = 0; g < NG; g++)
        if (512 * g < n) {
#pragma unroll
            for (int e = 0; e < 8; e++) v[g][e] = expf_poly(v[g][e] - mx);
            const float *x = v[g];
            if (512 * g + 8 * lane + 8 <= gend)
                part += (double)(((x[0] + x[4]) + (x[2] + x[6])) + ((x[1] + x[5]) + (x[3] + x[7])));
        }
    if (tail_owner)
#pragma unroll
        for (int e = 0; e < 8; e++)
            if (gend + e < n) part += (double)tail_exp(tv[e] - mx);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) part += __shfl_xor(part, o);
    const float scale = (float)(1.0 / part);
#pragma unroll
    for (int g = 0; g < NG; g++)
        if (512 * g < n) {
            const int j0 = 512 * g + 8 * lane;
            uint32_t pk[4];
#pragma unroll
            for (int e = 0; e < 4; e++)
                pk[e] = (uint32_t)f32_to_f16_bits(v[g][2 * e] * scale) |
                        ((uint32_t)f32_to_f16_bits(v[g][2 * e + 1] * scale) << 16);
            *reinterpret_cast<uint4 *>(pdst + j0) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
            if (A.p16 && p16_out)
#pragma unroll
                for (int e = 0; e < 8; e++)
                    if (j0 + e < n)
                        A.p16[(int64_t)h * A.ld + j0 + e] = (uint16_t)(pk[e >> 1] >> (16 * (e & 1)));
        }
    // the tail's probabilities replace the polynomial's (same lane, later stores)
    if (tail_owner)
#pragma unroll
        for (int e = 0; e < 8; e++)
            if (gend + e < n) {
                const uint16_t pb = f32_to_f16_bits(tail_exp(tv[e] - mx) * scale);
                pdst[gend + e] = pb;
                if (A.p16 && p16_out) A.p16[(int64_t)h * A.ld + gend + e] = pb;
            }
}

// Grid (ceil(n / kAttnRows), n_head_kv * ceil(gqa / kAttnHeads)): each
// workgroup scores kAttnRows cached positions against up to kAttnHeads
// query heads of one KV head, holding each key row in registers across
// the heads.
// VEC: hd % 4 == 0 and k 8-byte aligned (a lane's 4 key elements of a step
// in one load).
template <bool VEC>
__global__ __launch_bounds__(kAttnThreads) void attn_scores_kernel(AttnArgs A) {
    __shared__ uint16_t q16[kAttnHeads * kAttnMaxHd];
    const int chunks = (A.gqa + kAttnHeads - 1) / kAttnHeads;
    const int hk = blockIdx.y / chunks;
    const int h0 = hk * A.gqa + (blockIdx.y % chunks) * kAttnHeads;
    const int nh = min(kAttnHeads, hk * A.gqa + A.gqa - h0);
    const int hd = A.hd;
    const int L = threadIdx.x & (kAttnRowLanes - 1);
    const int64_t j = (int64_t)blockIdx.x * kAttnRows + threadIdx.x / kAttnRowLanes;
    const int64_t jr = j < A.n ? j : A.n - 1;  // rows past n score row n-1, unstored
    const uint16_t *krow = A.k + ((int64_t)hk * A.n_ctx + jr) * hd;
    const int body = hd & ~31;
    float kv[kAttnMaxHd / 32][4];
#pragma unroll
    for (int t = 0; t < kAttnMaxHd / 32; t++)
        if (32 * t < body) {
            if constexpr (VEC) {
                const uint2 w = *reinterpret_cast<const uint2 *>(krow + 32 * t + 4 * L);
                kv[t][0] = f16_bits_to_f32(w.x & 0xffffu);
                kv[t][1] = f16_bits_to_f32(w.x >> 16);
                kv[t][2] = f16_bits_to_f32(w.y & 0xffffu);
                kv[t][3] = f16_bits_to_f32(w.y >> 16);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++) kv[t][e] = f16_at(krow, 32 * t + 4 * L + e);
            }
        }
    // the query heads in f16, staged while the key loads are in flight
    for (int i = threadIdx.x; i < nh * hd; i += kAttnThreads)
        q16[i] = f32_to_f16_bits(A.q[(int64_t)h0 * hd + i]);
    __syncthreads();
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
            const float v = (float)total * A.kq_scale;
            A.sw[(int64_t)(h0 + hh) * A.lw + j] = v;
            if (A.sc) A.sc[(int64_t)(h0 + hh) * A.ld + j] = v;
        }
    }
}

// Positions b + 16t .. b + 16t + 15 of a row for thread t: two 8-groups.
struct SoftBlock {
    float v[16];
};

__device__ inline void load_soft_block(const float *row, int b, SoftBlock &blk) {
    const float4 *p = reinterpret_cast<const float4 *>(row + b + 16 * threadIdx.x);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float4 f = p[i];
        blk.v[4 * i] = f.x;
        blk.v[4 * i + 1] = f.y;
        blk.v[4 * i + 2] = f.z;
        blk.v[4 * i + 3] = f.w;
    }
}

// Grid n_head: one workgroup per query head. The max, the total and the
// f16 probabilities each take one pass over the row in blocks of
// kAttnBlock positions; with n <= kAttnBlock the block stays in registers
// and its exponentials are evaluated once.
__global__ __launch_bounds__(kAttnThreads) void attn_softmax_kernel(AttnArgs A) {
    __shared__ float redf[kAttnThreads / 64];
    __shared__ double redd[kAttnThreads / 64];
    const int h = blockIdx.x;
    const float *row = A.sw + (int64_t)h * A.lw;
    const int n = A.n, gend = n & ~7;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const bool one = n <= kAttnBlock;
    SoftBlock blk;
    float mx = -__builtin_inff();
    for (int b = 0; b < n; b += kAttnBlock) {
        load_soft_block(row, b, blk);
#pragma unroll
        for (int e = 0; e < 16; e++)
            if (b + 16 * (int)threadIdx.x + e < n && blk.v[e] > mx) mx = blk.v[e];
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float t = __shfl_xor(mx, o);
        mx = t > mx ? t : mx;
    }
    if (lane == 0) redf[wave] = mx;
    __syncthreads();
    mx = redf[0];
    for (int i = 1; i < kAttnThreads / 64; i++) mx = redf[i] > mx ? redf[i] : mx;
    // total: the 8-groups (lane order of the reference's 8-wide sum), then
    // the tail
    // the thread whose 16 positions hold the tail [gend, n)
    const int tail_b = gend / kAttnBlock * kAttnBlock;
    const bool tail_owner = gend < n && (int)threadIdx.x == (gend - tail_b) / 16;
    double part = 0.0;
    float ex[16];
    for (int b = 0; b < n; b += kAttnBlock) {
        if (!one) load_soft_block(row, b, blk);
#pragma unroll
        for (int e = 0; e < 16; e++) ex[e] = expf_poly(blk.v[e] - mx);
#pragma unroll
        for (int g = 0; g < 2; g++) {
            const int j0 = b + 16 * (int)threadIdx.x + 8 * g;
            const float *v = ex + 8 * g;
            if (j0 + 8 <= gend)
                part += (double)(((v[0] + v[4]) + (v[2] + v[6])) + ((v[1] + v[5]) + (v[3] + v[7])));
        }
    }
    if (tail_owner)
        for (int j = gend; j < n; j++) part += (double)tail_exp(row[j] - mx);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) part += __shfl_xor(part, o);
    if (lane == 0) redd[wave] = part;
    __syncthreads();
    part = redd[0];
    for (int i = 1; i < kAttnThreads / 64; i++) part += redd[i];
    const float scale = (float)(1.0 / part);
    uint16_t *pw = A.pw + (int64_t)h * A.lw;
    for (int b = 0; b < n; b += kAttnBlock) {
        if (!one) {
            load_soft_block(row, b, blk);
#pragma unroll
            for (int e = 0; e < 16; e++) ex[e] = expf_poly(blk.v[e] - mx);
        }
        const int j0 = b + 16 * (int)threadIdx.x;
        uint32_t pk[8];
#pragma unroll
        for (int e = 0; e < 8; e++)
            pk[e] = (uint32_t)f32_to_f16_bits(ex[2 * e] * scale) |
                    ((uint32_t)f32_to_f16_bits(ex[2 * e + 1] * scale) << 16);
        // whole 32-byte pieces into the workspace row (lw entries)
        uint4 *dst = reinterpret_cast<uint4 *>(pw + j0);
        dst[0] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        dst[1] = make_uint4(pk[4], pk[5], pk[6], pk[7]);
        if (A.p16)
            for (int e = 0; e < 16 && j0 + e < n; e++)
                A.p16[(int64_t)h * A.ld + j0 + e] = (uint16_t)(pk[e >> 1] >> (16 * (e & 1)));
    }
    // the tail's probabilities replace the polynomial's (same thread, later stores)
    if (tail_owner)
        for (int j = gend; j < n; j++) {
            const uint16_t pb = f32_to_f16_bits(tail_exp(row[j] - mx) * scale);
            pw[j] = pb;
            if (A.p16) A.p16[(int64_t)h * A.ld + j] = pb;
        }
}

// Grid (ceil(hd / kAttnPvRows), n_head_kv * ceil(gqa / kAttnHeads)):
// each workgroup owns kAttnPvRows value rows of one KV head and up to
// kAttnHeads query heads of it, wave w running head h0 + w. Per chunk of
// kAttnChunk positions every thread requests its share of the value rows
// and probability rows at once, stores them to LDS, and each wave runs its
// accumulator chains over the chunk: lane 8r + L holds accumulators
// 4L..4L+3 of row r. Then the reduction tree, the tail (inside the last
// chunk) and the store.
constexpr int kAttnPvRows = 8;
constexpr int kAttnChunk = 2048;  // positions per LDS chunk (a multiple of 32, divides kAttnBlock)
constexpr int kAttnVPieces = kAttnPvRows * kAttnChunk / 8 / kAttnThreads;  // 16-byte pieces
constexpr int kAttnPPieces = kAttnHeads * kAttnChunk / 8 / kAttnThreads;

// VEC: n_ctx % 8 == 0 and v 16-byte aligned (16-byte value pieces).
// NG > 0 (n <= 512 NG <= kAttnChunk, one chunk): wave w computes the
// softmax of head h0 + w itself (wave_softmax<NG>, from the scores launch's
// scores) into its LDS probability row while the value rows load, in place
// of loading probabilities; the caller's probs16 is written by the
// workgroups of blockIdx.x == 0.
template <bool VEC, int NG>
__global__ __launch_bounds__(kAttnThreads) void attn_pv_kernel(AttnArgs A) {
    __shared__ __attribute__((aligned(16))) uint16_t sv[kAttnPvRows * kAttnChunk];
    __shared__ __attribute__((aligned(16))) uint16_t sp[kAttnHeads * kAttnChunk];
    const int chunks = (A.gqa + kAttnHeads - 1) / kAttnHeads;
    const int hk = blockIdx.y / chunks;
    const int h0 = hk * A.gqa + (blockIdx.y % chunks) * kAttnHeads;
    const int nh = min(kAttnHeads, hk * A.gqa + A.gqa - h0);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const bool active = wave < nh;
    const int n = A.n, body = n & ~31;
    const int r = lane >> 3, L = lane & 7;
    const int c = blockIdx.x * kAttnPvRows + r;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int s0 = 0;
    for (;; s0 += kAttnChunk) {
        const int cl = min(kAttnChunk, n - s0);
        const int per_row = (cl + 7) / 8;  // 16-byte pieces of a row in this chunk
        // probability rows: whole pieces of the workspace (lw >= s0 + kAttnChunk);
        // heads past nh repeat head nh - 1
        uint4 pq[kAttnPPieces];
        if constexpr (NG == 0) {
#pragma unroll
            for (int i = 0; i < kAttnPPieces; i++) {
                const int t = threadIdx.x + kAttnThreads * i;
                const int hh = min(t / (kAttnChunk / 8), nh - 1), pc = t % (kAttnChunk / 8);
                pq[i] = reinterpret_cast<const uint4 *>(A.pw + (int64_t)(h0 + hh) * A.lw + s0)[pc];
            }
        }
        if constexpr (VEC) {
            // value rows (rows past hd repeat row hd - 1); pieces past the
            // chunk's end load the chunk's last piece again (n_ctx % 8 == 0:
            // it ends inside the row)
            uint4 vq[kAttnVPieces];
#pragma unroll
            for (int i = 0; i < kAttnVPieces; i++) {
                const int t = threadIdx.x + kAttnThreads * i;
                const int rr = t / (kAttnChunk / 8), pc = min(t % (kAttnChunk / 8), per_row - 1);
                const int cr = min(blockIdx.x * kAttnPvRows + rr, A.hd - 1);
                vq[i] = reinterpret_cast<const uint4 *>(
                    A.v + ((int64_t)hk * A.hd + cr) * A.n_ctx + s0)[pc];
            }
#pragma unroll
            for (int i = 0; i < kAttnVPieces; i++) {
                const int t = threadIdx.x + kAttnThreads * i;
                reinterpret_cast<uint4 *>(sv)[t] = vq[i];
            }
        } else {
#pragma unroll 8
            for (int t = threadIdx.x; t < kAttnPvRows * cl; t += kAttnThreads) {
                const int rr = t / cl, i = t - rr * cl;
                const int cr = min(blockIdx.x * kAttnPvRows + rr, A.hd - 1);
                sv[rr * kAttnChunk + i] = A.v[((int64_t)hk * A.hd + cr) * A.n_ctx + s0 + i];
            }
        }
        if constexpr (NG > 0) {
            if (active) wave_softmax<NG>(A, h0 + wave, lane, sp + wave * kAttnChunk, blockIdx.x == 0);
        } else {
#pragma unroll
            for (int i = 0; i < kAttnPPieces; i++)
                reinterpret_cast<uint4 *>(sp)[threadIdx.x + kAttnThreads * i] = pq[i];
        }
        __syncthreads();
        // the accumulator chains over the chunk's whole 32-steps
        if (active) {
            const uint16_t *vr = sv + r * kAttnChunk;
            const uint16_t *pr = sp + wave * kAttnChunk;
            const int steps_end = min(body - s0, cl);
#pragma unroll 4
            for (int i0 = 0; i0 < steps_end; i0 += 32) {
                const int i = i0 + 4 * L;
                const uint2 vw = *reinterpret_cast<const uint2 *>(vr + i);
                const uint2 pw = *reinterpret_cast<const uint2 *>(pr + i);
                acc[0] = __builtin_fmaf(f16_bits_to_f32(vw.x & 0xffffu), f16_bits_to_f32(pw.x & 0xffffu), acc[0]);
                acc[1] = __builtin_fmaf(f16_bits_to_f32(vw.x >> 16), f16_bits_to_f32(pw.x >> 16), acc[1]);
                acc[2] = __builtin_fmaf(f16_bits_to_f32(vw.y & 0xffffu), f16_bits_to_f32(pw.y & 0xffffu), acc[2]);
                acc[3] = __builtin_fmaf(f16_bits_to_f32(vw.y >> 16), f16_bits_to_f32(pw.y >> 16), acc[3]);
            }
        }
        if (s0 + cl >= n) break;
        __syncthreads();  // the next chunk overwrites sv and sp
    }
    // the tail [body, n) lies in the last chunk, still in LDS
    const float res = dot_tree(acc);
    if (active && L == 0 && c < A.hd) {
        const int h = h0 + wave;
        double total = 0.0;
        total += (double)res;
        for (int j = body; j < n; j++)
            total += (double)(f16_bits_to_f32(sv[r * kAttnChunk + j - s0]) *
                              f16_bits_to_f32(sp[wave * kAttnChunk + j - s0]));
        A.out[(int64_t)h * A.hd + c] = (float)total;
    }
}

}  // namespace sihip
