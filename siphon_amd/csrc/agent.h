// Loads that see other workgroups' agent-scope stores (device code only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// The cross-workgroup hand-off of K-slice and column-slice partial sums
// (slices_finish here, g2_slices_finish in gemm2.h, kf_finish in gemmkf.h,
// split_reduce in matvec.h) relies on what gfx950 does,
// not on the HIP memory model: sc1 stores and loads bypass the per-XCD L2,
// s_waitcnt vmcnt(0) waits for a wave's stores to complete before its
// workgroup counts its arrival with a relaxed agent-scope atomic, and the
// last workgroup's sc1 loads are issued after that count returns. Another
// target needs that ordering shown again (or release/acquire arrivals)
// before these kernels are built for it.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "agent.h: the K-slice partial-sum hand-off is validated on gfx950 only (sc1 stores/loads, vmcnt(0) before a relaxed agent-scope arrival count)"
#endif

namespace sihip {

// A load at agent scope (sc1: coherent across the XCDs' L2 caches, like an
// agent-scope atomic load) that the compiler does not serialize: atomic
// loads get a wait each, so a run of them costs one round trip apiece.
__device__ inline float load_agent_f32(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)byte_off, 0, 16));
}

// End of a K-sliced GEMM tile, after each wave of the workgroup has issued
// its agent-scope stores of the slice's partial sums into
// part[(slice * Mp + m) * ldp + n]: count the workgroup's arrival on *cnt;
// the last of the S workgroups of the tile adds the S partial tiles in
// slice order (so the result does not depend on arrival order) into
// y[m * ldy + n] for the tile's rows m0 .. m0 + BM - 1 below M and columns
// n0 .. n0 + BN - 1 below n_out, and resets the counter to zero for the
// next launch. Rows past M were not written and are not read.
//
// Ordering: each wave's partial-sum stores have completed (vmcnt 0) before
// the barrier and hence before the arrival is counted; the last
// workgroup's agent-scope loads are issued after the barrier that follows
// the count's return. The signal fences keep the compiler from moving
// memory operations across these points (they emit no instruction). The
// count itself stays relaxed: the partial sums never live in the
// non-coherent per-XCD L2 (sc1 stores and loads), and an agent-scope
// release or acquire would write back or invalidate that whole L2 on every
// arrival (measured: K-sliced Q4_K GEMMs 25-40% slower).
template <int BM, int BN, int THREADS>
__device__ inline void slices_finish(const float *part, uint32_t *cnt, int S, int64_t Mp,
                                     int64_t ldp, int64_t m0, int64_t M, int64_t n0,
                                     int64_t n_out, float *y, int64_t ldy) {
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
    // this thread's outputs: rows m0 + idx / BN, columns n0 + idx % BN for
    // idx = tid + THREADS q; the loads of kU slices (32 per thread, or
    // kOut if more) are issued together, since each group of loads costs a
    // round trip to memory (agent-scope loads miss the XCD's L2), and are
    // added in slice order
    constexpr int kOut = BM * BN / THREADS;
    constexpr int kU = kOut >= 32 ? 1 : 32 / kOut;
    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(part), (short)0, (int)((int64_t)S * Mp * ldp * 4), 0x00020000);
    const int64_t nn = n0 + threadIdx.x % BN;
    // byte offset of output q in slice sl; rows past M were not written:
    // read row 0's value, unused
    auto off = [&](int sl, int q) -> uint32_t {
        const int64_t m = m0 + (threadIdx.x + THREADS * q) / BN;
        return (uint32_t)((((int64_t)sl * Mp + (m < M ? m : 0)) * ldp + nn) * 4);
    };
    float v[kOut];
#pragma unroll
    for (int q = 0; q < kOut; q++) v[q] = 0.0f;
    int sl = 0;
    for (; sl + kU <= S; sl += kU) {
        float pv[kU][kOut];
#pragma unroll
        for (int u = 0; u < kU; u++)
#pragma unroll
            for (int q = 0; q < kOut; q++) pv[u][q] = load_agent_f32(pr, off(sl + u, q));
#pragma unroll
        for (int u = 0; u < kU; u++)
#pragma unroll
            for (int q = 0; q < kOut; q++) v[q] += pv[u][q];
    }
    if constexpr (kU > 1) {
        for (; sl < S; sl++) {
            float pv[kOut];
#pragma unroll
            for (int q = 0; q < kOut; q++) pv[q] = load_agent_f32(pr, off(sl, q));
#pragma unroll
            for (int q = 0; q < kOut; q++) v[q] += pv[q];
        }
    }
    if (nn < n_out) {
#pragma unroll
        for (int q = 0; q < kOut; q++) {
            const int64_t m = m0 + (threadIdx.x + THREADS * q) / BN;
            if (m < M) y[m * ldy + nn] = v[q];
        }
    }
    if (threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace sihip
