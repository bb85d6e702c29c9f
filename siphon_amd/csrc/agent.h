// Loads that see other workgroups' agent-scope stores (device code only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sihip {

// A load at agent scope (sc1: coherent across the XCDs' L2 caches, like an
// agent-scope atomic load) that the compiler does not serialize: atomic
// loads get a wait each, so a run of them costs one round trip apiece.
__device__ inline float load_agent_f32(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)byte_off, 0, 16));
}

}  // namespace sihip
