// Per-call tags for kernels that publish data to other workgroups of the
// same launch through a caller-owned workspace (decode shrink partials,
// prefill z rows).
//
// Every workgroup reads the epoch word at its start; the call's tag is
// epoch + 1. Once it holds its tag a workgroup counts itself in (one counter
// per blockIdx % 8, so no single address takes every atomic; it may do so
// right away and look at the returned count only at its end); the last of a
// group counts the group in, and the last group resets the counters and moves
// the epoch on. Every workgroup has read the epoch before it counts in, so all
// workgroups of a call see the same tag and no earlier call used it (tags
// cycle through 1 .. 2^32 - 1; zero never marks data, so a zeroed workspace
// holds no valid entry). Calls that share a workspace must not overlap.
#pragma once

#include "common.h"

namespace lf {

struct CallEpoch {
  uint32_t* epoch;   // the call's tag is epoch + 1
  uint32_t* groups;  // 8 arrival counters, 128 bytes apart
  uint32_t* total;   // groups counted in
};

__device__ __forceinline__ uint32_t epoch_tag(const CallEpoch& ce) {
  return __hip_atomic_load(ce.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
}

// A per-lane zero the compiler cannot see through: an atomic on a provably
// uniform address is turned into a wave-wide one whose result is waited for
// on the spot.
__device__ __forceinline__ uint32_t opaque_zero() {
  uint32_t z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  return z;
}

// Counts this workgroup in (lane 0); the old count is returned in lane 0 and
// nothing waits for it until depart_finish.
__device__ __forceinline__ uint32_t depart_issue(const CallEpoch& ce, int lane) {
  uint32_t* counter = ce.groups + 32 * (blockIdx.x & 7) + opaque_zero();
  uint32_t old = 0;
  if (lane == 0) old = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return old;
}

// The last workgroup of its group counts the group in; the last group
// resets the counts and moves the epoch on (epoch = tag - 1 of this call).
__device__ __forceinline__ void depart_finish(const CallEpoch& ce, uint32_t old, uint32_t epoch, int lane) {
  if (lane != 0) return;
  const uint32_t g = blockIdx.x & 7;
  const uint32_t members = (gridDim.x - g + 7) / 8;
  if (old != members - 1) return;
  __hip_atomic_store(ce.groups + 32 * g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint32_t groups = gridDim.x < 8 ? gridDim.x : 8u;
  if (__hip_atomic_fetch_add(ce.total, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != groups - 1) return;
  __hip_atomic_store(ce.total, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(ce.epoch, epoch + 1 == 0xffffffffu ? 0u : epoch + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Control header of a fused-linear workspace: epoch, status, the eight group
// arrival counts (128 bytes apart), the group total.
constexpr int64_t kEpochOffset = 0;
constexpr int64_t kStatusOffset = 8;
constexpr int64_t kGroupsOffset = 128;
constexpr int64_t kTotalOffset = kGroupsOffset + 8 * 128;

__host__ inline CallEpoch call_epoch_of(void* workspace) {
  char* ws = static_cast<char*>(workspace);
  return CallEpoch{reinterpret_cast<uint32_t*>(ws + kEpochOffset), reinterpret_cast<uint32_t*>(ws + kGroupsOffset),
                   reinterpret_cast<uint32_t*>(ws + kTotalOffset)};
}

}  // namespace lf
