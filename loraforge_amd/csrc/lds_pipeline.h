// Building blocks of the direct-copy LDS pipelines (decode and prefill
// kernels): global -> LDS copies, explicit vmcnt waits, LDS reads the
// compiler does not track, and workgroup barriers that wait for LDS only.
//
// Why untracked reads: while global -> LDS copies are in flight the compiler
// waits for every outstanding memory operation before any LDS read it
// tracks (it cannot tell which LDS bytes a copy writes). The kernels know
// which copies a read depends on and wait for exactly those (wait_vm), then
// tie the read results to the wait so no use is scheduled above it.
#pragma once

#include "common.h"

namespace lf {

template <class T>
__device__ __forceinline__ T sload(const T* base, int idx) {
  typedef const __attribute__((address_space(4))) T* ConstPtr;
  return ((ConstPtr)base)[idx];
}

__device__ __forceinline__ void barrier_only() { asm volatile("s_barrier" ::: "memory"); }

// Workgroup barrier after this wave's LDS accesses completed (lgkmcnt(0)),
// without waiting for its global memory operations.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);
  barrier_only();
}

template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0xF << 8) | (7 << 4));  // vmcnt(N) only
}

__device__ __forceinline__ void copy16(const void* src, char* lds) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}
__device__ __forceinline__ void copy4(const void* src, char* lds) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 4, 0, 0);
}

// LDS reads the compiler does not track (results valid after an explicit
// lgkmcnt wait and tie).
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ bf16x8 vec_bf16x8(const u32x4& v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ u32x2 lds_read64(uint32_t addr) {
  u32x2 v;
  asm volatile("ds_read_b64 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}
__device__ __forceinline__ u32x4 lds_read128(uint32_t addr) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}
__device__ __forceinline__ float lds_read32f(uint32_t addr) {
  float v;
  asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p));
}

// Adds one to a workgroup counter in LDS (a wave counting in). Through the
// compiler, an LDS atomic after direct global -> LDS copies gets a vmcnt(0)
// in front of it (the atomic is assumed to alias the copies' destinations),
// which drains every copy in flight; the caller waits lgkmcnt(0) for its own
// LDS writes first, and the counter is a location no copy writes.
__device__ __forceinline__ void lds_count_in(int* counter) {
  asm volatile("ds_add_u32 %0, %1" ::"v"(lds_addr(counter)), "v"(1) : "memory");
}

// Ties a value to the wait made before it: uses cannot be scheduled above.
template <class T>
__device__ __forceinline__ void tie(T& v) {
  asm volatile("" : "+v"(v));
}

__device__ __forceinline__ uint32_t lds_read32(uint32_t addr) {
  uint32_t v;
  asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}

__device__ __forceinline__ void lds_wait() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// A 16-byte global load into registers that the compiler does not track.
// While direct LDS copies are in flight, the compiler waits for every
// outstanding memory operation before using any tracked load result; the
// kernels wait for these loads with an explicit vmcnt (loads complete in
// issue order) and tie the result to that wait before its first use.
__device__ __forceinline__ u32x4 global_load128_untracked(const void* ptr) {
  u32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(ptr) : "memory");
  return v;
}

// The same for the lanes of `lanes` only (the others keep zero and issue no
// memory request): the whole exec change stays inside the statement.
__device__ __forceinline__ u32x4 global_load128_untracked_masked(const void* ptr, uint64_t lanes) {
  u32x4 v = {0u, 0u, 0u, 0u};
  uint64_t saved;
  asm volatile(
      "s_and_saveexec_b64 %1, %3\n\t"
      "global_load_dwordx4 %0, %2, off\n\t"
      "s_mov_b64 exec, %1"
      : "+v"(v), "=&s"(saved)
      : "v"(ptr), "s"(lanes)
      : "memory", "exec");
  return v;
}

// A pointer computed from uniform values, moved to scalar registers.
template <class T>
__device__ __forceinline__ const T* uniform_ptr(const T* p) {
  const uint64_t a = reinterpret_cast<uintptr_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(a >> 32));
  return reinterpret_cast<const T*>((uint64_t(hi) << 32) | lo);
}

// An ordinary 16-byte load from global memory at a uniform base plus a
// 32-bit per-lane byte offset (a global, not flat, load: flat loads also
// count as LDS operations and hold back the next direct copy).
__device__ __forceinline__ u32x4 global_load128(const void* base, uint32_t off) {
  typedef const __attribute__((address_space(1))) char* GPtr;
  return *(const __attribute__((address_space(1))) u32x4*)((GPtr)base + off);
}

}  // namespace lf
