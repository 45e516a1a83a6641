// Shared device helpers and host error plumbing for the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

namespace lf {

// ---------------------------------------------------------------------------
// Status codes returned by every extern "C" entry point.
// ---------------------------------------------------------------------------
enum Status : int {
  kOk = 0,
  kInvalid = 1,  // argument / layout contract violated (maps to ValueError)
  kHip = 2,      // HIP runtime error (maps to RuntimeError)
};

void set_error(const char* fmt, ...);
int fail(int code, const char* fmt, ...);
int hip_status(hipError_t err, const char* what);

#define LF_REQUIRE(cond, ...)                  \
  do {                                         \
    if (!(cond)) return ::lf::fail(::lf::kInvalid, __VA_ARGS__); \
  } while (0)

#define LF_HIP(call)                                     \
  do {                                                   \
    hipError_t lf_err_ = (call);                         \
    if (lf_err_ != hipSuccess) return ::lf::hip_status(lf_err_, #call); \
  } while (0)

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---------------------------------------------------------------------------
// Vector types used for MFMA operands and 128-bit memory traffic.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// bf16 bits -> fp32 (exact).
__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
__device__ __forceinline__ float bf16_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t pair) { return __uint_as_float(pair & 0xffff0000u); }

// Two fp32 -> packed bf16 pair (low half = a), round-to-nearest-even.
// gfx950 lowers this to one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2 v = __builtin_convertvector((f32x2){a, b}, bf16x2);
  return __builtin_bit_cast(uint32_t, v);
}

// fp32 -> bf16 bits, round-to-nearest-even.
__device__ __forceinline__ uint32_t f32_to_bf16(float a) { return pack_bf16x2(a, 0.0f) & 0xffffu; }

// fp32 -> nearest bf16 value, returned as fp32.
__device__ __forceinline__ float round_bf16(float a) { return bf16_to_f32(f32_to_bf16(a)); }

// bf16(silu(g)) * u in fp32 (the caller's store rounds the product to bf16),
// silu(g) = g / (1 + e^-g) as the reference's activation
// (benchmarks/qwen35_decode_silu.py:60-61), in about 13 instructions instead
// of about 30 for expf and an IEEE division:
//  - e^-g = 2^(t + lo) = 2^t (1 + lo ln 2) with t = fl(-c log2 e) and lo the
//    rounding error of t plus c times the tail of log2 e (Cody-Waite), 2^t
//    from the hardware exp2 (1 ulp); c is g clamped to [-126, 126], which
//    changes nothing past the clamp (there e^-g is 0 or overflows either
//    way) and keeps t and lo finite for every g;
//  - the quotient from the hardware reciprocal refined by one Newton step,
//    with the divisor scaled by 2^-64 above 2^64 (the reciprocal flushes
//    results below 2^-126 to zero, though g / d is still a normal number up
//    to d near 2^128), skipped where 1 + e^-g overflowed (g below about
//    -88.7: silu -0, as g / inf) or the quotient is infinite; silu has the
//    sign of g, which also keeps -0 for g = -0.
// Every SwiGLU path (lf_swiglu and the fused decode and prefill epilogues)
// uses this one function, so a fused activation and the linear followed by
// lf_swiglu give identical bits.
__device__ __forceinline__ float silu_times(float g, float u) {
  constexpr float kNegLog2eHi = -1.44269502162933349609375f;    // -log2(e) rounded to fp32
  constexpr float kNegLog2eLo = -1.925963033500011079e-08f;      // -log2(e) - kNegLog2eHi
  constexpr float kLn2 = 0.693147180559945309f;
  const float c = __builtin_fminf(__builtin_fmaxf(g, -126.0f), 126.0f);
  const float t = c * kNegLog2eHi;
  const float lo = fmaf(c, kNegLog2eLo, fmaf(c, kNegLog2eHi, -t));
  const float e = __builtin_amdgcn_exp2f(t) * fmaf(lo, kLn2, 1.0f);
  const float d = 1.0f + e;
  const float sc = d > 0x1p64f ? 0x1p-64f : 1.0f;
  const float ds = d * sc;
  const float r = __builtin_amdgcn_rcpf(ds);
  const float q = g * r;  // g / d / sc
  const bool refine = d < __builtin_huge_valf() && __builtin_fabsf(q) < __builtin_huge_valf();
  const float act = __builtin_copysignf((refine ? fmaf(fmaf(-q, ds, g), r, q) : q) * sc, g);
  return round_bf16(act) * u;
}

// One 16x16x32 bf16 MFMA step: acc[i = 4*(lane/16) + r][j = lane%16] +=
// sum_k a[i][k] * b[k][j], where lane l supplies a[l%16][8*(l/16) .. +8)
// and b[8*(l/16) .. +8)[l%16].
__device__ __forceinline__ f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& acc) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
}

// One 32x32x16 bf16 MFMA step (layout checked on gfx950 against a CPU matmul):
// lane l supplies a[l%32][8*(l/32) .. +8] and b[8*(l/32) .. +8][l%32];
// acc[r] of lane l is c[8*(r/4) + 4*(l/32) + r%4][l%32].
__device__ __forceinline__ f32x16 mfma32(const bf16x8& a, const bf16x8& b, const f32x16& acc) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4& v) { return __builtin_bit_cast(bf16x8, v); }

// Wave-wide fp32 sum (wave64) through cross-lane shuffles.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d, 64);
  return v;
}

}  // namespace lf
