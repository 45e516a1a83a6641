// SwiGLU step between the gate/up and down projections of an MLP:
// h[t, c] = bf16(bf16(silu(g)) * u) with g = gate_up[t, c], u = gate_up[t, n + c]
// (the merged gate/up output of one fused call with two slices).
// Reference: benchmarks/qwen35_decode_silu.py:60-61 (the activation after the
// two LoRA adds) and benchmarks/qwen35_prefill_fused.py:14-93 (the same
// chain at prefill). HBM-bound elementwise work: 4 bytes read and 2 written
// per output; 16-byte accesses when rows and strides allow.
#include "common.h"

namespace lf {
namespace {

constexpr int kSwigluThreads = 256;


// Eight outputs per thread: rows split into n / 8 chunks of 16 bytes.
__global__ __launch_bounds__(kSwigluThreads) void swiglu_vec_kernel(const uint16_t* gu, int64_t rows, int64_t n,
                                                                  int64_t in_stride, uint16_t* out,
                                                                  int64_t out_stride) {
  const int64_t chunks = n >> 3;
  const int64_t total = rows * chunks;
  for (int64_t i = int64_t(blockIdx.x) * kSwigluThreads + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * kSwigluThreads) {
    const int64_t r = i / chunks;
    const int64_t c = (i - r * chunks) << 3;
    const uint4 g = *reinterpret_cast<const uint4*>(gu + r * in_stride + c);
    const uint4 u = *reinterpret_cast<const uint4*>(gu + r * in_stride + n + c);
    const uint32_t gw[4] = {g.x, g.y, g.z, g.w};
    const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k)
      o[k] = pack_bf16x2(silu_times(bf16_lo(gw[k]), bf16_lo(uw[k])), silu_times(bf16_hi(gw[k]), bf16_hi(uw[k])));
    *reinterpret_cast<uint4*>(out + r * out_stride + c) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

__global__ __launch_bounds__(kSwigluThreads) void swiglu_scalar_kernel(const uint16_t* gu, int64_t rows, int64_t n,
                                                                     int64_t in_stride, uint16_t* out,
                                                                     int64_t out_stride) {
  const int64_t total = rows * n;
  for (int64_t i = int64_t(blockIdx.x) * kSwigluThreads + threadIdx.x; i < total;
       i += int64_t(gridDim.x) * kSwigluThreads) {
    const int64_t r = i / n;
    const int64_t c = i - r * n;
    const float g = bf16_to_f32(gu[r * in_stride + c]);
    const float u = bf16_to_f32(gu[r * in_stride + n + c]);
    out[r * out_stride + c] = uint16_t(pack_bf16x2(silu_times(g, u), 0.f) & 0xffffu);
  }
}

}  // namespace
}  // namespace lf

extern "C" int lf_swiglu(const uint16_t* gate_up, int64_t rows, int64_t n, int64_t in_stride, uint16_t* out,
                         int64_t out_stride, void* stream) {
  LF_REQUIRE(gate_up != nullptr && out != nullptr, "null pointer argument");
  LF_REQUIRE(rows >= 0 && n > 0, "rows must be non-negative and n positive");
  LF_REQUIRE(in_stride >= 2 * n && out_stride >= n, "row strides must cover 2 * n inputs and n outputs");
  if (rows == 0) return lf::kOk;
  const bool vec = n % 8 == 0 && in_stride % 8 == 0 && out_stride % 8 == 0 && lf::aligned16(gate_up) &&
                   lf::aligned16(out);
  const int64_t items = vec ? rows * (n / 8) : rows * n;
  const int64_t want = (items + lf::kSwigluThreads - 1) / lf::kSwigluThreads;
  const unsigned grid = unsigned(want < 8192 ? want : 8192);
  auto s = static_cast<hipStream_t>(stream);
  if (vec)
    hipLaunchKernelGGL(lf::swiglu_vec_kernel, dim3(grid), dim3(lf::kSwigluThreads), 0, s, gate_up, rows, n,
                       in_stride, out, out_stride);
  else
    hipLaunchKernelGGL(lf::swiglu_scalar_kernel, dim3(grid), dim3(lf::kSwigluThreads), 0, s, gate_up, rows, n,
                       in_stride, out, out_stride);
  LF_HIP(hipGetLastError());
  return lf::kOk;
}
