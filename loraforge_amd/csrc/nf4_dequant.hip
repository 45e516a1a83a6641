// Standalone NF4 -> bf16 dequantisation (reference: ops/nf4.py:7-38 and
// ops/_nf4_kernels.py:44-61, the byte-pair kernel) and the double-quant scale
// reconstruction of prepare_scales (ops/nf4.py:144-147).
//
// HBM-bound: per 64-element block it reads 32 packed bytes + 4 scale bytes
// and writes 128 bytes. Each lane decodes one packed dword (8 elements) per
// step and stores 16 bytes, so every load (256 B/wave) and store (1 KiB/wave)
// instruction is fully coalesced. Two independent steps per lane (2048
// workgroups at 8192 x 1024) measured best: 6.3 us against 7.1 us with four
// and 7.2 us with one. Packed bytes at an address that is not 4-byte
// aligned, or an output that is not 16-byte aligned (a contiguous view at an
// odd offset, which the reference accepts), take the same kernel with byte
// loads and 2-byte stores.
#include "nf4_common.h"
#include "../../include/loraforge_amd.h"

namespace lf {
namespace {

constexpr int kThreads = 256;
constexpr int kSteps = 2;

// Packed dword w of the weight (bytes 4w..4w+3, little endian).
template <bool kAligned>
__device__ __forceinline__ uint32_t load_packed(const uint8_t* __restrict__ packed, int64_t w) {
  if constexpr (kAligned) {
    return reinterpret_cast<const uint32_t*>(packed)[w];
  } else {
    const uint8_t* p = packed + 4 * w;
    return uint32_t(p[0]) | (uint32_t(p[1]) << 8) | (uint32_t(p[2]) << 16) | (uint32_t(p[3]) << 24);
  }
}

// Elements 8w..8w+7 of the output.
template <bool kAligned>
__device__ __forceinline__ void store_elements(uint16_t* __restrict__ out, int64_t w, uint4 v) {
  if constexpr (kAligned) {
    reinterpret_cast<uint4*>(out)[w] = v;
  } else {
    uint16_t* p = out + 8 * w;
    const uint32_t words[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[2 * i] = uint16_t(words[i] & 0xffffu);
      p[2 * i + 1] = uint16_t(words[i] >> 16);
    }
  }
}

template <bool kDouble, bool kAligned>
__global__ __launch_bounds__(kThreads) void nf4_dequant_kernel(const uint8_t* __restrict__ packed,
                                                               ScaleSource src, const float* __restrict__ code,
                                                               uint16_t* __restrict__ out, int64_t ndwords) {
  __shared__ float table[16];
  __shared__ float code2[kDouble ? 256 : 1];
  // Packed bytes are requested first; the codebook is staged while they travel.
  const int64_t base = int64_t(blockIdx.x) * (kThreads * kSteps) + threadIdx.x;
  uint32_t words[kSteps];
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int64_t w = base + s * kThreads;
    words[s] = w < ndwords ? load_packed<kAligned>(packed, w) : 0u;
  }
  const float offset = kDouble ? *src.offset : 0.0f;
  if (threadIdx.x < 16) table[threadIdx.x] = code[threadIdx.x];
  if constexpr (kDouble) code2[threadIdx.x] = src.code2[threadIdx.x];
  __syncthreads();
#pragma unroll
  for (int s = 0; s < kSteps; ++s) {
    const int64_t w = base + s * kThreads;
    if (w < ndwords) {
      // 8 elements per dword, 64 per block: block = w / 8.
      const float scale = block_scale(src, w >> 3, code2, offset);
      store_elements<kAligned>(out, w, decode_dword(words[s], scale, table));
    }
  }
}

__global__ __launch_bounds__(kThreads) void dq_scales_kernel(ScaleSource src, float* __restrict__ scales,
                                                             int64_t nblocks) {
  __shared__ float code2[256];
  code2[threadIdx.x] = src.code2[threadIdx.x];
  __syncthreads();
  const float offset = *src.offset;
  for (int64_t j = int64_t(blockIdx.x) * kThreads + threadIdx.x; j < nblocks;
       j += int64_t(gridDim.x) * kThreads) {
    scales[j] = block_scale(src, j, code2, offset);
  }
}

int launch_dequant(const uint8_t* qweight, const ScaleSource& src, const float* code, uint16_t* out,
                   int64_t numel, void* stream) {
  LF_REQUIRE(numel > 0 && numel % (kNf4Block * kNf4Block) == 0,
             "element count must be a positive multiple of 4096");
  LF_REQUIRE(qweight && code && out, "null pointer argument");
  LF_REQUIRE((reinterpret_cast<uintptr_t>(out) & 1u) == 0, "out must be 2-byte aligned (bf16)");
  const int64_t ndwords = numel / 8;
  const int64_t grid = (ndwords + kThreads * kSteps - 1) / (kThreads * kSteps);
  LF_REQUIRE(grid < (int64_t(1) << 31), "tensor too large");
  auto s = static_cast<hipStream_t>(stream);
  const bool vec = aligned16(out) && (reinterpret_cast<uintptr_t>(qweight) & 3u) == 0;
  if (src.scales) {
    auto k = vec ? nf4_dequant_kernel<false, true> : nf4_dequant_kernel<false, false>;
    hipLaunchKernelGGL(k, dim3(grid), dim3(kThreads), 0, s, qweight, src, code, out, ndwords);
  } else {
    auto k = vec ? nf4_dequant_kernel<true, true> : nf4_dequant_kernel<true, false>;
    hipLaunchKernelGGL(k, dim3(grid), dim3(kThreads), 0, s, qweight, src, code, out, ndwords);
  }
  LF_HIP(hipGetLastError());
  return kOk;
}

}  // namespace
}  // namespace lf

extern "C" int lf_nf4_dequant(const uint8_t* qweight, const float* scales, const float* code, uint16_t* out,
                              int64_t numel, void* stream) {
  LF_REQUIRE(scales != nullptr, "scales required");
  lf::ScaleSource src{scales, nullptr, nullptr, nullptr, nullptr, 1};
  return lf::launch_dequant(qweight, src, code, out, numel, stream);
}

extern "C" int lf_nf4_dequant_dq(const uint8_t* qweight, const uint8_t* absmax_q, const float* absmax2,
                                 const float* code2, const float* offset, int64_t dq_block, const float* code,
                                 uint16_t* out, int64_t numel, void* stream) {
  LF_REQUIRE(absmax_q && absmax2 && code2 && offset, "double-quant state pointers required");
  LF_REQUIRE(dq_block > 0 && dq_block <= (int64_t(1) << 30), "dq_block must be positive");
  lf::ScaleSource src{nullptr, absmax_q, absmax2, code2, offset, int(dq_block)};
  return lf::launch_dequant(qweight, src, code, out, numel, stream);
}

extern "C" int lf_nf4_prepare_scales_dq(const uint8_t* absmax_q, const float* absmax2, const float* code2,
                                        const float* offset, int64_t dq_block, float* scales, int64_t nblocks,
                                        void* stream) {
  LF_REQUIRE(absmax_q && absmax2 && code2 && offset && scales, "null pointer argument");
  LF_REQUIRE(dq_block > 0 && dq_block <= (int64_t(1) << 30), "dq_block must be positive");
  LF_REQUIRE(nblocks > 0, "nblocks must be positive");
  lf::ScaleSource src{nullptr, absmax_q, absmax2, code2, offset, int(dq_block)};
  const int64_t want = (nblocks + lf::kThreads - 1) / lf::kThreads;
  const int grid = int(want < 4096 ? want : 4096);
  hipLaunchKernelGGL(lf::dq_scales_kernel, dim3(grid), dim3(lf::kThreads), 0, static_cast<hipStream_t>(stream),
                     src, scales, nblocks);
  LF_HIP(hipGetLastError());
  return lf::kOk;
}
