// Allocation-free variant of the fused NF4 + multi-LoRA linear.
//
// lf_nf4_lora_linear takes a caller-allocated workspace. Callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc) call lf_nf4_lora_linear_noalloc instead:
// the workspace is a file-scope device array of kScratchBytes that every
// device holds from library load until the process ends. Host code never
// uses the array's name as an address: the first call on a device looks up
// that device's copy with hipGetSymbolAddress and keeps the pointer, which is
// what the kernels receive.
//
// The array is cleared once per device (a fill kernel on the first call's
// stream, which must therefore not be capturing, waited for before the
// pointer is published, so a later call on any other stream finds the array
// cleared); afterwards the kernels'
// call-epoch protocol keeps it valid (entries are tagged with the call that
// wrote them, arrival counters return to zero at the end of every call).
// Every call on a device shares that device's array and leaves its contents
// behind: calls that overlap in time on one GPU race.
#include <algorithm>
#include <mutex>

#include "nf4_common.h"
#include "../../include/loraforge_amd.h"

namespace lf {
namespace {

constexpr int64_t kScratchBytes = LF_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
static_assert(kScratchBytes % 256 == 0, "scratch size");

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_lock;
void* g_scratch_ptr[kMaxDevices] = {};

__global__ void fill_zero_kernel(uint4* dst, int64_t n16) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride) dst[i] = make_uint4(0, 0, 0, 0);
}

// This device's copy of the scratch array (looked up and cleared on the
// first call on the device, on `stream`, which is synchronised once).
int device_scratch(hipStream_t stream, void** out) {
  int dev = -1;
  LF_HIP(hipGetDevice(&dev));
  LF_REQUIRE(dev >= 0 && dev < kMaxDevices, "device index %d out of range", dev);
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (g_scratch_ptr[dev] == nullptr) {
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    LF_HIP(hipStreamIsCapturing(stream, &capture));
    LF_REQUIRE(capture == hipStreamCaptureStatusNone,
               "the first allocation-free call on a device must run outside graph capture (it clears the scratch)");
    void* ptr = nullptr;
    LF_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    LF_REQUIRE(ptr != nullptr && aligned16(ptr), "scratch symbol has no usable device address");
    hipLaunchKernelGGL(fill_zero_kernel, dim3(256), dim3(256), 0, stream, static_cast<uint4*>(ptr), kScratchBytes / 16);
    LF_HIP(hipGetLastError());
    // Calls on other streams are not ordered after this fill: finish it
    // before any call can see the pointer.
    LF_HIP(hipStreamSynchronize(stream));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return kOk;
}

}  // namespace
}  // namespace lf

extern "C" int lf_nf4_lora_linear_noalloc(const uint16_t* x, int64_t m, int64_t x_stride, const lf_nf4_weight* w,
                                          const uint16_t* bias, const lf_lora* lora, uint16_t* y, int64_t y_stride,
                                          int32_t flags, void* stream) {
  LF_REQUIRE(w != nullptr, "weight descriptor required");
  LF_REQUIRE(m >= 0, "token count out of range");
  if (m == 0) return lf::kOk;
  int64_t need =
      lf_nf4_lora_workspace_size(m, w->n, w->k, lora ? lora->num_slices : 1, lora ? lora->max_rank : 1);
  LF_REQUIRE(need >= 0, "invalid problem size");
  // A decode call with fp32 scales uses only the control header (the size
  // above also covers fp32 scales rebuilt from a nested state, which the
  // launch then checks against the scratch itself).
  if (w->scales && m <= 64) need = std::min<int64_t>(need, lf::kWorkspaceHeader);
  LF_REQUIRE(need <= lf::kScratchBytes,
             "problem needs %lld bytes of workspace; the allocation-free entry point holds %lld (use "
             "lf_nf4_lora_linear with a caller workspace)",
             (long long)need, (long long)lf::kScratchBytes);
  void* ws = nullptr;
  const int rc = lf::device_scratch(static_cast<hipStream_t>(stream), &ws);
  if (rc != lf::kOk) return rc;
  return lf_nf4_lora_linear(x, m, x_stride, w, bias, lora, y, y_stride, ws, lf::kScratchBytes, flags, stream);
}
