// Retained-rank LoRA row operators for gfx950.
//
// row_shrink (reference ops/csrc/lora_rows.cu:35-65): for token t with slot
//   g = slots[t] >= 0 and rank r = ranks[g] > 0, for slice s < S, k < r:
//   z[t, s*r + k] = bf16(sum_w x[t, w] * A[g, s*r + k, w]).
// row_expand (lora_rows.cu:67-162): for each active segment (one slot, at most
//   16 tokens) and column n of slice s:
//   y[t, n] = bf16(bf16(y[t, n]) + bf16(scale[g] * sum_{k<r} z[t, s*r+k] * B_g[n, k]))
//   with B_g = [N, b_strides[g]] at element b_offsets[g] of the flat store.
//
// Shrink: one wave per 4 output columns of one token; the x chunk each lane
// reads (8 bf16, one 128-bit load) is reused for the 4 A rows, and the fp32
// partial sums are combined with a wave64 butterfly.
// Expand: a persistent grid walks (segment, column block) items; the segment's
// z values are staged in LDS once, each thread keeps its B row in registers
// and updates every token of the segment.
#include "common.h"
#include "../../include/loraforge_amd.h"

namespace lf {
namespace {

constexpr int kShrinkThreads = 256;
constexpr int kShrinkWaves = kShrinkThreads / 64;
constexpr int kColsPerWave = 4;
constexpr int kMaxSegment = 16;
constexpr int kMaxRank = 64;
constexpr int kMaxSlices = 4;

__device__ __forceinline__ float dot8(const uint4& a, const uint4& x, float acc) {
  acc = __builtin_fmaf(bf16_lo(a.x), bf16_lo(x.x), acc);
  acc = __builtin_fmaf(bf16_hi(a.x), bf16_hi(x.x), acc);
  acc = __builtin_fmaf(bf16_lo(a.y), bf16_lo(x.y), acc);
  acc = __builtin_fmaf(bf16_hi(a.y), bf16_hi(x.y), acc);
  acc = __builtin_fmaf(bf16_lo(a.z), bf16_lo(x.z), acc);
  acc = __builtin_fmaf(bf16_hi(a.z), bf16_hi(x.z), acc);
  acc = __builtin_fmaf(bf16_lo(a.w), bf16_lo(x.w), acc);
  acc = __builtin_fmaf(bf16_hi(a.w), bf16_hi(x.w), acc);
  return acc;
}

__global__ __launch_bounds__(kShrinkThreads) void row_shrink_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ a, uint16_t* __restrict__ z,
    const int32_t* __restrict__ slots, const int32_t* __restrict__ ranks, int width, int64_t x_stride,
    int slices, int capacity, int max_rank) {
  const int t = blockIdx.x;
  const int g = slots[t];
  if (g < 0) return;
  const int r = ranks[g];
  if (r <= 0) return;
  const int lane = threadIdx.x & 63;
  const int first = (blockIdx.y * kShrinkWaves + (threadIdx.x >> 6)) * kColsPerWave;
  // Work item j covers slice j / max_rank, row j % max_rank (live when < r).
  int rows[kColsPerWave];
  int live = 0;
#pragma unroll
  for (int c = 0; c < kColsPerWave; ++c) {
    const int j = first + c;
    const int s = j / max_rank;
    const int k = j - s * max_rank;
    const bool ok = s < slices && k < r;
    rows[c] = ok ? s * r + k : -1;
    live += ok;
  }
  if (!live) return;
  const uint16_t* xp = x + int64_t(t) * x_stride;
  const uint16_t* ap = a + int64_t(g) * slices * capacity * int64_t(width);
  float acc[kColsPerWave] = {0.f, 0.f, 0.f, 0.f};
  for (int w = lane * 8; w < width; w += 64 * 8) {
    const uint4 xv = *reinterpret_cast<const uint4*>(xp + w);
#pragma unroll
    for (int c = 0; c < kColsPerWave; ++c) {
      if (rows[c] >= 0) {
        const uint4 av = *reinterpret_cast<const uint4*>(ap + int64_t(rows[c]) * width + w);
        acc[c] = dot8(av, xv, acc[c]);
      }
    }
  }
  const int64_t zrow = int64_t(t) * slices * capacity;
#pragma unroll
  for (int c = 0; c < kColsPerWave; ++c) {
    if (rows[c] >= 0) {
      const float total = wave_sum(acc[c]);
      if (lane == 0) z[zrow + rows[c]] = uint16_t(f32_to_bf16(total));
    }
  }
}

struct ExpandArgs {
  const uint16_t* z;
  const uint16_t* b;
  const int64_t* b_offsets;
  const int32_t* b_strides;
  uint16_t* y;
  const int32_t* indptr;
  const int32_t* seg_slots;
  const int32_t* token_indices;
  const int32_t* ranks;
  const float* scales;
  const int32_t* slice_offsets;
  const int32_t* segment_count;
  int n;          // output columns
  int slices;
  int capacity;   // z row = slices * capacity
  int64_t y_stride;
};

template <int BR>
__device__ __forceinline__ void load_b_row(const uint16_t* bp, float (&b)[BR]) {
  if constexpr (BR >= 8) {
#pragma unroll
    for (int q = 0; q < BR; q += 8) {
      const uint4 v = *reinterpret_cast<const uint4*>(bp + q);
      b[q + 0] = bf16_lo(v.x); b[q + 1] = bf16_hi(v.x);
      b[q + 2] = bf16_lo(v.y); b[q + 3] = bf16_hi(v.y);
      b[q + 4] = bf16_lo(v.z); b[q + 5] = bf16_hi(v.z);
      b[q + 6] = bf16_lo(v.w); b[q + 7] = bf16_hi(v.w);
    }
  } else if constexpr (BR == 4) {
    const uint2 v = *reinterpret_cast<const uint2*>(bp);
    b[0] = bf16_lo(v.x); b[1] = bf16_hi(v.x); b[2] = bf16_lo(v.y); b[3] = bf16_hi(v.y);
  } else if constexpr (BR == 2) {
    const uint32_t v = *reinterpret_cast<const uint32_t*>(bp);
    b[0] = bf16_lo(v); b[1] = bf16_hi(v);
  } else {
    b[0] = bf16_to_f32(bp[0]);
  }
}

// zs layout: [token][slice][64] fp32, zero-padded past the rank.
template <int BR>
__device__ __forceinline__ void expand_columns(const ExpandArgs& p, int col, int count, int rank, int slot,
                                               const int* rows, const float* zs) {
  if (col >= p.n) return;
  int s = 0;
  for (int i = 1; i < p.slices; ++i) s += col >= p.slice_offsets[i];
  float b[BR];
  load_b_row<BR>(p.b + p.b_offsets[slot] + int64_t(col) * BR, b);
  const float scale = p.scales[slot];
  for (int t = 0; t < count; ++t) {
    const float* zt = zs + (t * kMaxSlices + s) * kMaxRank;
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < BR; ++k) acc = __builtin_fmaf(zt[k], b[k], acc);
    uint16_t* yp = p.y + int64_t(rows[t]) * p.y_stride + col;
    const float delta = round_bf16(acc * scale);
    *yp = uint16_t(f32_to_bf16(bf16_to_f32(*yp) + delta));
  }
}

__global__ void row_expand_kernel(ExpandArgs p) {
  __shared__ int rows[kMaxSegment];
  __shared__ float zs[kMaxSegment * kMaxSlices * kMaxRank];
  const int column_blocks = (p.n + blockDim.x - 1) / blockDim.x;
  const int items = *p.segment_count * column_blocks;
  const int zrow = p.slices * p.capacity;
  for (int item = blockIdx.x; item < items; item += gridDim.x) {
    const int seg = item / column_blocks;
    const int cb = item - seg * column_blocks;
    const int begin = p.indptr[seg];
    const int count = p.indptr[seg + 1] - begin;
    const int slot = p.seg_slots[seg];
    if (slot < 0 || count <= 0) continue;
    const int rank = p.ranks[slot];
    // Metadata contract: at most 16 tokens per segment and rank <= 64.
    if (rank <= 0 || rank > kMaxRank || count > kMaxSegment) continue;
    const int br = p.b_strides[slot];
    if (threadIdx.x < kMaxSegment) rows[threadIdx.x] = threadIdx.x < count ? p.token_indices[begin + threadIdx.x] : 0;
    __syncthreads();
    for (int i = threadIdx.x; i < count * p.slices * br; i += blockDim.x) {
      const int t = i / (p.slices * br);
      const int rem = i - t * p.slices * br;
      const int s = rem / br;
      const int k = rem - s * br;
      zs[(t * kMaxSlices + s) * kMaxRank + k] =
          k < rank ? bf16_to_f32(p.z[int64_t(rows[t]) * zrow + s * rank + k]) : 0.f;
    }
    __syncthreads();
    const int col = cb * blockDim.x + threadIdx.x;
    switch (br) {
      case 1: expand_columns<1>(p, col, count, rank, slot, rows, zs); break;
      case 2: expand_columns<2>(p, col, count, rank, slot, rows, zs); break;
      case 4: expand_columns<4>(p, col, count, rank, slot, rows, zs); break;
      case 8: expand_columns<8>(p, col, count, rank, slot, rows, zs); break;
      case 16: expand_columns<16>(p, col, count, rank, slot, rows, zs); break;
      case 32: expand_columns<32>(p, col, count, rank, slot, rows, zs); break;
      case 64: expand_columns<64>(p, col, count, rank, slot, rows, zs); break;
      default: break;  // b_strides must be a power of two in 1..64
    }
    __syncthreads();
  }
}

}  // namespace
}  // namespace lf

extern "C" int lf_row_shrink(const uint16_t* x, const uint16_t* a, uint16_t* z, const int32_t* slots,
                             const int32_t* ranks, int64_t tokens, int64_t width, int64_t x_stride,
                             int32_t num_slices, int64_t capacity, int32_t max_rank, void* stream) {
  LF_REQUIRE(tokens >= 0 && tokens < (int64_t(1) << 31), "tokens out of range");
  if (tokens == 0) return lf::kOk;
  LF_REQUIRE(x && a && z && slots && ranks, "null pointer argument");
  LF_REQUIRE(num_slices >= 1 && num_slices <= lf::kMaxSlices, "num_slices must be in 1..4");
  LF_REQUIRE(max_rank >= 1 && max_rank <= 64 && capacity >= max_rank, "max_rank must be in 1..64 and <= capacity");
  LF_REQUIRE(width > 0 && width % 8 == 0 && x_stride >= width && x_stride % 8 == 0 && width < (int64_t(1) << 31),
             "x width and row stride must be multiples of 8");
  LF_REQUIRE(lf::aligned16(x) && lf::aligned16(a), "x and A must be 16-byte aligned");
  const int64_t work = int64_t(num_slices) * max_rank;
  const int64_t per_block = lf::kShrinkWaves * lf::kColsPerWave;
  dim3 grid(unsigned(tokens), unsigned((work + per_block - 1) / per_block));
  hipLaunchKernelGGL(lf::row_shrink_kernel, grid, dim3(lf::kShrinkThreads), 0, static_cast<hipStream_t>(stream), x,
                     a, z, slots, ranks, int(width), x_stride, int(num_slices), int(capacity), int(max_rank));
  LF_HIP(hipGetLastError());
  return lf::kOk;
}

extern "C" int lf_row_expand(const uint16_t* z, const uint16_t* b, const int64_t* b_offsets,
                             const int32_t* b_strides, uint16_t* y, const int32_t* segment_indptr,
                             const int32_t* segment_slots, const int32_t* token_indices, const int32_t* ranks,
                             const float* scales, const int32_t* slice_offsets, const int32_t* segment_count,
                             int64_t tokens, int64_t out_width, int64_t y_stride, int32_t num_slices,
                             int64_t capacity, int32_t blocks, int32_t threads, void* stream) {
  LF_REQUIRE(tokens >= 0 && tokens < (int64_t(1) << 31), "tokens out of range");
  if (tokens == 0) return lf::kOk;
  LF_REQUIRE(z && b && b_offsets && b_strides && y && segment_indptr && segment_slots && token_indices && ranks &&
                 scales && slice_offsets && segment_count,
             "null pointer argument");
  LF_REQUIRE(num_slices >= 1 && num_slices <= lf::kMaxSlices, "num_slices must be in 1..4");
  LF_REQUIRE(out_width > 0 && out_width < (int64_t(1) << 31) && y_stride >= out_width, "invalid output width/stride");
  LF_REQUIRE(capacity >= 1, "capacity must be positive");
  LF_REQUIRE(threads == 128 || threads == 256, "threads must be 128 or 256");
  LF_REQUIRE(blocks >= 1 && blocks <= 65535, "blocks must be in 1..65535");
  LF_REQUIRE(lf::aligned16(b), "B store must be 16-byte aligned");
  lf::ExpandArgs p{z, b, b_offsets, b_strides, y, segment_indptr, segment_slots, token_indices, ranks, scales,
                   slice_offsets, segment_count, int(out_width), int(num_slices), int(capacity), y_stride};
  hipLaunchKernelGGL(lf::row_expand_kernel, dim3(blocks), dim3(threads), 0, static_cast<hipStream_t>(stream), p);
  LF_HIP(hipGetLastError());
  return lf::kOk;
}
