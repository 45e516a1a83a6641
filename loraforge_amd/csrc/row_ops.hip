// Retained-rank LoRA row operators for gfx950, both on MFMA.
//
// row_shrink (reference ops/csrc/lora_rows.cu:35-65, contract
// ops/lora_rows.py:51-109): for token t with slot g = slots[t] >= 0 and rank
// r = ranks[g] > 0, for slice s < S and k < r:
//   z[t, s*r + k] = bf16(sum_w x[t, w] * A[g, s*r + k, w]);
// every other z entry is left as it was.
// row_expand (lora_rows.cu:67-162, contract ops/lora_rows.py:112-239): for
// each active segment (one slot, at most 16 tokens) and column n of slice s:
//   y[t, n] = bf16(bf16(y[t, n]) + bf16(scale[g] * sum_{k<r} z[t, s*r+k] * B_g[n, k]))
// with B_g = [N, b_strides[g]] at element b_offsets[g] of the flat store.
//
// Shrink, grouped by adapter: workgroup (g, j, p) owns A rows 16j .. 16j + 15
// of slot g and every p-th group of 16 tokens routed to g (it finds them by
// scanning the slot vector, 1024 entries at a time, with wave ballots). A
// group is a 16 (A rows) x 16 (tokens) tile contracted over the whole K on
// v_mfma_f32_16x16x32_bf16: the 16 waves of the workgroup take interleaved
// 32-wide k steps, all of a wave's loads are issued before its first MFMA,
// and the 16 partial tiles are summed through LDS in a fixed order, so the
// result does not depend on timing. A of one slot is read from HBM once per
// row tile; x rows come from L2.
// Expand: items (segment, 16 * 4 * waves output columns) on a persistent
// grid. The segment's z rows are staged in LDS as bf16, zero past the rank;
// each wave contracts 16-column tiles of B_g (A operand, one 16-byte row
// fragment per lane) with the staged z (B operand) over ceil(r / 32) MFMA
// steps, so a lane ends with four consecutive columns of one token. Columns
// of a tile that fall in another slice are masked out of that slice's MFMA.
#include <algorithm>

#include "common.h"
#include "../../include/loraforge_amd.h"

namespace lf {
namespace {

constexpr int kMaxSegment = 16;
constexpr int kMaxSlices = 4;

// ------------------------------- shrink ----------------------------------
constexpr int kShrinkWaves = 16;
constexpr int kShrinkThreads = 64 * kShrinkWaves;
constexpr int kShrinkBatch = 8;  // k steps whose loads a wave issues at once

struct ShrinkArgs {
  const uint16_t* x;
  const uint16_t* a;
  uint16_t* z;
  const int32_t* slots;
  const int32_t* ranks;
  int64_t x_stride;
  int tokens;
  int width;      // K
  int slices;
  int capacity;   // A rows per slice in the padded store; z row = slices * capacity
  int max_rank;
};

// Compacts the positions t in [c0, c0 + 1024) with slots[t] == g into `list`
// in token order; returns their count (uniform).
__device__ int gather_tokens(const ShrinkArgs& p, int g, int c0, int* list, int* wave_counts) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int t = c0 + tid;
  const bool hit = t < p.tokens && p.slots[t] == g;
  const uint64_t ballot = __ballot(hit);
  const int before = __builtin_amdgcn_mbcnt_hi(uint32_t(ballot >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(ballot), 0));
  if ((tid & 63) == 0) wave_counts[wave] = __popcll(ballot);
  __syncthreads();
  int base = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kShrinkWaves; ++w) {
    const int c = wave_counts[w];
    base += w < wave ? c : 0;
    total += c;
  }
  if (hit) list[base + before] = t;
  __syncthreads();
  return total;
}

__global__ __launch_bounds__(kShrinkThreads) void row_shrink_kernel(ShrinkArgs p) {
  __shared__ int list[kShrinkThreads];
  __shared__ int wave_counts[kShrinkWaves];
  __shared__ float red[kShrinkWaves][16][17];
  const int g = blockIdx.x;
  const int r = p.ranks[g];
  const int rows = p.slices * r;
  const int j0 = blockIdx.y * 16;
  if (r <= 0 || r > p.max_rank || j0 >= rows) return;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int c = lane & 15;
  const int kg = lane >> 4;
  const int steps = (p.width + 31) >> 5;
  // This lane's A row (rows past the slot's live rows read its last row and
  // are never stored).
  const uint16_t* arow = p.a + (int64_t(g) * p.slices * p.capacity + min(j0 + c, rows - 1)) * p.width + 8 * kg;
  int group = 0;  // running index of this slot's token groups
  for (int c0 = 0; c0 < p.tokens; c0 += kShrinkThreads) {
    const int found = gather_tokens(p, g, c0, list, wave_counts);
    for (int q = 0; q * 16 < found; ++q, ++group) {
      if (group % int(gridDim.z) != int(blockIdx.z)) continue;
      const int count = min(16, found - q * 16);
      const int tok = list[q * 16 + min(c, count - 1)];
      const uint16_t* xrow = p.x + int64_t(tok) * p.x_stride + 8 * kg;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      for (int s0 = wave; s0 < steps; s0 += kShrinkWaves * kShrinkBatch) {
        uint4 av[kShrinkBatch], xv[kShrinkBatch];
#pragma unroll
        for (int i = 0; i < kShrinkBatch; ++i) {
          const int k = (s0 + i * kShrinkWaves) * 32 + 8 * kg;
          const bool in = k < p.width;  // whole 8-element groups: width % 8 == 0
          av[i] = in ? *reinterpret_cast<const uint4*>(arow + k - 8 * kg) : make_uint4(0, 0, 0, 0);
          xv[i] = in ? *reinterpret_cast<const uint4*>(xrow + k - 8 * kg) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < kShrinkBatch; ++i) acc = mfma16(as_bf16x8(av[i]), as_bf16x8(xv[i]), acc);
      }
      // acc[e] = partial z[token c][A row j0 + 4 kg + e].
#pragma unroll
      for (int e = 0; e < 4; ++e) red[wave][4 * kg + e][c] = acc[e];
      __syncthreads();
      if (tid < 256) {
        const int j = tid >> 4;  // A row within the tile
        const int t = tid & 15;  // token within the group
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < kShrinkWaves; ++w) sum += red[w][j][t];
        if (t < count && j0 + j < rows) {
          const int token = list[q * 16 + t];
          p.z[int64_t(token) * p.slices * p.capacity + j0 + j] = uint16_t(f32_to_bf16(sum));
        }
      }
      __syncthreads();
    }
  }
}

// ------------------------------- expand ----------------------------------
constexpr int kTilesPerWave = 4;
constexpr int kZPitch = 72;  // bf16 per staged z row (64 + 8: rows land on different banks)

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

// B values k .. k + 7 of one row (stride st, rank r; k a multiple of 8), zero
// at and past the rank. Rows of stride >= 8 are 16-byte aligned; a narrower
// row is one 8-, 4- or 2-byte piece (aligned: offsets are multiples of 8).
__device__ __forceinline__ uint4 b_fragment(const uint16_t* row, int st, int r, int k) {
  uint32_t v[4] = {0u, 0u, 0u, 0u};
  if (k < st) {
    if (st >= 8) {
      const uint4 q = *reinterpret_cast<const uint4*>(row + k);
      v[0] = q.x, v[1] = q.y, v[2] = q.z, v[3] = q.w;
    } else if (st == 4) {
      const uint2 q = *reinterpret_cast<const uint2*>(row);
      v[0] = q.x, v[1] = q.y;
    } else if (st == 2) {
      v[0] = *reinterpret_cast<const uint32_t*>(row);
    } else {
      v[0] = row[0];
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e)  // keep k + e < r only
    if (k + e >= r) v[e >> 1] &= (e & 1) ? 0x0000ffffu : 0xffff0000u;
  return make_uint4(v[0], v[1], v[2], v[3]);
}

template <int kWaves>
__global__ __launch_bounds__(64 * kWaves) void row_expand_kernel(ExpandArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t zs[kMaxSlices][kMaxSegment][kZPitch];
  __shared__ int tokens[kMaxSegment];
  constexpr int kCols = 16 * kTilesPerWave * kWaves;  // output columns per item
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int c = lane & 15;
  const int kg = lane >> 4;
  const int chunks = (p.n + kCols - 1) / kCols;
  const int items = *p.segment_count * chunks;
  for (int item = blockIdx.x; item < items; item += gridDim.x) {
    const int seg = item / chunks;
    const int n_base = (item - seg * chunks) * kCols;
    const int start = p.indptr[seg];
    const int count = p.indptr[seg + 1] - start;
    const int g = p.seg_slots[seg];
    if (g < 0 || count <= 0) continue;
    const int r = p.ranks[g];
    if (r <= 0 || r > 64 || count > kMaxSegment) continue;  // outside the metadata contract: untouched
    const int st = p.b_strides[g];
    const uint16_t* bg = p.b + p.b_offsets[g];
    const float scale = p.scales[g];
    const int ksteps = (r + 31) >> 5;
    // B fragments of this wave's tiles: rows n (clamped into [0, N)), k from 8 kg.
    uint4 bf[kTilesPerWave][2];
#pragma unroll
    for (int tt = 0; tt < kTilesPerWave; ++tt) {
      const int n = min(n_base + (wave * kTilesPerWave + tt) * 16 + c, p.n - 1);
      const uint16_t* row = bg + int64_t(n) * st;
#pragma unroll
      for (int h = 0; h < 2; ++h) bf[tt][h] = h < ksteps ? b_fragment(row, st, r, 32 * h + 8 * kg) : make_uint4(0, 0, 0, 0);
    }
    __syncthreads();  // the previous item is done with the staged z
    if (tid < kMaxSegment) tokens[tid] = tid < count ? p.token_indices[start + tid] : 0;
    __syncthreads();
    // Stage z[token][s*r + k] for k < 32 * ksteps, zero past r and past the
    // segment: every load of a thread is issued before the first LDS store.
    {
      constexpr int kPer = kMaxSlices * kMaxSegment * 64 / (64 * kWaves);
      const int kbits = ksteps == 1 ? 5 : 6;
      const int total = p.slices * kMaxSegment << kbits;
      const int64_t zrow = int64_t(p.slices) * p.capacity;
      uint16_t v[kPer];
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int e = tid + j * 64 * kWaves;
        const int k = e & ((1 << kbits) - 1);
        const int i = (e >> kbits) & (kMaxSegment - 1);
        const int s = e >> (kbits + 4);
        v[j] = (e < total && i < count && k < r) ? p.z[tokens[i] * zrow + s * r + k] : uint16_t(0);
      }
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int e = tid + j * 64 * kWaves;
        if (e < total) zs[e >> (kbits + 4)][(e >> kbits) & (kMaxSegment - 1)][e & ((1 << kbits) - 1)] = v[j];
      }
    }
    __syncthreads();
    const int my_token = tokens[c];
#pragma unroll
    for (int tt = 0; tt < kTilesPerWave; ++tt) {
      const int n0 = n_base + (wave * kTilesPerWave + tt) * 16;
      if (n0 >= p.n) break;
      // Slices touching columns n0 .. n0 + 15.
      int s_lo = 0;
      while (s_lo + 1 < p.slices && p.slice_offsets[s_lo + 1] <= n0) ++s_lo;
      int s_hi = s_lo;
      while (s_hi + 1 < p.slices && p.slice_offsets[s_hi + 1] < n0 + 16) ++s_hi;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      for (int s = s_lo; s <= s_hi; ++s) {
        const int n = n0 + c;  // this lane's B row
        const bool mine = n >= p.slice_offsets[s] && n < p.slice_offsets[s + 1];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if (h < ksteps) {
            const uint4 zf = *reinterpret_cast<const uint4*>(&zs[s][c][32 * h + 8 * kg]);
            const uint4 bv = mine ? bf[tt][h] : make_uint4(0, 0, 0, 0);
            acc = mfma16(as_bf16x8(bv), as_bf16x8(zf), acc);
          }
        }
      }
      // acc[e] = delta sum for column n0 + 4 kg + e of token c.
      if (c < count) {
        uint16_t* yrow = p.y + int64_t(my_token) * p.y_stride;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int n = n0 + 4 * kg + e;
          if (n < p.n) {
            const float delta = round_bf16(acc[e] * scale);
            yrow[n] = uint16_t(f32_to_bf16(bf16_to_f32(yrow[n]) + delta));
          }
        }
      }
    }
  }
}

}  // namespace
}  // namespace lf

extern "C" int lf_row_shrink(const uint16_t* x, const uint16_t* a, uint16_t* z, const int32_t* slots,
                             const int32_t* ranks, int64_t tokens, int64_t width, int64_t x_stride,
                             int64_t num_adapters, int32_t num_slices, int64_t capacity, int32_t max_rank,
                             void* stream) {
  LF_REQUIRE(tokens >= 0 && tokens < (int64_t(1) << 31), "tokens out of range");
  if (tokens == 0) return lf::kOk;
  LF_REQUIRE(x && a && z && slots && ranks, "null pointer argument");
  LF_REQUIRE(num_adapters >= 1 && num_adapters < (int64_t(1) << 31), "num_adapters out of range");
  LF_REQUIRE(num_slices >= 1 && num_slices <= lf::kMaxSlices, "num_slices must be in 1..4");
  LF_REQUIRE(max_rank >= 1 && max_rank <= 64 && capacity >= max_rank, "max_rank must be in 1..64 and <= capacity");
  LF_REQUIRE(width > 0 && width % 8 == 0 && x_stride >= width && x_stride % 8 == 0 && width < (int64_t(1) << 31),
             "x width and row stride must be multiples of 8");
  LF_REQUIRE(lf::aligned16(x) && lf::aligned16(a), "x and A must be 16-byte aligned");
  LF_REQUIRE(capacity * num_slices < (int64_t(1) << 31), "capacity out of range");
  lf::ShrinkArgs p{x, a, z, slots, ranks, x_stride, int(tokens), int(width), int(num_slices), int(capacity), int(max_rank)};
  // Row tiles cover num_slices * max_rank A rows; the token groups of a slot
  // are spread over up to `parts` workgroups so that about 512 are launched.
  const int64_t row_tiles = (int64_t(num_slices) * max_rank + 15) / 16;
  const int64_t groups = (tokens + 15) / 16;
  const int64_t parts = std::max<int64_t>(1, std::min<int64_t>(groups, 512 / std::max<int64_t>(1, num_adapters * row_tiles)));
  const dim3 grid{unsigned(num_adapters), unsigned(row_tiles), unsigned(parts)};
  hipLaunchKernelGGL(lf::row_shrink_kernel, grid, dim3(lf::kShrinkThreads), 0, static_cast<hipStream_t>(stream), p);
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
  LF_REQUIRE(capacity >= 1 && capacity * num_slices < (int64_t(1) << 31), "capacity out of range");
  LF_REQUIRE(threads == 128 || threads == 256, "threads must be 128 or 256");
  LF_REQUIRE(blocks >= 1 && blocks <= 65535, "blocks must be in 1..65535");
  LF_REQUIRE(lf::aligned16(b), "B store must be 16-byte aligned");
  lf::ExpandArgs p{z, b, b_offsets, b_strides, y, segment_indptr, segment_slots, token_indices, ranks, scales,
                   slice_offsets, segment_count, int(out_width), int(num_slices), int(capacity), y_stride};
  auto s = static_cast<hipStream_t>(stream);
  if (threads == 256)
    hipLaunchKernelGGL(lf::row_expand_kernel<4>, dim3(blocks), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(lf::row_expand_kernel<2>, dim3(blocks), dim3(128), 0, s, p);
  LF_HIP(hipGetLastError());
  return lf::kOk;
}
