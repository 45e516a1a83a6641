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
// v_mfma_f32_16x16x32_bf16: the four waves of the workgroup take interleaved
// 32-wide k steps with eight steps of loads in flight each, and the partial
// tiles are summed through LDS in a fixed order, so the result does not
// depend on timing. A of one slot is read from HBM once per row tile; x rows
// come from L2. For small token counts K is also split over workgroups
// (tagged fp32 partials summed in chunk order by the last to arrive).
// Expand: items (segment, 16 * 4 * waves output columns) on a persistent
// grid. The segment's z rows are staged in LDS as bf16, zero past the rank;
// each wave contracts 16-column tiles of B_g (A operand, one 16-byte row
// fragment per lane) with the staged z (B operand) over ceil(r / 32) MFMA
// steps, so a lane ends with four consecutive columns of one token (read and
// written as one 8-byte access when y's rows are 8-byte aligned and the width
// is a multiple of 4; z values are staged 4 per 8-byte load when z's rows are
// 8-byte aligned and the slot's rank is a multiple of 4). Columns of a tile
// that fall in another slice are masked out of that slice's MFMA; the slice
// bounds are read once per workgroup.
#include <algorithm>

#include "call_epoch.h"
#include "common.h"
#include "../../include/loraforge_amd.h"

namespace lf {
namespace {

constexpr int kMaxSegment = 16;
constexpr int kMaxSlices = 4;

// ------------------------------- shrink ----------------------------------
constexpr int kShrinkWaves = 4;
constexpr int kShrinkThreads = 64 * kShrinkWaves;
constexpr int kShrinkBatch = 8;  // k steps per wave whose loads are in flight together
constexpr int kMaxChunks = 4;    // K chunks of a split shrink (the summing code is unrolled over them)

struct ShrinkArgs {
  const uint16_t* x;
  const uint16_t* a;
  uint16_t* z;
  const int32_t* slots;
  const int32_t* ranks;
  int64_t x_stride;
  int tokens;
  int width;        // K
  int slices;
  int capacity;     // A rows per slice in the padded store; z row = slices * capacity
  int max_rank;
  int adapters;     // G
  int row_tiles;    // 16-row tiles over slices * max_rank
  int chunks;       // K chunks (1: no cross-workgroup sum)
  int chunk_steps;  // 32-wide k steps per chunk
  int parts;        // workgroups sharing the token groups of one (slot, row tile, chunk)
  int group_cap;    // election counters per (slot, row tile)
  uint64_t* partials;  // [tokens][slices * max_rank][chunks]: fp32 bits | tag << 32
  uint32_t* counters;  // [adapters][row_tiles][group_cap], zero between calls
  CallEpoch ce;
  int* status;      // set to 1 when a partial had to be recomputed
  int spin_limit;
  int withhold;     // test hook: chunks >= 1 publish nothing, so the reducer recomputes them
};

__device__ __forceinline__ void tagged_store(uint64_t* p, float v, uint32_t tag) {
  __hip_atomic_store(p, (uint64_t(tag) << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t tagged_load(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Compacts the positions t in [c0, c0 + 256) with slots[t] == g into `list`
// in token order; `mine` is this thread's slot entry. Returns the count.
__device__ int gather_tokens(int g, int c0, int tokens, int entry, int* list, int* wave_counts) {
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const bool hit = c0 + tid < tokens && entry == g;
  const uint64_t ballot = __ballot(hit);
  const int before = __builtin_amdgcn_mbcnt_hi(uint32_t(ballot >> 32), __builtin_amdgcn_mbcnt_lo(uint32_t(ballot), 0));
  if ((tid & 63) == 0) wave_counts[wave] = __popcll(ballot);
  __syncthreads();
  int base = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kShrinkWaves; ++w) {
    const int n = wave_counts[w];
    base += w < wave ? n : 0;
    total += n;
  }
  if (hit) list[base + before] = c0 + tid;
  __syncthreads();
  return total;
}

// sum_k x[token][k] * A-row[k] over the 32-wide steps [s0, s1) (the reducer's
// fallback for a partial that never arrived).
__device__ float chunk_dot(const uint16_t* xrow, const uint16_t* arow, int s0, int s1, int width) {
  float acc = 0.f;
  for (int k = s0 * 32; k < min(s1 * 32, width); k += 8) {
    const uint4 xv = *reinterpret_cast<const uint4*>(xrow + k);
    const uint4 av = *reinterpret_cast<const uint4*>(arow + k);
    const uint32_t xs[4] = {xv.x, xv.y, xv.z, xv.w};
    const uint32_t as[4] = {av.x, av.y, av.z, av.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc = __builtin_fmaf(bf16_lo(xs[i]), bf16_lo(as[i]), acc);
      acc = __builtin_fmaf(bf16_hi(xs[i]), bf16_hi(as[i]), acc);
    }
  }
  return acc;
}

__global__ __launch_bounds__(kShrinkThreads) void row_shrink_kernel(ShrinkArgs p) {
  __shared__ int list[kShrinkThreads];
  __shared__ int wave_counts[kShrinkWaves];
  __shared__ float red[kShrinkWaves][16][17];
  __shared__ uint32_t arrived;
  // First round: the epoch, the slot's rank and this thread's first slot entry together.
  const int tid = threadIdx.x;
  const int r = p.ranks[blockIdx.x % p.adapters];
  int entry = p.slots[min(tid, p.tokens - 1)];
  const uint32_t tag = p.chunks > 1 ? __builtin_amdgcn_readfirstlane(epoch_tag(p.ce)) : 0u;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int c = lane & 15;
  const int kg = lane >> 4;
  // The workgroup has its tag, so it counts itself in now; the count comes back
  // while it works and is looked at only at its end (no wait there).
  uint32_t departed = 0;
  if (p.chunks > 1 && wave == 0) departed = depart_issue(p.ce, lane);
  int b = blockIdx.x;
  const int g = b % p.adapters;
  b /= p.adapters;
  const int kc = b % p.chunks;
  b /= p.chunks;
  const int jt = b % p.row_tiles;
  const int part = b / p.row_tiles;
  if (tid >= p.tokens) entry = -1;
  const int rows = p.slices * r;
  const int j0 = jt * 16;
  const int zw = p.slices * p.max_rank;
  const int steps = (p.width + 31) >> 5;
  const int s_begin = kc * p.chunk_steps;
  const int s_end = min(s_begin + p.chunk_steps, steps);
  if (r > 0 && r <= p.max_rank && j0 < rows) {
    const uint16_t* arow = p.a + (int64_t(g) * p.slices * p.capacity + min(j0 + c, rows - 1)) * p.width + 8 * kg;
    int group = 0;  // running index of this slot's token groups
    for (int c0 = 0; c0 < p.tokens; c0 += kShrinkThreads) {
      if (c0 > 0) {
        entry = p.slots[min(c0 + tid, p.tokens - 1)];
        if (c0 + tid >= p.tokens) entry = -1;
      }
      const int found = gather_tokens(g, c0, p.tokens, entry, list, wave_counts);
      for (int q = 0; q * 16 < found; ++q, ++group) {
        if (group % p.parts != part) continue;
        const int count = min(16, found - q * 16);
        const uint16_t* xrow = p.x + int64_t(list[q * 16 + min(c, count - 1)]) * p.x_stride + 8 * kg;
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int s0 = s_begin + wave; s0 < s_end; s0 += kShrinkWaves * kShrinkBatch) {
          // Every load is issued (from a clamped, readable address) before any
          // result is masked: a select on a load result waits for that load.
          uint4 av[kShrinkBatch], xv[kShrinkBatch];
#pragma unroll
          for (int i = 0; i < kShrinkBatch; ++i) {
            if (s0 + i * kShrinkWaves < s_end) {  // uniform in the wave
              const int k = min((s0 + i * kShrinkWaves) * 32, p.width - 8 - 8 * kg);
              av[i] = *reinterpret_cast<const uint4*>(arow + k);
              xv[i] = *reinterpret_cast<const uint4*>(xrow + k);
            }
          }
#pragma unroll
          for (int i = 0; i < kShrinkBatch; ++i) {
            const int st = s0 + i * kShrinkWaves;
            const bool in = st < s_end && st * 32 + 8 * kg < p.width;  // width % 8 == 0
            const uint4 zero = make_uint4(0, 0, 0, 0);
            acc = mfma16(as_bf16x8(in ? av[i] : zero), as_bf16x8(in ? xv[i] : zero), acc);
          }
        }
        // acc[e] = this wave's partial of z[token c][A row j0 + 4 kg + e].
#pragma unroll
        for (int e = 0; e < 4; ++e) red[wave][4 * kg + e][c] = acc[e];
        __syncthreads();
        const int j = tid >> 4;  // A row within the tile (tid < 256 covers the tile)
        const int t = tid & 15;  // token within the group
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < kShrinkWaves; ++w) sum += red[w][j][t];
        const bool live = t < count && j0 + j < rows;
        const int token = list[q * 16 + min(t, count - 1)];
        uint64_t* cell = p.partials + (int64_t(token) * zw + j0 + j) * p.chunks;
        if (p.chunks == 1) {
          if (live) p.z[int64_t(token) * p.slices * p.capacity + j0 + j] = uint16_t(f32_to_bf16(sum));
          __syncthreads();  // red and list are reused by the next group
          continue;
        }
        if (live && !(p.withhold && kc > 0)) tagged_store(cell + kc, sum, tag);
        __syncthreads();  // every partial of this workgroup is issued before it counts in
        uint32_t* counter = p.counters + (int64_t(g * p.row_tiles + jt) * p.group_cap + group);
        if (tid == 0) arrived = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (arrived == uint32_t(p.chunks - 1)) {
          // The last chunk to arrive sums all of them, in chunk order. The others
          // have issued their partials; a bounded wait recomputes any that does not
          // show up (flagging the status word), so the result never depends on it.
          if (live) {
            // Every chunk's partial is requested at once; only one that has not
            // arrived yet is polled.
            // (Fully unrolled with uniform guards, so `got` stays in registers.)
            uint64_t got[kMaxChunks];
#pragma unroll
            for (int k2 = 0; k2 < kMaxChunks; ++k2)
              if (k2 < p.chunks) got[k2] = tagged_load(cell + k2);
            float total = 0.f;
#pragma unroll
            for (int k2 = 0; k2 < kMaxChunks; ++k2) {
              if (k2 >= p.chunks) continue;
              float v = sum;
              if (k2 != kc) {
                uint64_t e = got[k2];
                int spins = 0;
                while (uint32_t(e >> 32) != tag && spins < p.spin_limit) {
                  __builtin_amdgcn_s_sleep(1);
                  e = tagged_load(cell + k2);
                  ++spins;
                }
                if (uint32_t(e >> 32) == tag) {
                  v = __uint_as_float(uint32_t(e));
                } else {
                  __hip_atomic_store(p.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                  const uint16_t* xr = p.x + int64_t(token) * p.x_stride;
                  const uint16_t* ar = p.a + (int64_t(g) * p.slices * p.capacity + j0 + j) * p.width;
                  v = chunk_dot(xr, ar, k2 * p.chunk_steps, min((k2 + 1) * p.chunk_steps, steps), p.width);
                }
              }
              total += v;
            }
            p.z[int64_t(token) * p.slices * p.capacity + j0 + j] = uint16_t(f32_to_bf16(total));
          }
          if (tid == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();  // red, list and `arrived` are reused by the next group
      }
    }
  }
  if (p.chunks > 1 && wave == 0) depart_finish(p.ce, departed, tag - 1, lane);
}

// ------------------------------- expand ----------------------------------
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
  int segments;   // entries of seg_slots (indptr holds one more)
  int n;          // output columns
  int slices;
  int capacity;   // z row = slices * capacity
  int64_t y_stride;
  int y_vec;      // y rows 8-byte aligned and n % 4 == 0: 4 columns per load/store
  int z_vec;      // z rows 8-byte aligned: a slot of rank % 4 == 0 stages 4 z values per load
};

// Raw B values k .. k + 7 of one row (stride st; k a multiple of 8), loaded
// unconditionally: rows of stride >= 8 are 16-byte aligned and k is clamped
// into the row; a narrower row is one 8-, 4- or 2-byte piece (aligned:
// offsets are multiples of 8), read whole. `b_mask` zeroes what is not B[k..].
__device__ __forceinline__ uint4 b_load(const uint16_t* row, int st, int k) {
  if (st >= 8) return *reinterpret_cast<const uint4*>(row + min(k, st - 8));
  if (st == 4) {
    const uint2 q = *reinterpret_cast<const uint2*>(row);
    return make_uint4(q.x, q.y, 0u, 0u);
  }
  if (st == 2) return make_uint4(*reinterpret_cast<const uint32_t*>(row), 0u, 0u, 0u);
  return make_uint4(row[0], 0u, 0u, 0u);
}

// Keeps B[k + e] for k + e < min(st, r) only.
__device__ __forceinline__ uint4 b_mask(uint4 q, int st, int r, int k) {
  uint32_t v[4] = {q.x, q.y, q.z, q.w};
  const int keep = min(st, r) - k;  // elements of this fragment that are B values below the rank
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (e >= keep) v[e >> 1] &= (e & 1) ? 0x0000ffffu : 0xffff0000u;
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// Loads are grouped into three dependent rounds per item: the segment's
// bounds and slot; the slot's metadata and the token ids; then B, z and the
// y values the tile will update, all together. Only then LDS, MFMA, stores.
template <int kWaves, int kTilesPerWave>
__global__ __launch_bounds__(64 * kWaves) void row_expand_kernel(ExpandArgs p) {
  __shared__ __attribute__((aligned(16))) uint16_t zs[kMaxSlices][kMaxSegment][kZPitch];
  constexpr int kCols = 16 * kTilesPerWave * kWaves;  // output columns per item
  constexpr int kPer = kMaxSlices * kMaxSegment * 64 / (64 * kWaves);  // staged z values per thread (max)
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int c = lane & 15;
  const int kg = lane >> 4;
  const int chunks = (p.n + kCols - 1) / kCols;
  // Slice bounds (slices + 1 of them), read once ahead of every item.
  int so[kMaxSlices + 1];
#pragma unroll
  for (int i = 0; i <= kMaxSlices; ++i) so[i] = i <= p.slices ? p.slice_offsets[i] : p.n;
  for (int item = blockIdx.x; item < p.segments * chunks; item += gridDim.x) {
    const int seg = item / chunks;
    const int n_base = (item - seg * chunks) * kCols;
    // Round 1: the live count with this segment's bounds and slot (seg < segments: readable).
    const int live = *p.segment_count;
    const int start = p.indptr[seg];
    const int count = p.indptr[seg + 1] - start;
    const int g = p.seg_slots[seg];
    if (seg >= live) break;  // items only grow
    if (g < 0 || count <= 0 || count > kMaxSegment) continue;  // nothing to do, or outside the contract
    const int r = p.ranks[g];
    const int st = p.b_strides[g];
    const int64_t boff = p.b_offsets[g];
    const float scale = p.scales[g];
    const int my_token = p.token_indices[start + min(c, count - 1)];  // lanes c >= count: a duplicate
    if (r <= 0 || r > 64) continue;
    const int ksteps = (r + 31) >> 5;
    const int kbits = ksteps == 1 ? 5 : 6;
    // Round 3, all issued before any result is used (a select on a load result
    // waits for it): B fragments, the z values to stage and the y values this
    // lane updates, each from a readable (clamped) address.
    uint4 bf[kTilesPerWave][2];
    uint16_t yv[kTilesPerWave][4];
    const uint16_t* yrow = p.y + int64_t(my_token) * p.y_stride;
#pragma unroll
    for (int tt = 0; tt < kTilesPerWave; ++tt) {
      const int n0 = n_base + (wave * kTilesPerWave + tt) * 16;
      const uint16_t* row = p.b + boff + int64_t(min(n0 + c, p.n - 1)) * st;
      bf[tt][0] = b_load(row, st, 8 * kg);
      if (ksteps > 1) bf[tt][1] = b_load(row, st, 32 + 8 * kg);
      if (p.y_vec) {
        const uint2 q = *reinterpret_cast<const uint2*>(yrow + min(n0 + 4 * kg, p.n - 4));
        yv[tt][0] = uint16_t(q.x);
        yv[tt][1] = uint16_t(q.x >> 16);
        yv[tt][2] = uint16_t(q.y);
        yv[tt][3] = uint16_t(q.y >> 16);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) yv[tt][e] = yrow[min(n0 + 4 * kg + e, p.n - 1)];
      }
    }
    const int total = p.slices * kMaxSegment << kbits;
    const int64_t zrow = int64_t(p.slices) * p.capacity;
    const bool zq_ok = p.z_vec && (r & 3) == 0;  // uniform
    uint16_t zv[kPer];
    uint2 zq[kPer / 4];
    if (zq_ok) {
#pragma unroll
      for (int j = 0; j < kPer / 4; ++j) {
        const int e = (tid + j * 64 * kWaves) * 4;  // first of four consecutive k
        const int k = e & ((1 << kbits) - 1);
        const int i = (e >> kbits) & (kMaxSegment - 1);
        const int s = e >> (kbits + 4);
        const int tok = __shfl(my_token, i, 64);  // lane i holds token i of the segment
        const bool in = e < total && k < r;
        zq[j] = *reinterpret_cast<const uint2*>(p.z + tok * zrow + (in ? s * r + k : 0));
      }
    } else {
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int e = tid + j * 64 * kWaves;
        const int k = e & ((1 << kbits) - 1);
        const int i = (e >> kbits) & (kMaxSegment - 1);
        const int s = e >> (kbits + 4);
        const int tok = __shfl(my_token, i, 64);
        const bool in = e < total && k < r;
        zv[j] = p.z[tok * zrow + (in ? s * r + k : 0)];
      }
    }
#pragma unroll
    for (int tt = 0; tt < kTilesPerWave; ++tt) {
      bf[tt][0] = b_mask(bf[tt][0], st, r, 8 * kg);
      bf[tt][1] = ksteps > 1 ? b_mask(bf[tt][1], st, r, 32 + 8 * kg) : make_uint4(0, 0, 0, 0);
    }
    __syncthreads();  // the previous item is done reading the staged z
    if (zq_ok) {
#pragma unroll
      for (int j = 0; j < kPer / 4; ++j) {
        const int e = (tid + j * 64 * kWaves) * 4;
        const int k = e & ((1 << kbits) - 1);
        const int i = (e >> kbits) & (kMaxSegment - 1);
        if (e < total)
          *reinterpret_cast<uint2*>(&zs[e >> (kbits + 4)][i][k]) = (i < count && k < r) ? zq[j] : make_uint2(0, 0);
      }
    } else {
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int e = tid + j * 64 * kWaves;
        const int k = e & ((1 << kbits) - 1);
        const int i = (e >> kbits) & (kMaxSegment - 1);
        if (e < total) zs[e >> (kbits + 4)][i][k] = (i < count && k < r) ? zv[j] : uint16_t(0);
      }
    }
    __syncthreads();
#pragma unroll
    for (int tt = 0; tt < kTilesPerWave; ++tt) {
      const int n0 = n_base + (wave * kTilesPerWave + tt) * 16;
      if (n0 >= p.n) break;
      // Slices touching columns n0 .. n0 + 15: s_lo .. s_hi.
      int s_lo = 0, s_hi = 0;
#pragma unroll
      for (int i = 1; i < kMaxSlices; ++i) {
        s_lo += (i < p.slices && so[i] <= n0) ? 1 : 0;
        s_hi += (i < p.slices && so[i] < n0 + 16) ? 1 : 0;
      }
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < kMaxSlices; ++s) {
        if (s < s_lo || s > s_hi) continue;
        const int n = n0 + c;  // this lane's B row
        const bool mine = n >= so[s] && n < so[s + 1];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if (h < ksteps) {
            const uint4 zf = *reinterpret_cast<const uint4*>(&zs[s][c][32 * h + 8 * kg]);
            acc = mfma16(as_bf16x8(mine ? bf[tt][h] : make_uint4(0, 0, 0, 0)), as_bf16x8(zf), acc);
          }
        }
      }
      // acc[e] = delta sum for column n0 + 4 kg + e of token c.
      if (c < count) {
        uint16_t* yrow = p.y + int64_t(my_token) * p.y_stride;
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = f32_to_bf16(bf16_to_f32(yv[tt][e]) + round_bf16(acc[e] * scale));
        if (p.y_vec) {
          if (n0 + 4 * kg < p.n)
            *reinterpret_cast<uint2*>(yrow + n0 + 4 * kg) = make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n0 + 4 * kg + e < p.n) yrow[n0 + 4 * kg + e] = uint16_t(o[e]);
        }
      }
    }
  }
}

}  // namespace
}  // namespace lf

namespace lf {
namespace {

constexpr int64_t kRowsHeader = 4096;  // call epoch, status word, arrival counts
constexpr int64_t kMaxCounters = 1 << 16;  // election counters, at a fixed place after the header
constexpr int kTargetGroups = 512;      // workgroups a shrink launch aims for (2 per CU)

struct ShrinkPlan {
  int row_tiles, chunks, chunk_steps, parts, group_cap;
  int64_t grid, counters_off, partials_off, bytes;
};

// Splits K across workgroups only for small token counts (decode), where one
// workgroup per (slot, row tile) would leave most CUs idle and each of them
// streaming a whole A tile. Every chunk keeps at least kMinChunkSteps 32-wide
// k steps: a finer split adds more to the partials' cross-workgroup round
// trips than it takes off each workgroup's stream, and the summing
// workgroup's gather is unrolled over kMaxChunks (c2, 64 tokens over 32
// rank-16 adapters at K = 4096, shrink + expand: up to 16 chunks 19.5 us,
// 8 chunks 16.9, 4 chunks with the gather unrolled over 16 slots 17.8 and
// over 4 slots 16.2, 2 chunks 18.5, no split 20.2).
constexpr int kMinChunkSteps = 32;

ShrinkPlan plan_shrink(int64_t tokens, int64_t width, int64_t adapters, int slices, int max_rank) {
  ShrinkPlan pl{};
  const int64_t steps = (width + 31) / 32;
  pl.row_tiles = int((int64_t(slices) * max_rank + 15) / 16);
  const int64_t active = std::max<int64_t>(1, std::min(adapters, tokens));
  const int64_t groups = (tokens + 15) / 16;
  pl.group_cap = int(groups + (tokens + kShrinkThreads - 1) / kShrinkThreads);
  int64_t chunks = 1;
  if (tokens <= 256 && adapters * pl.row_tiles * pl.group_cap <= kMaxCounters)
    while (active * pl.row_tiles * chunks * 2 <= kTargetGroups && steps >= chunks * 2 * kMinChunkSteps &&
           chunks * 2 <= kMaxChunks)
      chunks *= 2;
  pl.chunk_steps = int((steps + chunks - 1) / chunks);
  pl.chunks = int((steps + pl.chunk_steps - 1) / pl.chunk_steps);
  pl.parts = int(std::max<int64_t>(1, std::min<int64_t>(groups, kTargetGroups / (active * pl.row_tiles * pl.chunks))));
  pl.grid = adapters * pl.row_tiles * pl.chunks * pl.parts;
  if (pl.chunks > 1) {
    // Fixed places, whatever the shape: the counters are all zero between
    // calls (each is reset by the workgroup that sums its tile), so a call of
    // another shape finds zeros wherever its own counters land; partials are
    // tagged and need no clearing.
    pl.counters_off = kRowsHeader;
    pl.partials_off = kRowsHeader + kMaxCounters * 4;
    pl.bytes = pl.partials_off + tokens * slices * max_rank * int64_t(pl.chunks) * 8;
  }
  return pl;
}

}  // namespace
}  // namespace lf

extern "C" int64_t lf_row_shrink_workspace_size(int64_t tokens, int64_t width, int64_t num_adapters, int32_t num_slices,
                                                int32_t max_rank) {
  if (tokens < 0 || width <= 0 || num_adapters < 1 || num_slices < 1 || num_slices > lf::kMaxSlices || max_rank < 1 ||
      max_rank > 64)
    return -1;
  if (tokens == 0) return 0;
  return lf::plan_shrink(tokens, width, num_adapters, num_slices, max_rank).bytes;
}

extern "C" int lf_row_shrink(const uint16_t* x, const uint16_t* a, uint16_t* z, const int32_t* slots,
                             const int32_t* ranks, int64_t tokens, int64_t width, int64_t x_stride,
                             int64_t num_adapters, int32_t num_slices, int64_t capacity, int32_t max_rank,
                             void* workspace, int64_t workspace_bytes, int32_t flags, void* stream) {
  LF_REQUIRE(tokens >= 0 && tokens < (int64_t(1) << 31), "tokens out of range");
  LF_REQUIRE((flags & ~LF_TEST_WITHHOLD_PARTIALS) == 0, "unknown flags");
  if (tokens == 0) return lf::kOk;
  LF_REQUIRE(x && a && z && slots && ranks, "null pointer argument");
  LF_REQUIRE(num_adapters >= 1 && num_adapters < (int64_t(1) << 24), "num_adapters out of range");
  LF_REQUIRE(num_slices >= 1 && num_slices <= lf::kMaxSlices, "num_slices must be in 1..4");
  LF_REQUIRE(max_rank >= 1 && max_rank <= 64 && capacity >= max_rank, "max_rank must be in 1..64 and <= capacity");
  LF_REQUIRE(width > 0 && width % 8 == 0 && x_stride >= width && x_stride % 8 == 0 && width < (int64_t(1) << 31),
             "x width and row stride must be multiples of 8");
  LF_REQUIRE(lf::aligned16(x) && lf::aligned16(a), "x and A must be 16-byte aligned");
  LF_REQUIRE(capacity * num_slices < (int64_t(1) << 31), "capacity out of range");
  const lf::ShrinkPlan pl = lf::plan_shrink(tokens, width, num_adapters, num_slices, max_rank);
  LF_REQUIRE(pl.grid < (int64_t(1) << 31), "launch too large");
  if (pl.chunks > 1) {
    LF_REQUIRE(workspace && workspace_bytes >= pl.bytes, "workspace too small: need %lld bytes", (long long)pl.bytes);
    LF_REQUIRE(lf::aligned16(workspace), "workspace must be 16-byte aligned");
  }
  char* ws = static_cast<char*>(workspace);
  lf::ShrinkArgs p{x, a, z, slots, ranks, x_stride, int(tokens), int(width), int(num_slices), int(capacity),
                   int(max_rank), int(num_adapters), pl.row_tiles, pl.chunks, pl.chunk_steps, pl.parts, pl.group_cap,
                   pl.chunks > 1 ? reinterpret_cast<uint64_t*>(ws + pl.partials_off) : nullptr,
                   pl.chunks > 1 ? reinterpret_cast<uint32_t*>(ws + pl.counters_off) : nullptr,
                   pl.chunks > 1 ? lf::call_epoch_of(workspace) : lf::CallEpoch{nullptr, nullptr, nullptr},
                   pl.chunks > 1 ? reinterpret_cast<int*>(ws + lf::kStatusOffset) : nullptr,
                   (flags & LF_TEST_WITHHOLD_PARTIALS) ? 64 : (1 << 20),
                   (flags & LF_TEST_WITHHOLD_PARTIALS) ? 1 : 0};
  hipLaunchKernelGGL(lf::row_shrink_kernel, dim3(unsigned(pl.grid)), dim3(lf::kShrinkThreads), 0,
                     static_cast<hipStream_t>(stream), p);
  LF_HIP(hipGetLastError());
  return lf::kOk;
}

namespace lf {
namespace {

// The widest item (tiles of 16 columns per wave, at most max_tiles) that
// still gives one item per CU; narrower items otherwise. Narrow outputs with
// few segments are latency chains that only more workgroups shorten (C32,
// four adapters: 1024 columns 6.2 -> 4.3 us with 64-column items, QKV
// 4096/512/512 6.5 -> 4.6 us); with enough segments the wide items win
// (c2, 4096 columns: 14.4 us against 18.1 us), since every item stages its
// segment's z once.
int expand_tiles(int64_t segments, int64_t n, int waves, int max_tiles) {
  int tiles = max_tiles;
  while (tiles > 1 && segments * ((n + 16 * tiles * waves - 1) / (16 * tiles * waves)) < 256) tiles /= 2;
  return tiles;
}

int row_expand_launch(const uint16_t* z, const uint16_t* b, const int64_t* b_offsets, const int32_t* b_strides,
                      uint16_t* y, const int32_t* segment_indptr, const int32_t* segment_slots,
                      const int32_t* token_indices, const int32_t* ranks, const float* scales,
                      const int32_t* slice_offsets, const int32_t* segment_count, int64_t segments, int64_t tokens,
                      int64_t out_width, int64_t y_stride, int32_t num_slices, int64_t capacity, int32_t blocks,
                      int32_t threads, int max_tiles, void* stream) {
  LF_REQUIRE(tokens >= 0 && tokens < (int64_t(1) << 31), "tokens out of range");
  if (tokens == 0) return kOk;
  LF_REQUIRE(z && b && b_offsets && b_strides && y && segment_indptr && segment_slots && token_indices && ranks &&
                 scales && slice_offsets && segment_count,
             "null pointer argument");
  LF_REQUIRE(num_slices >= 1 && num_slices <= kMaxSlices, "num_slices must be in 1..4");
  LF_REQUIRE(out_width > 0 && out_width < (int64_t(1) << 31) && y_stride >= out_width, "invalid output width/stride");
  LF_REQUIRE(capacity >= 1 && capacity * num_slices < (int64_t(1) << 31), "capacity out of range");
  LF_REQUIRE(threads == 128 || threads == 256, "threads must be 128 or 256");
  LF_REQUIRE(blocks >= 1 && blocks <= 65535, "blocks must be in 1..65535");
  LF_REQUIRE(aligned16(b), "B store must be 16-byte aligned");
  LF_REQUIRE(segments >= 0 && segments * ((out_width + 31) / 32) < (int64_t(1) << 31), "segment work count out of range");
  if (segments == 0) return kOk;
  ExpandArgs p{z, b, b_offsets, b_strides, y, segment_indptr, segment_slots, token_indices, ranks, scales,
               slice_offsets, segment_count, int(segments), int(out_width), int(num_slices), int(capacity), y_stride,
               (out_width % 4 == 0 && y_stride % 4 == 0 && reinterpret_cast<uintptr_t>(y) % 8 == 0) ? 1 : 0,
               (capacity * num_slices % 4 == 0 && reinterpret_cast<uintptr_t>(z) % 8 == 0) ? 1 : 0};
  auto s = static_cast<hipStream_t>(stream);
  const int waves = threads / 64;
  const int tiles = expand_tiles(segments, out_width, waves, max_tiles);
  // Workgroups past the item count would only read the slice bounds and exit.
  const int64_t cols = 16 * tiles * waves;
  blocks = int32_t(std::min<int64_t>(blocks, segments * ((out_width + cols - 1) / cols)));
  if (waves == 4) {
    if (tiles == 1)
      hipLaunchKernelGGL((row_expand_kernel<4, 1>), dim3(blocks), dim3(256), 0, s, p);
    else if (tiles == 2)
      hipLaunchKernelGGL((row_expand_kernel<4, 2>), dim3(blocks), dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL((row_expand_kernel<4, 4>), dim3(blocks), dim3(256), 0, s, p);
  } else {
    if (tiles == 1)
      hipLaunchKernelGGL((row_expand_kernel<2, 1>), dim3(blocks), dim3(128), 0, s, p);
    else if (tiles == 2)
      hipLaunchKernelGGL((row_expand_kernel<2, 2>), dim3(blocks), dim3(128), 0, s, p);
    else
      hipLaunchKernelGGL((row_expand_kernel<2, 4>), dim3(blocks), dim3(128), 0, s, p);
  }
  LF_HIP(hipGetLastError());
  return kOk;
}

}  // namespace
}  // namespace lf

extern "C" int lf_row_expand(const uint16_t* z, const uint16_t* b, const int64_t* b_offsets,
                             const int32_t* b_strides, uint16_t* y, const int32_t* segment_indptr,
                             const int32_t* segment_slots, const int32_t* token_indices, const int32_t* ranks,
                             const float* scales, const int32_t* slice_offsets, const int32_t* segment_count,
                             int64_t segments, int64_t tokens, int64_t out_width, int64_t y_stride,
                             int32_t num_slices, int64_t capacity, int32_t blocks, int32_t threads, void* stream) {
  return lf::row_expand_launch(z, b, b_offsets, b_strides, y, segment_indptr, segment_slots, token_indices, ranks,
                               scales, slice_offsets, segment_count, segments, tokens, out_width, y_stride, num_slices,
                               capacity, blocks, threads, 4, stream);
}

extern "C" int lf_row_expand_tiled(const uint16_t* z, const uint16_t* b, const int64_t* b_offsets,
                                   const int32_t* b_strides, uint16_t* y, const int32_t* segment_indptr,
                                   const int32_t* segment_slots, const int32_t* token_indices, const int32_t* ranks,
                                   const float* scales, const int32_t* slice_offsets,
                                   const int32_t* segment_count, int64_t segments, int64_t tokens,
                                   int64_t out_width, int64_t y_stride, int32_t num_slices, int64_t capacity,
                                   int32_t blocks, int32_t threads, int32_t row_tile, void* stream) {
  LF_REQUIRE(row_tile == 2 || row_tile == 4 || row_tile == 8 || row_tile == 16, "row_tile must be 2, 4, 8, or 16");
  return lf::row_expand_launch(z, b, b_offsets, b_strides, y, segment_indptr, segment_slots, token_indices, ranks,
                               scales, slice_offsets, segment_count, segments, tokens, out_width, y_stride, num_slices,
                               capacity, blocks, threads, row_tile >= 16 ? 4 : row_tile == 8 ? 2 : 1, stream);
}
