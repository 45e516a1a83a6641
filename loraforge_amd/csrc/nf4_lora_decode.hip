// Fused NF4 base linear + per-token multi-LoRA for decode batches (M <= 64),
// one kernel launch per call.
//
// Reference chain being fused (all in one launch here):
//   integrations/_sglang_nf4_linear.py:116-129  y = bf16(x @ dequant(W)^T) (+bias)
//   ops/csrc/lora_rows.cu:35-65                 z = bf16(A_g @ x)
//   ops/csrc/lora_rows.cu:67-117                y = bf16(y + bf16(scale * B_g @ z))
//
// Work split (blockIdx ranges):
//   [0, nz)        shrink groups: (token, 4 A rows). Only the first token of
//                  each slot works; it contracts its 4 A rows against every
//                  token sharing that slot, so each A row is read once.
//   [nz, grid)     base groups: 16-row tiles of W. NF4 bytes are decoded in
//                  registers (codebook in LDS) to exact bf16 W values and fed
//                  to v_mfma_f32_16x16x32_bf16 with x as the A operand
//                  (tokens padded to 16) and W^T as the B operand.
//                  kRowTiles == 1: the 4 waves split K, x comes straight from
//                  L2 into registers (small batches).
//                  kRowTiles == 4: each wave owns a tile and the 4 waves share
//                  x chunks staged in LDS; K is split across groups and the
//                  last group to finish a tile reduces the fp32 partials.
//   The epilogue (bf16 round, bias, LoRA expand, bf16 rounds) runs on the
//   group that completes a tile; it waits on the shrink counter (bounded
//   spin; shrink groups have lower ids, so they are dispatched first).
//   Counters are reset by their last user, so the workspace is left zeroed.
#include "nf4_common.h"
#include "../../include/loraforge_amd.h"

namespace lf {
namespace {

constexpr int kThreads = 256;
constexpr int kChunkK = 128;       // k per chunk: 4 lane groups x 32 nibbles
constexpr int kCtrlBytes = 256;
constexpr int kSpinLimit = 1 << 22;
enum Ctrl { kZDone = 0, kTilesDone = 1, kStatus = 2 };

struct DecodeParams {
  const uint16_t* x;
  int64_t x_stride;
  int m;
  const uint8_t* q;
  ScaleSource src;
  const float* code;
  int n;
  int k;
  const uint16_t* bias;
  uint16_t* y;
  int64_t y_stride;
  // LoRA (a_store == nullptr disables it)
  const uint16_t* a_store;
  const int64_t* a_offsets;
  const uint16_t* b_store;
  const int64_t* b_offsets;
  const int32_t* b_strides;
  const int32_t* ranks;
  const float* lscales;
  const int32_t* token_slots;
  const int32_t* slice_offsets;
  int slices;
  int max_rank;
  // schedule
  int nz;        // shrink groups
  int zgroups;   // shrink groups per token
  int ksplit;    // K splits across groups
  int chunks;    // ceil(K / 128)
  int ntiles;    // N / 16
  int zw;        // z row width = slices * max_rank
  // workspace
  int* ctrl;
  int* tile_count;
  float* zbuf;
  float* part;
};

__device__ __forceinline__ int atomic_add_agent(int* p, int v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int load_acquire(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_relaxed(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

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

// ---------------------------------------------------------------------------
// Shrink group: z[t, j] = bf16(A_g[j] . x[t]) for the 4 A rows j of this group
// and every token t whose slot is g. Stored as fp32 (exact bf16 values).
// ---------------------------------------------------------------------------
__device__ void shrink_group(const DecodeParams& p, int* shared_list) {
  const int tok = blockIdx.x / p.zgroups;
  const int rg = blockIdx.x - tok * p.zgroups;
  const int g = p.token_slots[tok];
  int r = g >= 0 ? p.ranks[g] : 0;
  if (r > p.max_rank) r = 0;  // metadata contract: rank <= max_rank
  const int rows = p.slices * r;
  bool work = r > 0 && rg * 4 < rows;
  if (work && threadIdx.x == 0) {
    int count = 0;
    bool leader = true;
    for (int t = 0; t < p.m; ++t) {
      const int st = p.token_slots[t];
      if (st == g) {
        if (t < tok) { leader = false; break; }
        shared_list[count++] = t;
      }
    }
    shared_list[64] = leader ? count : 0;
  }
  __syncthreads();
  const int count = work ? shared_list[64] : 0;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int row = rg * 4 + wave;
  if (count > 0 && row < rows) {
    const uint16_t* arow = p.a_store + p.a_offsets[g] + int64_t(row) * p.k;
    for (int base = 0; base < count; base += 8) {
      const int nb = min(8, count - base);
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int kk = lane * 8; kk < p.k; kk += 512) {
        const uint4 av = *reinterpret_cast<const uint4*>(arow + kk);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if (i < nb) {
            const int t = shared_list[base + i];
            const uint4 xv = *reinterpret_cast<const uint4*>(p.x + int64_t(t) * p.x_stride + kk);
            acc[i] = dot8(av, xv, acc[i]);
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (i < nb) {
          const float total = wave_sum(acc[i]);
          if (lane == 0) p.zbuf[int64_t(shared_list[base + i]) * p.zw + row] = round_bf16(total);
        }
      }
    }
  }
  __threadfence();
  __syncthreads();
  if (threadIdx.x == 0) atomic_add_agent(p.ctrl + kZDone, 1);
}

// ---------------------------------------------------------------------------
// Base contraction helpers.
// Lane l: row n = 16*tile + (l & 15), lane group gq = l >> 4 covering
// k = 128c + 32gq .. +32 of chunk c. MFMA step j uses k = 128c + 32gq + 8j ..+8
// for both operands (the contraction order inside a chunk is a permutation).
// ---------------------------------------------------------------------------
struct WChunk {
  uint4 q;
  float scale;
};

template <bool kDouble>
__device__ __forceinline__ WChunk load_w(const DecodeParams& p, int n, int c, int gq, const float* code2_lds,
                                         float offset) {
  WChunk w;
  const int kb = c * kChunkK + gq * 32;
  if (kb < p.k) {
    w.q = *reinterpret_cast<const uint4*>(p.q + (int64_t(n) * p.k + kb) / 2);
    const int64_t block = (int64_t(n) * p.k + kb) / kNf4Block;
    if constexpr (kDouble) {
      w.scale = block_scale(p.src, block, code2_lds, offset);
    } else {
      w.scale = p.src.scales[block];
    }
  } else {
    w.q = make_uint4(0, 0, 0, 0);
    w.scale = 0.f;  // code * 0 = +/-0: contributes nothing
  }
  return w;
}

template <int TM>
__device__ __forceinline__ void mfma_chunk(const WChunk& w, const uint4 (&xf)[TM][4], f32x4 (&acc)[TM],
                                           const float* table) {
  const uint4 wd[4] = {decode_dword(w.q.x, w.scale, table), decode_dword(w.q.y, w.scale, table),
                       decode_dword(w.q.z, w.scale, table), decode_dword(w.q.w, w.scale, table)};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bf16x8 b = as_bf16x8(wd[j]);
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) acc[tm] = mfma16(as_bf16x8(xf[tm][j]), b, acc[tm]);
  }
}

// x fragment of chunk c for token group tm, straight from global memory.
template <int TM>
__device__ __forceinline__ void load_x_direct(const DecodeParams& p, int c, int lane, uint4 (&xf)[TM][4]) {
  const int gq = lane >> 4;
  const int kb = c * kChunkK + gq * 32;
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
    const int t = tm * 16 + (lane & 15);
    if (t < p.m && kb < p.k) {
      const uint4* src = reinterpret_cast<const uint4*>(p.x + int64_t(t) * p.x_stride + kb);
#pragma unroll
      for (int j = 0; j < 4; ++j) xf[tm][j] = src[j];
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) xf[tm][j] = make_uint4(0, 0, 0, 0);
    }
  }
}

// ---------------------------------------------------------------------------
// Epilogue for one 16-row tile: c_tile is [16*TM tokens][16 rows] fp32 in LDS.
// ---------------------------------------------------------------------------
template <bool kLora>
__device__ void epilogue_tile(const DecodeParams& p, int tile, const float* c_tile) {
  const int n0 = tile * 16;
  for (int idx = threadIdx.x; idx < p.m * 16; idx += kThreads) {
    const int t = idx >> 4;
    const int row = idx & 15;
    const int n = n0 + row;
    float v = round_bf16(c_tile[idx]);
    if (p.bias) v = round_bf16(v + bf16_to_f32(p.bias[n]));
    if constexpr (kLora) {
      const int g = p.token_slots[t];
      const int r = g >= 0 ? p.ranks[g] : 0;
      if (r > 0 && r <= p.max_rank) {
        int s = 0;
        for (int i = 1; i < p.slices; ++i) s += n >= p.slice_offsets[i];
        const int br = p.b_strides[g];
        const uint16_t* brow = p.b_store + p.b_offsets[g] + int64_t(n) * br;
        const float* zt = p.zbuf + int64_t(t) * p.zw + s * r;
        float acc = 0.f;
        for (int j = 0; j < r; ++j) acc = __builtin_fmaf(zt[j], bf16_to_f32(brow[j]), acc);
        v = round_bf16(v + round_bf16(acc * p.lscales[g]));
      }
    }
    p.y[int64_t(t) * p.y_stride + n] = uint16_t(f32_to_bf16(v));
  }
}

__device__ void wait_shrink(const DecodeParams& p, int* flag) {
  if (threadIdx.x == 0) {
    int spins = 0;
    while (load_acquire(p.ctrl + kZDone) < p.nz) {
      __builtin_amdgcn_s_sleep(2);
      if (++spins > kSpinLimit) {
        store_relaxed(p.ctrl + kStatus, 1);
        break;
      }
    }
    *flag = spins <= kSpinLimit;
  }
  __syncthreads();
  __threadfence();
}

__device__ void finish_tile(const DecodeParams& p) {
  // The last tile epilogue resets the shrink and tile counters.
  if (threadIdx.x == 0) {
    const int done = atomic_add_agent(p.ctrl + kTilesDone, 1);
    if (done == p.ntiles - 1) {
      store_relaxed(p.ctrl + kZDone, 0);
      store_relaxed(p.ctrl + kTilesDone, 0);
    }
  }
}

// ---------------------------------------------------------------------------
// kRowTiles == 1: one tile per group, the 4 waves split the chunks of K.
// ---------------------------------------------------------------------------
template <int TM, bool kDouble, bool kLora>
__device__ void base_split_k(const DecodeParams& p, const float* table, const float* code2, float offset,
                             float* red, int* flag) {
  const int tile = blockIdx.x - p.nz;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int gq = lane >> 4;
  const int n = tile * 16 + (lane & 15);
  const int per = (p.chunks + 3) >> 2;
  const int c0 = wave * per;
  const int c1 = min(p.chunks, c0 + per);
  f32x4 acc[TM];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) acc[tm] = (f32x4){0.f, 0.f, 0.f, 0.f};
  constexpr int kBatch = 4;
  WChunk w[kBatch];
  uint4 xf[kBatch][TM][4];
  for (int cb = c0; cb < c1; cb += kBatch) {
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      if (cb + i < c1) {
        w[i] = load_w<kDouble>(p, n, cb + i, gq, code2, offset);
        load_x_direct<TM>(p, cb + i, lane, xf[i]);
      }
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      if (cb + i < c1) mfma_chunk<TM>(w[i], xf[i], acc, table);
    }
  }
  // Cross-wave reduction: red[wave][tm][lane][4].
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
    *reinterpret_cast<f32x4*>(red + ((wave * TM + tm) * 64 + lane) * 4) = acc[tm];
  __syncthreads();
  // c_tile[token][row], token = 16*tm + 4*(l>>4) + e, row = l & 15.
  float* c_tile = red + 4 * TM * 256;
  for (int i = threadIdx.x; i < TM * 256; i += kThreads) {
    const int tm = i >> 8;
    const int l = (i >> 2) & 63;
    const int e = i & 3;
    float s = 0.f;
#pragma unroll
    for (int wv = 0; wv < 4; ++wv) s += red[((wv * TM + tm) * 64 + l) * 4 + e];
    const int token = tm * 16 + 4 * (l >> 4) + e;
    c_tile[token * 16 + (l & 15)] = s;
  }
  __syncthreads();
  if constexpr (kLora) wait_shrink(p, flag);
  epilogue_tile<kLora>(p, tile, c_tile);
  if constexpr (kLora) finish_tile(p);
}

// ---------------------------------------------------------------------------
// kRowTiles == 4: each wave owns one tile; x chunks staged in LDS in MFMA
// fragment order ([chunk][tm][step][lane] x 16 B, conflict-free reads).
// ---------------------------------------------------------------------------
template <int TM>
__device__ __forceinline__ void stage_x(const DecodeParams& p, int c, uint4* xs) {
  // 16 pieces of 16 B per token row per chunk; pieces for padded tokens are zero.
  for (int i = threadIdx.x; i < TM * 16 * 16; i += kThreads) {
    const int t = i >> 4;
    const int qd = i & 15;
    const int kb = c * kChunkK + qd * 8;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (t < p.m && kb < p.k) v = *reinterpret_cast<const uint4*>(p.x + int64_t(t) * p.x_stride + kb);
    const int tm = t >> 4;
    const int j = qd & 3;
    const int lane = (t & 15) + 16 * (qd >> 2);
    xs[(tm * 4 + j) * 64 + lane] = v;
  }
}

template <int TM, bool kDouble, bool kLora>
__device__ void base_split_rows(const DecodeParams& p, const float* table, const float* code2, float offset,
                                uint4* xs, float* c_tiles, int* flag) {
  const int grp_split = blockIdx.x - p.nz;
  const int grp = grp_split / p.ksplit;
  const int split = grp_split - grp * p.ksplit;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int gq = lane >> 4;
  const int tile = grp * 4 + wave;
  const int n = tile * 16 + (lane & 15);
  const int per = (p.chunks + p.ksplit - 1) / p.ksplit;
  const int c0 = split * per;
  const int c1 = min(p.chunks, c0 + per);
  f32x4 acc[TM];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) acc[tm] = (f32x4){0.f, 0.f, 0.f, 0.f};
  WChunk w_next = c0 < c1 ? load_w<kDouble>(p, n, c0, gq, code2, offset) : WChunk{};
  for (int c = c0; c < c1; ++c) {
    const WChunk w = w_next;
    __syncthreads();  // previous chunk's x fragments are consumed
    stage_x<TM>(p, c, xs);
    if (c + 1 < c1) w_next = load_w<kDouble>(p, n, c + 1, gq, code2, offset);
    __syncthreads();
    uint4 xf[TM][4];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int j = 0; j < 4; ++j) xf[tm][j] = xs[(tm * 4 + j) * 64 + lane];
    mfma_chunk<TM>(w, xf, acc, table);
  }
  // Each wave writes its tile as c_tiles[wave][token][row].
  float* mine = c_tiles + wave * (TM * 256);
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int e = 0; e < 4; ++e) mine[(tm * 16 + 4 * gq + e) * 16 + (lane & 15)] = acc[tm][e];
  __syncthreads();
  const int tile_elems = 4 * TM * 256;
  if (p.ksplit > 1) {
    // Publish this split's partial tiles, then let the last split reduce.
    float* mypart = p.part + (int64_t(grp) * p.ksplit + split) * tile_elems;
    for (int i = threadIdx.x; i < tile_elems; i += kThreads) mypart[i] = c_tiles[i];
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
      const int prev = atomic_add_agent(p.tile_count + grp, 1);
      const bool last = prev == p.ksplit - 1;
      if (last) store_relaxed(p.tile_count + grp, 0);
      *flag = last;
    }
    __syncthreads();
    if (!*flag) return;
    __threadfence();
    const float* parts = p.part + int64_t(grp) * p.ksplit * tile_elems;
    for (int i = threadIdx.x; i < tile_elems; i += kThreads) {
      float s = 0.f;
      for (int sp = 0; sp < p.ksplit; ++sp) s += parts[int64_t(sp) * tile_elems + i];
      c_tiles[i] = s;
    }
    __syncthreads();
  }
  if constexpr (kLora) wait_shrink(p, flag);
  for (int t = 0; t < 4; ++t) epilogue_tile<kLora>(p, grp * 4 + t, c_tiles + t * TM * 256);
  if constexpr (kLora) {
    if (threadIdx.x == 0) {
      const int done = atomic_add_agent(p.ctrl + kTilesDone, 4);
      if (done == p.ntiles - 4) {
        store_relaxed(p.ctrl + kZDone, 0);
        store_relaxed(p.ctrl + kTilesDone, 0);
      }
    }
  }
}

template <int TM, int kRowTiles, bool kDouble, bool kLora>
__global__ __launch_bounds__(kThreads) void nf4_lora_decode_kernel(DecodeParams p) {
  __shared__ float table[16];
  __shared__ float code2[kDouble ? 256 : 1];
  __shared__ int flag[72];
  constexpr int kRed = kRowTiles == 1 ? (4 * TM * 256 + TM * 256) : 1;
  constexpr int kXs = kRowTiles == 4 ? TM * 4 * 64 : 1;
  constexpr int kCt = kRowTiles == 4 ? 4 * TM * 256 : 1;
  __shared__ float red[kRed];
  __shared__ uint4 xs[kXs];
  __shared__ float c_tiles[kCt];
  if constexpr (kLora) {
    if (int(blockIdx.x) < p.nz) {
      shrink_group(p, flag);
      return;
    }
  }
  if (threadIdx.x < 16) table[threadIdx.x] = p.code[threadIdx.x];
  if constexpr (kDouble) code2[threadIdx.x] = p.src.code2[threadIdx.x];
  __syncthreads();
  const float offset = kDouble ? *p.src.offset : 0.f;
  if constexpr (kRowTiles == 1) {
    base_split_k<TM, kDouble, kLora>(p, table, code2, offset, red, flag);
  } else {
    base_split_rows<TM, kDouble, kLora>(p, table, code2, offset, xs, c_tiles, flag);
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
struct Plan {
  int tm;
  int row_tiles;
  int ksplit;
  int chunks;
  int groups;
};

Plan make_plan(int64_t m, int64_t n, int64_t k) {
  Plan pl;
  pl.tm = int((m + 15) / 16);
  pl.chunks = int((k + kChunkK - 1) / kChunkK);
  if (pl.tm == 1) {
    pl.row_tiles = 1;
    pl.ksplit = 1;
  } else {
    pl.row_tiles = 4;
    // Enough groups to cover every CU at least once (256 on MI355X).
    const int64_t row_groups = n / 64;
    int ks = 1;
    while (row_groups * ks < 256 && ks * 2 <= pl.chunks) ks *= 2;
    pl.ksplit = ks;
  }
  pl.groups = int(pl.row_tiles == 1 ? n / 16 : (n / 64) * pl.ksplit);
  return pl;
}

int64_t align256(int64_t v) { return (v + 255) / 256 * 256; }

struct Layout {
  int64_t tile_count;
  int64_t zbuf;
  int64_t part;
  int64_t total;
};

Layout workspace_layout(int64_t m, int64_t n, int64_t k, int slices, int max_rank) {
  const Plan pl = make_plan(m, n, k);
  Layout l;
  l.tile_count = kCtrlBytes;
  l.zbuf = align256(l.tile_count + 4 * (n / 64 + 1));
  l.part = align256(l.zbuf + 4 * m * int64_t(slices) * max_rank);
  int64_t part_bytes = 0;
  if (pl.row_tiles == 4 && pl.ksplit > 1) part_bytes = int64_t(n / 64) * pl.ksplit * 4 * pl.tm * 256 * 4;
  l.total = align256(l.part + part_bytes);
  return l;
}

template <int TM, int RT, bool D>
void launch_lora_variant(bool lora, dim3 grid, hipStream_t s, const DecodeParams& p) {
  if (lora) {
    hipLaunchKernelGGL((nf4_lora_decode_kernel<TM, RT, D, true>), grid, dim3(kThreads), 0, s, p);
  } else {
    hipLaunchKernelGGL((nf4_lora_decode_kernel<TM, RT, D, false>), grid, dim3(kThreads), 0, s, p);
  }
}

template <int TM, int RT>
void launch_dq_variant(bool dq, bool lora, dim3 grid, hipStream_t s, const DecodeParams& p) {
  if (dq) launch_lora_variant<TM, RT, true>(lora, grid, s, p);
  else launch_lora_variant<TM, RT, false>(lora, grid, s, p);
}

}  // namespace

int decode_workspace_bytes(int64_t m, int64_t n, int64_t k, int slices, int max_rank) {
  return int(workspace_layout(m, n, k, slices, max_rank).total);
}

int launch_nf4_lora_decode(const uint16_t* x, int64_t m, int64_t x_stride, const lf_nf4_weight* w,
                           const uint16_t* bias, const lf_lora* lora, uint16_t* y, int64_t y_stride,
                           void* workspace, int64_t workspace_bytes, void* stream) {
  const int64_t n = w->n, k = w->k;
  const int slices = lora ? lora->num_slices : 1;
  const int max_rank = lora ? lora->max_rank : 1;
  const Layout lay = workspace_layout(m, n, k, slices, max_rank);
  LF_REQUIRE(workspace && workspace_bytes >= lay.total, "workspace too small: need %lld bytes",
             (long long)lay.total);
  LF_REQUIRE(aligned16(workspace), "workspace must be 16-byte aligned");
  const Plan pl = make_plan(m, n, k);
  DecodeParams p{};
  p.x = x;
  p.x_stride = x_stride;
  p.m = int(m);
  p.q = w->qweight;
  p.src = ScaleSource{w->scales, w->absmax_q, w->absmax2, w->code2, w->offset, int(w->dq_block)};
  p.code = w->code;
  p.n = int(n);
  p.k = int(k);
  p.bias = bias;
  p.y = y;
  p.y_stride = y_stride;
  p.slices = slices;
  p.max_rank = max_rank;
  p.zw = slices * max_rank;
  p.ksplit = pl.ksplit;
  p.chunks = pl.chunks;
  p.ntiles = int(n / 16);
  char* ws = static_cast<char*>(workspace);
  p.ctrl = reinterpret_cast<int*>(ws);
  p.tile_count = reinterpret_cast<int*>(ws + lay.tile_count);
  p.zbuf = reinterpret_cast<float*>(ws + lay.zbuf);
  p.part = reinterpret_cast<float*>(ws + lay.part);
  if (lora) {
    p.a_store = lora->a_store;
    p.a_offsets = lora->a_offsets;
    p.b_store = lora->b_store;
    p.b_offsets = lora->b_offsets;
    p.b_strides = lora->b_strides;
    p.ranks = lora->ranks;
    p.lscales = lora->scales;
    p.token_slots = lora->token_slots;
    p.slice_offsets = lora->slice_offsets;
    p.zgroups = (slices * max_rank + 3) / 4;
    p.nz = int(m) * p.zgroups;
  }
  const dim3 grid(unsigned(p.nz + pl.groups));
  auto s = static_cast<hipStream_t>(stream);
  const bool dq = w->scales == nullptr;
  const bool has_lora = lora != nullptr;
  switch (pl.tm * 10 + pl.row_tiles) {
    case 11: launch_dq_variant<1, 1>(dq, has_lora, grid, s, p); break;
    case 24: launch_dq_variant<2, 4>(dq, has_lora, grid, s, p); break;
    case 34: launch_dq_variant<3, 4>(dq, has_lora, grid, s, p); break;
    case 44: launch_dq_variant<4, 4>(dq, has_lora, grid, s, p); break;
    default: return fail(kInvalid, "unsupported decode plan");
  }
  LF_HIP(hipGetLastError());
  return kOk;
}

}  // namespace lf
