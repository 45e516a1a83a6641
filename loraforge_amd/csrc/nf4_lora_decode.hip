// Fused NF4 base linear + per-token multi-LoRA for decode batches (M <= 64),
// one kernel launch per call.
//
// Reference chain being fused (all in one launch here):
//   integrations/_sglang_nf4_linear.py:116-129  y = bf16(x @ dequant(W)^T) (+bias)
//   ops/csrc/lora_rows.cu:35-65                 z = bf16(A_g @ x)
//   ops/csrc/lora_rows.cu:67-117                y = bf16(y + bf16(scale * B_g @ z))
//
// Work split (blockIdx ranges):
//   [0, nz)     shrink groups: (token, 4 A rows). Only the first token of each
//               slot works; it contracts its 4 A rows against every token
//               sharing that slot, so each A row is read once.
//   [nz, grid)  base groups over 16-row tiles of W. Every W byte of a group is
//               requested before any arithmetic (one memory round trip per
//               segment of <= 8 chunks of 128 k), NF4 is decoded in registers
//               (codebook in LDS) to the exact bf16 W values, and
//               v_mfma_f32_16x16x32_bf16 takes x as the A operand (tokens
//               padded to 16) and W^T as the B operand.
//               kRowTiles == 1 (M <= 16): the 4 waves split K; x fragments
//               come straight from L2 into registers (only real tokens load).
//               kRowTiles == 4 (M > 16): each wave owns a tile, the 4 waves
//               share x, which is copied global -> LDS by the gfx950 direct
//               load (global_load_lds_dwordx4) in MFMA fragment order; K may
//               be split across groups, the last group of a tile reduces the
//               fp32 partials.
//   The epilogue (bf16 round, bias, LoRA expand, bf16 rounds) runs on the
//   group that completes a tile; it waits on the shrink counter (bounded
//   spin; shrink groups have lower ids, so they are dispatched first).
//   Counters are reset by their last user, so the workspace is left zeroed.
//
// Cross-workgroup exchange uses no cache-wide fences: every value another
// workgroup reads (z, partials, counters) is written and read with
// device-coherent (agent-scope) relaxed atomic accesses, which keep each
// location coherent across the XCD L2s. A producer's stores complete (the
// workgroup release inside __syncthreads waits for them) before its counter
// update is issued; a consumer loads data only after observing the counter.
#include "nf4_common.h"
#include "../../include/loraforge_amd.h"

namespace lf {
namespace {

constexpr int kThreads = 256;
constexpr int kChunkK = 128;  // k per chunk: 4 lane groups x 32 nibbles
constexpr int kSeg = 8;       // chunks requested per memory round trip
constexpr int kCtrlBytes = 256;
constexpr int kSpinLimit = 1 << 22;
constexpr int kMaxZ = 64 * 192;  // tokens x (slices * max_rank)
constexpr int kCopiesSplitK = 32;  // pair-table copies (bank-private) when waves split K
constexpr int kCopiesSplitRows = 16;  // fewer copies when x fills most of LDS
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
  int nz;      // shrink groups
  int zgroups; // shrink groups per token
  int ksplit;  // K splits across groups (kRowTiles == 4)
  int chunks;  // ceil(K / 128)
  int ntiles;  // N / 16
  int zw;      // z row width = slices * max_rank
  int* ctrl;
  int* tile_count;
  float* zbuf;
  float* part;
};

__device__ __forceinline__ int counter_add(int* p, int v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int counter_load(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void counter_store(int* p, int v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void shared_store(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float shared_load(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
// Shrink group: z[t, j] = bf16(A_g[j] . x[t]) for this group's 4 A rows and
// every token t routed to slot g. Each lane owns 8 consecutive k of every
// 512-wide step; all A and x loads of a 4096-k segment are issued together.
// ---------------------------------------------------------------------------
__device__ void shrink_group(const DecodeParams& p, int* list, int* slots) {
  const int tok = blockIdx.x / p.zgroups;
  const int rg = blockIdx.x - tok * p.zgroups;
  if (threadIdx.x < p.m) slots[threadIdx.x] = p.token_slots[threadIdx.x];
  __syncthreads();
  const int g = slots[tok];
  int r = g >= 0 ? p.ranks[g] : 0;
  if (r > p.max_rank) r = 0;  // metadata contract: rank <= max_rank
  const int rows = p.slices * r;
  const bool work = r > 0 && rg * 4 < rows;
  if (work && threadIdx.x == 0) {
    int count = 0;
    bool leader = true;
    for (int t = 0; t < p.m; ++t) {
      if (slots[t] == g) {
        if (t < tok) {
          leader = false;
          break;
        }
        list[count++] = t;
      }
    }
    list[64] = leader ? count : 0;
  }
  __syncthreads();
  const int count = work ? list[64] : 0;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int row = rg * 4 + wave;
  if (count > 0 && row < rows) {
    const uint16_t* arow = p.a_store + p.a_offsets[g] + int64_t(row) * p.k;
    for (int base = 0; base < count; base += 2) {
      const int t0 = list[base];
      const int t1 = base + 1 < count ? list[base + 1] : t0;
      const uint16_t* x0 = p.x + int64_t(t0) * p.x_stride;
      const uint16_t* x1 = p.x + int64_t(t1) * p.x_stride;
      float acc0 = 0.f, acc1 = 0.f;
      for (int seg = 0; seg < p.k; seg += 8 * 512) {
        uint4 av[8], xv0[8], xv1[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int kk = seg + i * 512 + lane * 8;
          const bool ok = kk < p.k;
          av[i] = ok ? *reinterpret_cast<const uint4*>(arow + kk) : make_uint4(0, 0, 0, 0);
          xv0[i] = ok ? *reinterpret_cast<const uint4*>(x0 + kk) : make_uint4(0, 0, 0, 0);
          xv1[i] = ok ? *reinterpret_cast<const uint4*>(x1 + kk) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          acc0 = dot8(av[i], xv0[i], acc0);
          acc1 = dot8(av[i], xv1[i], acc1);
        }
      }
      acc0 = wave_sum(acc0);
      acc1 = wave_sum(acc1);
      if (lane == 0) {
        shared_store(p.zbuf + int64_t(t0) * p.zw + row, round_bf16(acc0));
        if (base + 1 < count) shared_store(p.zbuf + int64_t(t1) * p.zw + row, round_bf16(acc1));
      }
    }
  }
  __syncthreads();  // all z stores of this group have completed
  if (threadIdx.x == 0) counter_add(p.ctrl + kZDone, 1);
}

// ---------------------------------------------------------------------------
// Base contraction. Lane l: row n = 16*tile + (l & 15), lane group gq = l >> 4.
// Chunk c covers k in [128c, 128c + 128) = NF4 blocks 2c and 2c + 1; the lane
// loads 8 packed bytes of each block (k = 128c + 64h + 16gq .. +16, h = 0, 1)
// so that MFMA step j (k = 128c + 64(j >> 1) + 16gq + 8(j & 1) .. +8, same
// mapping for both operands) stays inside block 2c + (j >> 1).
//
// Fast path (default): the B operand is bf16(code[nibble]) read from a
// byte -> bf16-pair table, and the fp32 block scale is applied to the
// per-block MFMA sums (acc += s_b * sum_b), so a weight costs one table read
// per two elements plus address arithmetic. The table holds 256 entries x
// kCopies copies with copy c at dword e * kCopies + c: lane l always reads its
// own bank, so random byte values never conflict.
// Exact path: the B operand is bf16_rne(code[nibble] * scale) (the reference's
// dequantised weight, bit for bit) and MFMA accumulates it directly.
// ---------------------------------------------------------------------------
struct WRaw {
  uint2 q0, q1;     // packed bytes of blocks 2c and 2c + 1
  float s0, s1;     // fp32 block scales, or second-level scales (double quant)
  uint32_t a0, a1;  // double-quant absmax codes
  bool v0, v1;      // block inside this wave's chunk range / inside K
};

// Branch-free: out-of-range chunks load clamped (valid) addresses and are
// neutralised by a zero scale, so the compiler can count outstanding loads
// exactly and compute on early chunks while later ones are in flight.
template <bool kDouble>
__device__ __forceinline__ WRaw load_w(const DecodeParams& p, int n, int c, int c_end, int gq) {
  WRaw w;
  w.v0 = c < c_end;
  const int cc = w.v0 ? c : 0;
  w.v1 = w.v0 && cc * kChunkK + 64 < p.k;
  const int64_t row = int64_t(n) * p.k;
  const int kb0 = cc * kChunkK;
  const int kb1 = w.v1 ? kb0 + 64 : kb0;
  const int64_t blk0 = (row + kb0) / kNf4Block;
  const int64_t blk1 = (row + kb1) / kNf4Block;
  w.q0 = *reinterpret_cast<const uint2*>(p.q + (row + kb0) / 2 + gq * 8);
  w.q1 = *reinterpret_cast<const uint2*>(p.q + (row + kb1) / 2 + gq * 8);
  if constexpr (kDouble) {
    w.a0 = p.src.absmax_q[blk0];
    w.a1 = p.src.absmax_q[blk1];
    w.s0 = p.src.absmax2[blk0 / p.src.dq_block];
    w.s1 = p.src.absmax2[blk1 / p.src.dq_block];
  } else {
    w.s0 = p.src.scales[blk0];
    w.s1 = p.src.scales[blk1];
    w.a0 = w.a1 = 0;
  }
  return w;
}

// Final fp32 block scales (0 for neutralised blocks).
template <bool kDouble>
__device__ __forceinline__ void finish_scales(const WRaw& w, const float* code2, float offset, float& s0,
                                              float& s1) {
  if constexpr (kDouble) {
    s0 = code2[w.a0] * w.s0 + offset;
    s1 = code2[w.a1] * w.s1 + offset;
  } else {
    s0 = w.s0;
    s1 = w.s1;
  }
  s0 = w.v0 ? s0 : 0.f;
  s1 = w.v1 ? s1 : 0.f;
}

// 8 elements (one packed dword) -> 4 unscaled bf16 pairs; ptl = table + (lane % kCopies).
template <int kCopies>
__device__ __forceinline__ uint4 codes_dword(uint32_t d, const uint32_t* ptl) {
  uint4 r;
  r.x = ptl[(d & 0xffu) * kCopies];
  r.y = ptl[__builtin_amdgcn_ubfe(d, 8, 8) * kCopies];
  r.z = ptl[__builtin_amdgcn_ubfe(d, 16, 8) * kCopies];
  r.w = ptl[(d >> 24) * kCopies];
  return r;
}

template <int TM, bool kDouble, bool kExact, int kCopies>
__device__ __forceinline__ void mfma_chunk(const WRaw& w, const uint4 (&xf)[TM][4], f32x4 (&acc)[TM],
                                           const float* table, const uint32_t* ptl, const float* code2,
                                           float offset) {
  float s0, s1;
  finish_scales<kDouble>(w, code2, offset, s0, s1);
  if constexpr (kExact) {
    const uint4 wd[4] = {decode_dword(w.q0.x, s0, table), decode_dword(w.q0.y, s0, table),
                         decode_dword(w.q1.x, s1, table), decode_dword(w.q1.y, s1, table)};
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) acc[tm] = mfma16(as_bf16x8(xf[tm][j]), as_bf16x8(wd[j]), acc[tm]);
  } else {
    const uint4 wd[4] = {codes_dword<kCopies>(w.q0.x, ptl), codes_dword<kCopies>(w.q0.y, ptl),
                         codes_dword<kCopies>(w.q1.x, ptl), codes_dword<kCopies>(w.q1.y, ptl)};
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      f32x4 b0 = mfma16(as_bf16x8(xf[tm][0]), as_bf16x8(wd[0]), zero);
      b0 = mfma16(as_bf16x8(xf[tm][1]), as_bf16x8(wd[1]), b0);
      f32x4 b1 = mfma16(as_bf16x8(xf[tm][2]), as_bf16x8(wd[2]), zero);
      b1 = mfma16(as_bf16x8(xf[tm][3]), as_bf16x8(wd[3]), b1);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[tm][e] = __builtin_fmaf(s1, b1[e], __builtin_fmaf(s0, b0[e], acc[tm][e]));
    }
  }
}

// k offset of MFMA step j for lane group gq inside chunk c.
__device__ __forceinline__ int step_k(int c, int gq, int j) { return c * kChunkK + 64 * (j >> 1) + 16 * gq + 8 * (j & 1); }

// Per-token LoRA metadata gathered into LDS once per group, in parallel, while
// the weight loads are in flight (the epilogue then reads no metadata chains).
struct TokenMeta {
  int rank[64];  // 0 = base only
  int stride[64];
  float scale[64];
  int64_t boff[64];
  int bounds[4];
};

// Three steps so the dependent loads never force a wait on the weight stream:
// the slot ids are loaded before the weights, the slot-indexed values right
// after them, and the LDS writes happen once the contraction is done.
struct MetaRegs {
  int g;
  int r;
  int stride;
  float scale;
  int64_t boff;
  int bound;
};

__device__ __forceinline__ MetaRegs meta_slots(const DecodeParams& p) {
  MetaRegs m{};
  const int t = threadIdx.x;
  m.g = t < p.m ? p.token_slots[t] : -1;
  const int b = t - 64;
  m.bound = (b >= 0 && b <= p.slices && b < 4) ? p.slice_offsets[b] : 0;
  return m;
}

__device__ __forceinline__ void meta_values(const DecodeParams& p, MetaRegs& m) {
  const int gs = m.g >= 0 ? m.g : 0;  // slot 0 exists whenever LoRA is on
  const int r = p.ranks[gs];
  m.stride = p.b_strides[gs];
  m.scale = p.lscales[gs];
  m.boff = p.b_offsets[gs];
  m.r = (m.g >= 0 && r <= p.max_rank) ? r : 0;
}

__device__ __forceinline__ void meta_commit(const DecodeParams& p, const MetaRegs& m, TokenMeta* meta) {
  const int t = threadIdx.x;
  if (t < p.m) {
    meta->rank[t] = m.r;
    meta->stride[t] = m.stride;
    meta->scale[t] = m.scale;
    meta->boff[t] = m.boff;
  }
  if (t >= 64 && t < 68) meta->bounds[t - 64] = m.bound;
}

// NF4 tables in LDS. The codebook values are loaded before any weight load
// (vector loads retire in order, so waiting for them does not wait for the
// weight stream) and written to LDS after the weight loads are issued.
struct CodeRegs {
  float c16;  // code[lane % 16] (exact table)
  float hi, lo;  // code[e >> 4], code[e & 15] for pair entry e = thread id
  float c2;   // code2[thread id] (double quant)
};

template <bool kDouble>
__device__ __forceinline__ CodeRegs load_code(const DecodeParams& p) {
  CodeRegs r;
  const int e = threadIdx.x;
  r.c16 = p.code[e & 15];
  r.hi = p.code[e >> 4];
  r.lo = p.code[e & 15];
  r.c2 = kDouble ? p.src.code2[e] : 0.f;
  return r;
}

template <bool kDouble, bool kExact, int kCopies>
__device__ __forceinline__ void stage_tables(const CodeRegs& r, float* table, uint32_t* pt, float* code2) {
  if (threadIdx.x < 16) table[threadIdx.x] = r.c16;
  if constexpr (kDouble) code2[threadIdx.x] = r.c2;
  if constexpr (!kExact) {
    const uint32_t v = pack_bf16x2(r.hi, r.lo);
    uint4* dst = reinterpret_cast<uint4*>(pt + threadIdx.x * kCopies);
#pragma unroll
    for (int c = 0; c < kCopies / 4; ++c) dst[c] = make_uint4(v, v, v, v);
  }
}

// ---------------------------------------------------------------------------
// Epilogue for one 16-row tile: c_tile is [16*TM tokens][16 rows] fp32 in LDS,
// zl the call's z values [m][zw] staged in LDS.
// ---------------------------------------------------------------------------
template <bool kLora>
__device__ void epilogue_tile(const DecodeParams& p, int tile, const float* c_tile, const float* zl,
                              const TokenMeta* meta) {
  const int n0 = tile * 16;
  for (int idx = threadIdx.x; idx < p.m * 16; idx += kThreads) {
    const int t = idx >> 4;
    const int row = idx & 15;
    const int n = n0 + row;
    float v = round_bf16(c_tile[idx]);
    if (p.bias) v = round_bf16(v + bf16_to_f32(p.bias[n]));
    if constexpr (kLora) {
      const int r = meta->rank[t];
      if (r > 0) {
        int s = 0;
        for (int i = 1; i < p.slices; ++i) s += n >= meta->bounds[i];
        const int br = meta->stride[t];
        const uint16_t* brow = p.b_store + meta->boff[t] + int64_t(n) * br;
        const float* zt = zl + t * p.zw + s * r;
        float acc = 0.f;
        int j = 0;
        if ((br & 7) == 0) {
          for (; j + 8 <= r; j += 8) {
            const uint4 bv = *reinterpret_cast<const uint4*>(brow + j);
            acc = __builtin_fmaf(zt[j + 0], bf16_lo(bv.x), acc);
            acc = __builtin_fmaf(zt[j + 1], bf16_hi(bv.x), acc);
            acc = __builtin_fmaf(zt[j + 2], bf16_lo(bv.y), acc);
            acc = __builtin_fmaf(zt[j + 3], bf16_hi(bv.y), acc);
            acc = __builtin_fmaf(zt[j + 4], bf16_lo(bv.z), acc);
            acc = __builtin_fmaf(zt[j + 5], bf16_hi(bv.z), acc);
            acc = __builtin_fmaf(zt[j + 6], bf16_lo(bv.w), acc);
            acc = __builtin_fmaf(zt[j + 7], bf16_hi(bv.w), acc);
          }
        }
        for (; j < r; ++j) acc = __builtin_fmaf(zt[j], bf16_to_f32(brow[j]), acc);
        v = round_bf16(v + round_bf16(acc * meta->scale[t]));
      }
    }
    p.y[int64_t(t) * p.y_stride + n] = uint16_t(f32_to_bf16(v));
  }
}

// Wait (bounded) until every shrink group has published, then stage z in LDS.
__device__ void wait_and_stage_z(const DecodeParams& p, float* zl) {
  if (threadIdx.x == 0) {
    int spins = 0;
    while (counter_load(p.ctrl + kZDone) < p.nz) {
      __builtin_amdgcn_s_sleep(2);
      if (++spins > kSpinLimit) {
        counter_store(p.ctrl + kStatus, 1);
        break;
      }
    }
  }
  __syncthreads();
  const int total = p.m * p.zw;
  for (int i = threadIdx.x; i < total; i += kThreads) zl[i] = shared_load(p.zbuf + i);
  __syncthreads();
}

__device__ void finish_tiles(const DecodeParams& p, int tiles) {
  if (threadIdx.x == 0) {
    const int done = counter_add(p.ctrl + kTilesDone, tiles);
    if (done == p.ntiles - tiles) {  // last tile epilogue: reset for the next call
      counter_store(p.ctrl + kZDone, 0);
      counter_store(p.ctrl + kTilesDone, 0);
    }
  }
}

// ---------------------------------------------------------------------------
// kRowTiles == 1 (M <= 16): one tile per group, the 4 waves split K.
// ---------------------------------------------------------------------------
template <bool kDouble, bool kLora, bool kExact>
__device__ void base_split_k(const DecodeParams& p, float* table, uint32_t* pt, float* code2, float* red, float* zl,
                             TokenMeta* meta) {
  const int tile = blockIdx.x - p.nz;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int gq = lane >> 4;
  const int n = tile * 16 + (lane & 15);
  const int tok = lane & 15;
  const bool real = tok < p.m;
  const uint16_t* xrow = p.x + int64_t(real ? tok : 0) * p.x_stride;
  const uint32_t* ptl = pt + (lane % kCopiesSplitK);
  const int per = (p.chunks + 3) >> 2;
  const int c0 = wave * per;
  const int c1 = min(p.chunks, c0 + per);
  const CodeRegs codes = load_code<kDouble>(p);
  const float offset = kDouble ? *p.src.offset : 0.f;
  MetaRegs mr{};
  if constexpr (kLora) mr = meta_slots(p);
  f32x4 acc[1] = {(f32x4){0.f, 0.f, 0.f, 0.f}};
  WRaw w[kSeg];
  uint4 xf[kSeg][1][4];
  // Padded token lanes read token 0 (their output rows are never stored);
  // chunks past the range read chunk 0 and are scaled by 0.
  auto issue = [&](int cs) {
#pragma unroll
    for (int i = 0; i < kSeg; ++i) w[i] = load_w<kDouble>(p, n, cs + i, c1, gq);
#pragma unroll
    for (int i = 0; i < kSeg; ++i) {
      const int cc = cs + i < c1 ? cs + i : 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int kk = step_k(cc, gq, j);
        xf[i][0][j] = *reinterpret_cast<const uint4*>(xrow + (kk < p.k ? kk : 0));
      }
    }
  };
  issue(c0);  // unconditional: a wave without chunks computes zeros
  if constexpr (kLora) meta_values(p, mr);
  stage_tables<kDouble, kExact, kCopiesSplitK>(codes, table, pt, code2);
  __syncthreads();
  for (int cs = c0;;) {
#pragma unroll
    for (int i = 0; i < kSeg; ++i) mfma_chunk<1, kDouble, kExact, kCopiesSplitK>(w[i], xf[i], acc, table, ptl, code2, offset);
    cs += kSeg;
    if (cs >= c1) break;
    issue(cs);
  }
  *reinterpret_cast<f32x4*>(red + (wave * 64 + lane) * 4) = acc[0];
  if constexpr (kLora) meta_commit(p, mr, meta);
  __syncthreads();
  // c_tile[token][row], token = 4*(l>>4) + e, row = l & 15.
  float* c_tile = red + 4 * 256;
  {
    const int i = threadIdx.x;
    const int l = i >> 2;
    const int e = i & 3;
    float s = 0.f;
#pragma unroll
    for (int wv = 0; wv < 4; ++wv) s += red[(wv * 64 + l) * 4 + e];
    c_tile[(4 * (l >> 4) + e) * 16 + (l & 15)] = s;
  }
  __syncthreads();
  if constexpr (kLora) wait_and_stage_z(p, zl);
  epilogue_tile<kLora>(p, tile, c_tile, zl, meta);
  if constexpr (kLora) finish_tiles(p, 1);
}

// ---------------------------------------------------------------------------
// kRowTiles == 4 (M > 16): each wave owns a tile; x is copied to LDS in MFMA
// fragment order: block (chunk i, tm, step j) holds lane l's 16 bytes
// x[16tm + (l & 15)][128c + 32(l >> 4) + 8j ..] at offset l*16 (conflict-free
// ds_read_b128). Padded token lanes read row 0; their rows are never stored.
// ---------------------------------------------------------------------------
template <int TM>
__device__ __forceinline__ void stage_x_lds(const DecodeParams& p, int cs, int nseg, uint4* xs) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int blocks = nseg * TM * 4;
  for (int b = wave; b < blocks; b += 4) {
    const int i = b / (TM * 4);
    const int tm = (b / 4) % TM;
    const int j = b & 3;
    const int t = tm * 16 + (lane & 15);
    const int kb = step_k(cs + i, lane >> 4, j);
    const int row = t < p.m ? t : 0;
    const int kk = kb < p.k ? kb : 0;
    const uint16_t* src = p.x + int64_t(row) * p.x_stride + kk;
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(xs + b * 64), 16, 0, 0);
  }
}

template <int TM, bool kDouble, bool kLora, bool kExact>
__device__ void base_split_rows(const DecodeParams& p, float* table, uint32_t* pt, float* code2, uint4* xs,
                                float* c_tiles, float* zl, int* flag, TokenMeta* meta) {
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
  const uint32_t* ptl = pt + (lane % kCopiesSplitRows);
  const CodeRegs codes = load_code<kDouble>(p);
  const float offset = kDouble ? *p.src.offset : 0.f;
  MetaRegs mr{};
  if constexpr (kLora) mr = meta_slots(p);
  f32x4 acc[TM];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) acc[tm] = (f32x4){0.f, 0.f, 0.f, 0.f};
  WRaw w[kSeg];
  for (int cs = c0; cs < c1; cs += kSeg) {
    const int nseg = min(kSeg, c1 - cs);
#pragma unroll
    for (int i = 0; i < kSeg; ++i) w[i] = load_w<kDouble>(p, n, cs + i, c1, gq);
    stage_x_lds<TM>(p, cs, nseg, xs);
    if (cs == c0) {
      if constexpr (kLora) meta_values(p, mr);
      stage_tables<kDouble, kExact, kCopiesSplitRows>(codes, table, pt, code2);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's direct LDS loads landed
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kSeg; ++i) {
      if (i < nseg) {
        uint4 xf[TM][4];
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
          for (int j = 0; j < 4; ++j) xf[tm][j] = xs[((i * TM + tm) * 4 + j) * 64 + lane];
        mfma_chunk<TM, kDouble, kExact, kCopiesSplitRows>(w[i], xf, acc, table, ptl, code2, offset);
      }
    }
    __syncthreads();  // x buffer free for the next segment
  }
  if (c0 >= c1) {  // a split without chunks still provides tables and metadata
    if constexpr (kLora) meta_values(p, mr);
    stage_tables<kDouble, kExact, kCopiesSplitRows>(codes, table, pt, code2);
    __syncthreads();
  }
  if constexpr (kLora) meta_commit(p, mr, meta);
  float* mine = c_tiles + wave * (TM * 256);
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int e = 0; e < 4; ++e) mine[(tm * 16 + 4 * gq + e) * 16 + (lane & 15)] = acc[tm][e];
  __syncthreads();
  const int tile_elems = 4 * TM * 256;
  if (p.ksplit > 1) {
    float* mypart = p.part + (int64_t(grp) * p.ksplit + split) * tile_elems;
    for (int i = threadIdx.x; i < tile_elems; i += kThreads) shared_store(mypart + i, c_tiles[i]);
    __syncthreads();  // all partial stores of this group have completed
    if (threadIdx.x == 0) {
      const int prev = counter_add(p.tile_count + grp, 1);
      const bool last = prev == p.ksplit - 1;
      if (last) counter_store(p.tile_count + grp, 0);
      *flag = last;
    }
    __syncthreads();
    if (!*flag) return;
    const float* parts = p.part + int64_t(grp) * p.ksplit * tile_elems;
    for (int i = threadIdx.x; i < tile_elems; i += kThreads) {
      float s = 0.f;
      for (int sp = 0; sp < p.ksplit; ++sp) s += shared_load(parts + int64_t(sp) * tile_elems + i);
      c_tiles[i] = s;
    }
    __syncthreads();
  }
  if constexpr (kLora) wait_and_stage_z(p, zl);
  for (int t = 0; t < 4; ++t) epilogue_tile<kLora>(p, grp * 4 + t, c_tiles + t * TM * 256, zl, meta);
  if constexpr (kLora) finish_tiles(p, 4);
}

template <int TM, int kRowTiles, bool kDouble, bool kLora, bool kExact>
__global__ __launch_bounds__(kThreads) void nf4_lora_decode_kernel(DecodeParams p) {
  constexpr int kCopies = kRowTiles == 1 ? kCopiesSplitK : kCopiesSplitRows;
  __shared__ float table[16];
  __shared__ float code2[kDouble ? 256 : 1];
  __shared__ int flag[72];
  __shared__ uint32_t pt[kExact ? 1 : 256 * kCopies];
  constexpr int kRed = kRowTiles == 1 ? 5 * 256 : 1;
  constexpr int kXs = kRowTiles == 4 ? kSeg * TM * 4 * 64 : 1;
  constexpr int kCt = 4 * TM * 256;
  constexpr int kZl = kLora && kRowTiles == 1 ? 16 * 192 : 1;
  static_assert(kRowTiles == 1 || kXs * 4 >= kCt + (kLora ? kMaxZ : 0), "tiles and z reuse the x buffer");
  __shared__ float red[kRed];
  __shared__ uint4 xs[kXs];
  __shared__ float zl_own[kZl];
  __shared__ TokenMeta meta[1];
  __shared__ int slot_copy[kLora ? 64 : 1];
  // With row tiles, the output tiles and z reuse the x buffer (dead by then).
  float* c_tiles = reinterpret_cast<float*>(xs);
  float* zl = kRowTiles == 4 ? reinterpret_cast<float*>(xs) + kCt : zl_own;
  if constexpr (kLora) {
    if (int(blockIdx.x) < p.nz) {
      shrink_group(p, flag, slot_copy);
      return;
    }
  }
  if constexpr (kRowTiles == 1) {
    base_split_k<kDouble, kLora, kExact>(p, table, pt, code2, red, zl, meta);
  } else {
    base_split_rows<TM, kDouble, kLora, kExact>(p, table, pt, code2, xs, c_tiles, zl, flag, meta);
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
    // Enough groups to cover every CU (256 on MI355X) without splitting K
    // more than needed: every split adds a partial-tile exchange.
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

template <int TM, int RT, bool D, bool E>
void launch_lora_variant(bool lora, dim3 grid, hipStream_t s, const DecodeParams& p) {
  if (lora) {
    hipLaunchKernelGGL((nf4_lora_decode_kernel<TM, RT, D, true, E>), grid, dim3(kThreads), 0, s, p);
  } else {
    hipLaunchKernelGGL((nf4_lora_decode_kernel<TM, RT, D, false, E>), grid, dim3(kThreads), 0, s, p);
  }
}

template <int TM, int RT>
void launch_variant(bool dq, bool lora, bool exact, dim3 grid, hipStream_t s, const DecodeParams& p) {
  if (exact) {
    if (dq) launch_lora_variant<TM, RT, true, true>(lora, grid, s, p);
    else launch_lora_variant<TM, RT, false, true>(lora, grid, s, p);
  } else {
    if (dq) launch_lora_variant<TM, RT, true, false>(lora, grid, s, p);
    else launch_lora_variant<TM, RT, false, false>(lora, grid, s, p);
  }
}

}  // namespace

int decode_workspace_bytes(int64_t m, int64_t n, int64_t k, int slices, int max_rank) {
  return int(workspace_layout(m, n, k, slices, max_rank).total);
}

int launch_nf4_lora_decode(const uint16_t* x, int64_t m, int64_t x_stride, const lf_nf4_weight* w,
                           const uint16_t* bias, const lf_lora* lora, uint16_t* y, int64_t y_stride,
                           void* workspace, int64_t workspace_bytes, bool exact, void* stream) {
  const int64_t n = w->n, k = w->k;
  const int slices = lora ? lora->num_slices : 1;
  const int max_rank = lora ? lora->max_rank : 1;
  LF_REQUIRE(m <= 64, "decode path handles at most 64 tokens");
  const Layout lay = workspace_layout(m, n, k, slices, max_rank);
  LF_REQUIRE(workspace && workspace_bytes >= lay.total, "workspace too small: need %lld bytes",
             (long long)lay.total);
  LF_REQUIRE(aligned16(workspace), "workspace must be 16-byte aligned");
  const Plan pl = make_plan(m, n, k);
  LF_REQUIRE(!lora || int64_t(slices) * max_rank * (pl.row_tiles == 1 ? 16 : 64) <= kMaxZ,
             "z staging exceeds its LDS budget");
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
    case 11: launch_variant<1, 1>(dq, has_lora, exact, grid, s, p); break;
    case 24: launch_variant<2, 4>(dq, has_lora, exact, grid, s, p); break;
    case 34: launch_variant<3, 4>(dq, has_lora, exact, grid, s, p); break;
    case 44: launch_variant<4, 4>(dq, has_lora, exact, grid, s, p); break;
    default: return fail(kInvalid, "unsupported decode plan");
  }
  LF_HIP(hipGetLastError());
  return kOk;
}

}  // namespace lf
