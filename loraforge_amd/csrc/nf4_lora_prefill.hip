// Prefill (M > 64 tokens): NF4 GEMM on bf16 MFMA with a multi-LoRA epilogue.
//
// Reference chain (integrations/_sglang_nf4_linear.py:116-129 for the base,
// benchmarks/qwen35_prefill_fused.py:95-171 segmented_ab_kernel for the
// LoRA part):  y = bf16(x @ dequant(W)^T) (+bias);  z = bf16(A_g x);
//              y = bf16(y + bf16(scale_g * B_g z)).
//
// One launch (wide::gemm_kernel) on the caller's stream (a double-quant
// weight first gets its fp32 block scales rebuilt into the workspace):
//  - LoRA launches start with zparts z producers per 256-token tile, each
//    serving a share of the tile's distinct adapters: z = bf16(x A_g^T) of
//    just the tokens routed to g (gathered, 16 per wave, MFMA), into a
//    slice-padded workspace zpad[m][s*64 + j] (zeros past r), then the
//    producer's flag is set to the call's tag (call_epoch.h).
//  - GEMM tiles of 256 tokens x 192 output features: x streamed by direct
//    global -> LDS copies, W decoded once per tile to the reference's exact
//    weights bf16_rne(code * scale) into LDS, contracted on
//    v_mfma_f32_16x16x32_bf16. LDS rows are 128 B with a 16-byte-unit XOR
//    swizzle (unit ^ row % 8). Epilogue: round, bias; with LoRA, wait for the
//    flags of the tile's producers (lower block ids, so already running), stage the tile's z rows per slice in LDS and, for every
//    distinct slot in the tile, a second MFMA pass z x B_g^T over the 16-row
//    blocks holding its tokens gives the delta, applied with the reference's
//    two bf16 roundings to the rows routed to that slot.
#include <algorithm>

#include "call_epoch.h"
#include "lds_pipeline.h"
#include "nf4_common.h"
#include "../../include/loraforge_amd.h"

namespace lf {
namespace {

constexpr int kThreads = 256;
constexpr int kBM = 256;
constexpr int kBK = 64;
constexpr int kZSlice = 64;  // zpad columns per slice

struct PrefillParams {
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
  int num_slots;      // entries of the per-slot arrays (0: not given; slots at or past it run base only)
  uint16_t* zpad;     // [m][slices * 64]
  int y_vec;          // 2: 16-byte aligned y rows, 1: 8-byte aligned, 0: neither
  uint32_t* zflags;   // [mtiles * zparts]: the call's tag once a producer's z rows are stored
  CallEpoch ce;
  int* status;  // set to 1 if a wait for z gives up (cannot happen while producers run first)
  int mtiles;
  int zparts;   // z producers per M-tile
  int spin_limit;  // polls of the bounded wait for a producer's flag
  int withhold;    // test hook: producers store nothing and set no flag, so consumers recompute z
};

__device__ __forceinline__ int swz(int row, int unit) { return row * 8 + (unit ^ (row & 7)); }

// Live slot of each token of [t0, t0 + count) (rank 0 or above 64: base
// only, -1), loaded by one thread per token, and the distinct live slots in
// order of first use: list[0 .. list[kMaxList]). Wave 0 extracts them with
// one ballot per distinct slot of each 64-token chunk; a slot already listed
// (checked 64 entries per ballot) is not added again.
constexpr int kMaxList = kBM;  // a tile routes to at most one slot per token
__device__ void live_slots(const PrefillParams& p, int t0, int count, int* tslot, int* list) {
  for (int t = threadIdx.x; t < kThreads; t += blockDim.x) {
    int g = t < count ? p.token_slots[t0 + t] : -1;
    if (p.num_slots > 0 && g >= p.num_slots) g = -1;
    const int r = g >= 0 ? p.ranks[g] : 0;
    if (r <= 0 || r > kZSlice) g = -1;  // rank 0 / contract violation: base only
    tslot[t] = g;
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    int nd = 0;
    for (int c = 0; c < count; c += 64) {
      const int g = c + lane < count ? tslot[c + lane] : -1;
      uint64_t left = __ballot(g >= 0);
      while (left) {
        const int gf = __builtin_amdgcn_readlane(g, __builtin_ctzll(left));
        left &= ~__ballot(g == gf);
        bool seen = false;
        for (int b = 0; b < nd && !seen; b += 64) seen = __ballot(b + lane < nd && list[b + lane] == gf) != 0;
        if (!seen) {
          if (lane == 0) list[nd] = gf;
          ++nd;
        }
      }
    }
    if (lane == 0) list[kMaxList] = nd;
  }
  __syncthreads();
}

// Raw B values kk .. kk + 7 of one row (stride br, a power of two; kk a
// multiple of 8) from a readable place: rows of stride >= 8 are 16-byte
// aligned and kk is clamped into the row; a narrower row is read whole (8,
// 4 or 2 bytes, aligned). keep_first() then keeps what belongs to B[kk..].
__device__ __forceinline__ uint4 b_raw(const uint16_t* row, int br, int kk) {
  if (br >= 8) return *reinterpret_cast<const uint4*>(row + min(kk, br - 8));
  if (br == 4) {
    const uint2 v = *reinterpret_cast<const uint2*>(row);
    return make_uint4(v.x, v.y, 0u, 0u);
  }
  if (br == 2) return make_uint4(*reinterpret_cast<const uint32_t*>(row), 0u, 0u, 0u);
  return make_uint4(row[0], 0u, 0u, 0u);
}

// The first `keep` bf16 values of v (none when keep <= 0), zeros after.
__device__ __forceinline__ uint4 keep_first(uint4 v, int keep) {
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (e >= keep) w[e >> 1] &= (e & 1) ? 0x0000ffffu : 0xffff0000u;
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// ---------------------------------------------------------------------------
// 2. GEMM + epilogue: 512 threads (two waves per SIMD), tile 256 tokens x
// 192 output features, BK = 64 (one NF4 block per W row).
//
// Per k-step a workgroup
//  - copies the x tile two steps ahead straight into a three-stage LDS ring
//    (global -> LDS, 16-byte XOR swizzle), four copies per wave;
//  - loads the packed W bytes and block scales two steps ahead into
//    registers (three dwords, 24 elements, per lane), and decodes the step
//    ahead to exact bf16_rne(code * scale) into the other half of a
//    two-stage decoded-W buffer, so each weight is decoded once per tile;
//  - contracts the current stage: waves (2 x 4) own 128 x 48 outputs
//    (8 x 3 fragments of v_mfma_f32_16x16x32_bf16), the decode work of the
//    next step interleaved with these MFMAs;
//  - waits for the next x copies and meets the other waves at one barrier.
// Tile order keeps M-tile b % mtiles on consecutive block ids (one 2 MiB x
// panel per XCD L2 with 8 M-tiles).
// ---------------------------------------------------------------------------
namespace wide {

constexpr int kThreads = 512;
constexpr int kBM = 256;
constexpr int kBN = 192;
constexpr int kXD = 3;                   // x ring depth
constexpr int kXBytes = kBM * 128;       // one x stage: 256 rows x 64 bf16
constexpr int kWBytes = kBN * 128;       // one decoded-W stage: 192 rows x 64 bf16
constexpr int kXCopies = kXBytes / 1024 / (kThreads / 64);  // 16-byte copies per lane and stage
constexpr int kDw = kBN * 8 / kThreads;  // packed W dwords per lane and stage
constexpr int kJ = 3;                    // 16-column fragments per wave
static_assert(kBN * 8 % kThreads == 0 && kXBytes % (1024 * (kThreads / 64)) == 0, "tile split");
static_assert(kXD * kXBytes + 2 * kWBytes + 2048 + 12 * 1024 <= 160 * 1024, "LDS budget (codebook pairs, LoRA tables)");
static_assert(kThreads == 512, "one codebook-pair float per thread");

// Packed W dwords and fp32 block scales of one k-step, loaded without
// compiler tracking (the x copies in flight would otherwise make every use of
// them wait for all outstanding memory operations).
struct Packed {
  uint32_t q[kDw];
  uint32_t s[kDw];  // fp32 scale bits
  static constexpr int kLoads = 2 * kDw;
};

__device__ __forceinline__ uint32_t gload32(const void* base, uint32_t voff) {
  uint32_t v;
  asm volatile("global_load_dword %0, %1, %2" : "=v"(v) : "v"(voff), "s"(base) : "memory");
  return v;
}

// Per-lane W addressing: lane dword i covers tile row (tid >> 3) + 64 i,
// elements 8 (tid & 7) .. + 8 of the k-step. Rows past N are clamped (their
// results are never stored).
struct WLane {
  uint32_t qoff[kDw];  // byte offset of the dword at k-step 0
  uint32_t soff[kDw];  // byte offset of the row's block scale at k-step 0
};

__device__ __forceinline__ void issue_w(const PrefillParams& p, int kt, const WLane& wl, Packed& w) {
  const uint8_t* qb = p.q + int64_t(kt) * 32;
#pragma unroll
  for (int i = 0; i < kDw; ++i) w.q[i] = gload32(qb, wl.qoff[i]);
  const float* sb = p.src.scales + kt;
#pragma unroll
  for (int i = 0; i < kDw; ++i) w.s[i] = gload32(sb, wl.soff[i]);
}

__device__ __forceinline__ void tie_w(Packed& w) {
#pragma unroll
  for (int i = 0; i < kDw; ++i) {
    tie(w.q[i]);
    tie(w.s[i]);
  }
}

// LDS accesses the compiler does not track, with immediate offsets.
template <int kOff>
__device__ __forceinline__ u32x4 ldsr128(uint32_t addr) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(kOff));
  return v;
}
template <int kOff>
__device__ __forceinline__ void ldsw128(uint32_t addr, const u32x4& v) {
  asm volatile("ds_write_b128 %0, %1 offset:%2" : : "v"(addr), "v"(v), "i"(kOff) : "memory");
}

// Decode of one loaded step into a decoded-W stage, in two halves: the
// codebook lookups of all dwords, then the scaling, rounding and the stores.
// The codebook sits in LDS as a byte -> (code[hi nibble], code[lo nibble])
// table of fp32 pairs (2 KiB, 2 KiB-aligned), so one 8-byte read returns the
// two codes of a packed byte.
struct Looked {
  float v[kDw][8];
};

struct LookAddr {
  uint32_t a[kDw][4];  // table address of packed byte b of dword i
};

__device__ __forceinline__ void lookup_addresses(const Packed& w, uint32_t table_addr, LookAddr& la) {
#pragma unroll
  for (int i = 0; i < kDw; ++i) {
    const uint32_t d = w.q[i];
    la.a[i][0] = ((d << 3) & 0x7f8u) | table_addr;
    la.a[i][1] = ((d >> 5) & 0x7f8u) | table_addr;
    la.a[i][2] = ((d >> 13) & 0x7f8u) | table_addr;
    la.a[i][3] = ((d >> 21) & 0x7f8u) | table_addr;
  }
}

// The 4 lookups of dword i (its 8 elements in order).
__device__ __forceinline__ void lookup_dword(const LookAddr& la, int i, Looked& lk) {
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const u32x2 v = lds_read64(la.a[i][b]);
    lk.v[i][2 * b] = __uint_as_float(v.x);
    lk.v[i][2 * b + 1] = __uint_as_float(v.y);
  }
}

__device__ __forceinline__ void tie_lookups(Looked& lk) {
#pragma unroll
  for (int i = 0; i < kDw; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) tie(lk.v[i][e]);
}

// bf16_rne(code * scale) of dword i's 8 elements, stored at row offset i * 64.
__device__ __forceinline__ void decode_store(const Packed& w, const Looked& lk, uint32_t dst) {
#pragma unroll
  for (int i = 0; i < kDw; ++i) {
    const float scale = __uint_as_float(w.s[i]);
    u32x4 r;
    r.x = pack_bf16x2(lk.v[i][0] * scale, lk.v[i][1] * scale);
    r.y = pack_bf16x2(lk.v[i][2] * scale, lk.v[i][3] * scale);
    r.z = pack_bf16x2(lk.v[i][4] * scale, lk.v[i][5] * scale);
    r.w = pack_bf16x2(lk.v[i][6] * scale, lk.v[i][7] * scale);
    if (i == 0) ldsw128<0>(dst, r);
    if (i == 1) ldsw128<64 * 128>(dst, r);
    if (i == 2) ldsw128<128 * 128>(dst, r);
  }
}
static_assert(kDw == 3, "decode_store writes three rows");

// Copies of x k-step kt into a ring stage: position P (16-byte unit) of the
// 32 KiB stage -> row P / 8, slot P % 8 holding unit (P % 8) ^ (row & 7).
// Rows past M are clamped (their results are never stored).
// (32-bit byte offsets from x, so the copies take a scalar base: the
// launcher checks that x spans less than 4 GiB.)
__device__ __forceinline__ void issue_x(const PrefillParams& p, char* stage, int m0, int kt, int wave, int lane) {
  const char* xk = reinterpret_cast<const char*>(p.x) + kt * (kBK * 2);
#pragma unroll
  for (int d = 0; d < kXCopies; ++d) {
    const int pos = (wave * kXCopies + d) * 64 + lane;
    const int row = pos >> 3;
    const int u = (pos & 7) ^ (row & 7);
    const int tok = min(m0 + row, p.m - 1);
    const uint32_t off = uint32_t(tok) * uint32_t(p.x_stride) * 2u + uint32_t(u) * 16u;
    copy16(xk + off, stage + (wave * kXCopies + d) * 1024);
  }
}

template <int N>
__device__ __forceinline__ void wait_lgkm() {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  __builtin_amdgcn_s_waitcnt(0xC07F | (N << 8));  // lgkmcnt(N) only
}

// z producers: the launch's first mtiles * zparts workgroups. The tokens of
// M-tile mt routed to live slots are sorted by slot (counting sort in LDS)
// and cut into units of up to 16 tokens of one slot; producer (mt, q) takes
// units q, q + zparts, ... For a unit it contracts just those tokens with the
// slices * r rows of A_g, 64 rows (four 16-row tiles) per pass: the eight
// waves take interleaved 32-wide k steps (v_mfma_f32_16x16x32_bf16, A rows as
// the A operand, the tokens' x as the B operand, four steps of loads in
// flight), the partial tiles meet in LDS in a fixed order, and
// z = bf16(x A_g^T) is stored in the slice-padded layout zpad[t][s * 64 + j]
// (zeros for r <= j < 64). Finally the producer sets its flag
// zflags[mt * zparts + q] to the call's tag. Work follows the routed tokens:
// a dense pass over the whole tile for every slot's rows would multiply the
// LoRA FLOPs by the number of slots in the tile (Zipf routing over 128
// adapters puts dozens in one tile).
// A device-coherent (sc1) 2-byte store: performed at the level the
// consumers' sc1 z loads read, so the producer needs no L2 write-back
// (release fence) before its flag, only a wait for its stores to complete.
__device__ __forceinline__ void store_z(uint16_t* dst, uint16_t v) {
  asm volatile("global_store_short %0, %1, off sc1" : : "v"(dst), "v"(uint32_t(v)) : "memory");
}

constexpr int kUnit = 16;        // tokens per unit
constexpr int kUnitRows = 64;    // A rows per pass
constexpr int kUnitSteps = 4;    // k steps of loads in flight per wave

__device__ void produce_units(const PrefillParams& p, int mt, int q, int* tslot, int* list, int* order, int* cnt,
                              int* ustart, float* red) {
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int c = lane & 15;
  const int kg = lane >> 4;
  constexpr int kWaves = kThreads / 64;
  const int m0 = mt * kBM;
  const int count = min(kBM, p.m - m0);
  const int zw = p.slices * kZSlice;
  const int steps = p.k / 32;
  live_slots(p, m0, count, tslot, list);
  const int nd = list[kMaxList];
  // Counting sort of the tile's live tokens by distinct slot index.
  for (int d = tid; d <= nd; d += kThreads) cnt[d] = 0;
  __syncthreads();
  // Every producer of the tile must cut the same units, so a token's place is
  // fixed: its slot's first position plus the number of earlier tokens of the
  // same slot (a broadcast scan of tslot, not an LDS atomic's arrival order).
  int my_d = -1, my_rank = 0;
  if (tid < count && tslot[tid] >= 0) {
    const int gt = tslot[tid];
    for (int d = 0; d < nd; ++d)
      if (list[d] == gt) my_d = d;
    for (int i = 0; i < tid; ++i) my_rank += tslot[i] == gt;
    atomicAdd(&cnt[my_d], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int pos = 0, units = 0;
    for (int d = 0; d < nd; ++d) {
      const int n = cnt[d];
      cnt[d] = pos;       // first position of slot d's tokens in `order`
      ustart[d] = units;  // first unit of slot d
      pos += n;
      units += (n + kUnit - 1) / kUnit;
    }
    cnt[nd] = pos;
    ustart[nd] = units;
  }
  __syncthreads();
  if (my_d >= 0) order[cnt[my_d] + my_rank] = tid;  // slot d holds positions cnt[d] .. cnt[d + 1]
  __syncthreads();
  // Zero the padding columns r .. 63 of every slice of the tokens this producer serves.
  const int units = ustart[nd];
  for (int u = q; u < units; u += p.zparts) {
    int d = 0;
    while (ustart[d + 1] <= u) ++d;
    const int first = cnt[d] + (u - ustart[d]) * kUnit;
    const int ntok = min(kUnit, cnt[d + 1] - first);
    const int r = p.ranks[list[d]];
    for (int i = tid; i < ntok * zw; i += kThreads) {
      const int t = i / zw;
      const int col = i - t * zw;
      if ((col & (kZSlice - 1)) >= r) store_z(p.zpad + int64_t(m0 + order[first + t]) * zw + col, 0);
    }
  }
  for (int u = q; u < units; u += p.zparts) {
    int d = 0;
    while (ustart[d + 1] <= u) ++d;
    const int first = cnt[d] + (u - ustart[d]) * kUnit;
    const int ntok = min(kUnit, cnt[d + 1] - first);
    const int gd = list[d];
    const int r = p.ranks[gd];
    const int rows = p.slices * r;
    const uint16_t* abase = p.a_store + p.a_offsets[gd];
    const int tok = m0 + order[first + min(c, ntok - 1)];
    const uint16_t* xrow = p.x + int64_t(tok) * p.x_stride + 8 * kg;
    for (int j0 = 0; j0 < rows; j0 += kUnitRows) {
      f32x4 acc[4];
#pragma unroll
      for (int jt = 0; jt < 4; ++jt) acc[jt] = (f32x4){0.f, 0.f, 0.f, 0.f};
      const int tiles = (min(kUnitRows, rows - j0) + 15) >> 4;  // uniform
      for (int s0 = wave; s0 < steps; s0 += kWaves * kUnitSteps) {
        // Loads of this batch's steps first (past the end: a readable step, not contracted).
        uint4 xb[kUnitSteps], ab[kUnitSteps][4];
#pragma unroll
        for (int v = 0; v < kUnitSteps; ++v) {
          const int st = min(s0 + v * kWaves, steps - 1);
          xb[v] = *reinterpret_cast<const uint4*>(xrow + st * 32);
#pragma unroll
          for (int jt = 0; jt < 4; ++jt)
            if (jt < tiles)
              ab[v][jt] = *reinterpret_cast<const uint4*>(abase + int64_t(min(j0 + jt * 16 + c, rows - 1)) * p.k +
                                                          st * 32 + 8 * kg);
        }
#pragma unroll
        for (int v = 0; v < kUnitSteps; ++v)
          if (s0 + v * kWaves < steps)
#pragma unroll
            for (int jt = 0; jt < 4; ++jt)
              if (jt < tiles) acc[jt] = mfma16(as_bf16x8(ab[v][jt]), as_bf16x8(xb[v]), acc[jt]);
      }
      // acc[jt][e] = this wave's partial of z[token c][A row j0 + 16 jt + 4 kg + e].
#pragma unroll
      for (int jt = 0; jt < 4; ++jt)
#pragma unroll
        for (int e = 0; e < 4; ++e) red[((wave * 4 + jt) * 16 + 4 * kg + e) * 17 + c] = acc[jt][e];
      __syncthreads();
      for (int o = tid; o < kUnitRows * kUnit; o += kThreads) {
        const int jr = o >> 4;  // A row within the pass
        const int t = o & 15;
        const int j = j0 + jr;
        if (t < ntok && j < rows) {
          float sum = 0.f;
#pragma unroll
          for (int w = 0; w < kWaves; ++w) sum += red[((w * 4 + (jr >> 4)) * 16 + (jr & 15)) * 17 + t];
          const int sl = j / r;
          store_z(p.zpad + int64_t(m0 + order[first + t]) * zw + sl * kZSlice + (j - sl * r), uint16_t(f32_to_bf16(sum)));
        }
      }
      __syncthreads();  // red is reused by the next pass
    }
  }
  // Every thread's z stores have completed (sc1: at device scope) when this
  // returns (asm with a memory clobber, so the compiler keeps later stores
  // after it).
  asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
  __syncthreads();
}

// Producer (mt, q): its units, then its flag carries the call's tag.
__device__ __forceinline__ void produce_z(const PrefillParams& p, int mt, int q, uint32_t tag, int* tslot, int* list,
                                          int* order, int* cnt, int* ustart, float* red) {
  if (p.withhold) return;  // test hook: the tile's consumers must recompute
  produce_units(p, mt, q, tslot, list, order, cnt, ustart, red);
  if (threadIdx.x == 0) __hip_atomic_store(p.zflags + mt * p.zparts + q, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Waits until the z rows of M-tile mt carry the call's tag (their producers
// have lower block ids, so they were dispatched before this workgroup).
// The flags and the z rows are read with device-scope loads (coherent past
// the caches of this CU and XCD), so no acquire fence is needed: an acquire
// at device scope would invalidate the whole L2 of the XCD under the other
// workgroups' feet. Each wait is bounded (about a quarter second); a
// producer that has not set its flag by then has its units recomputed here
// (same arithmetic, so the same z bits), the status word records it, and the
// tile's slot metadata, whose LDS the recomputation borrowed, is reloaded.
// Returns whether it recomputed anything.
__device__ bool wait_z(const PrefillParams& p, int mt, uint32_t tag, int* tslot, int* list, int* order, int* mrank,
                       int* mstride, float* mscale, int64_t* mboff, float* red, uint32_t* missing) {
  if (threadIdx.x < 2) missing[threadIdx.x] = 0;
  __syncthreads();
  if (threadIdx.x < p.zparts) {
    const uint32_t* flag = p.zflags + mt * p.zparts + threadIdx.x;
    for (int spins = 0; __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != tag; ++spins) {
      if (spins > p.spin_limit) {
        atomicOr(&missing[threadIdx.x >> 5], 1u << (threadIdx.x & 31));
        break;
      }
      __builtin_amdgcn_s_sleep(8);
    }
  }
  __syncthreads();
  const uint64_t lost = uint64_t(missing[0]) | (uint64_t(missing[1]) << 32);
  if (lost == 0) return false;
  if (threadIdx.x == 0) __hip_atomic_store(p.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (int q = 0; q < p.zparts; ++q)
    if ((lost >> q) & 1) produce_units(p, mt, q, tslot, list, order, mrank, mstride, red);
  for (int d = threadIdx.x; d < list[kMaxList]; d += blockDim.x) {
    const int gg = list[d];
    mrank[d] = p.ranks[gg];
    mstride[d] = p.b_strides[gg];
    mscale[d] = p.lscales[gg];
    mboff[d] = p.b_offsets[gg];
  }
  __syncthreads();
  return true;
}

// 16 bytes of z rows in one device-scope (sc1) load, coherent past this
// XCD's L2 like the agent-scope atomics; one request instead of four.
// Untracked: the caller waits (vmcnt) and ties the value before any use.
__device__ __forceinline__ u32x4 load_z16(const uint16_t* src) {
  u32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, off sc1" : "=v"(v) : "v"(src) : "memory");
  return v;
}

// Counts the workgroup in; the last one moves the epoch on (call_epoch.h).
__device__ __forceinline__ void depart(const PrefillParams& p, uint32_t tag) {
  if (threadIdx.x < 64) {
    const uint32_t old = depart_issue(p.ce, threadIdx.x);
    depart_finish(p.ce, old, tag - 1u, threadIdx.x);
  }
}

// bf16 rounding of the contraction, then of the bias add:
// acc[i][j][e] holds feature wn0 + 16j + 4g + e.
__device__ __forceinline__ void round_bias(const PrefillParams& p, f32x4 (&acc)[8][kJ], int wn0, int g) {
#pragma unroll
  for (int j = 0; j < kJ; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int n = wn0 + j * 16 + 4 * g + e;
      const float bias = (p.bias && n < p.n) ? bf16_to_f32(p.bias[n]) : 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float v = round_bf16(acc[i][j][e]);
        if (p.bias) v = round_bf16(v + bias);
        acc[i][j][e] = v;
      }
    }
}

// Weight row of tile row r (0 .. kBN - 1) in column tile nt. SwiGLU output:
// tile nt produces activation columns kBN/2 nt .. + kBN/2; its rows below
// kBN/2 are the gate rows of those columns, the others the matching up rows
// (n / 2 further on), so a wave's 48 rows stay contiguous.
template <bool kSwiglu>
__device__ __forceinline__ int tile_row(const PrefillParams& p, int nt, int r) {
  if constexpr (!kSwiglu) return nt * kBN + r;
  constexpr int kHalf = kBN / 2;
  return r < kHalf ? nt * kHalf + r : (p.n >> 1) + nt * kHalf + (r - kHalf);
}

// Block ids below mtiles * zparts (LoRA launches only) produce the tiles' z
// rows; the others are GEMM tiles, M-tile b % mtiles on consecutive ids.
template <bool kLora, bool kSwiglu>
__global__ __launch_bounds__(kThreads) void gemm_kernel(PrefillParams p) {
  __shared__ __attribute__((aligned(16))) char xring[kXD * kXBytes];
  __shared__ __attribute__((aligned(16))) uint4 wdec[2][kBN * 8];
  __shared__ __attribute__((aligned(2048))) float table[512];  // [byte] -> (code[byte >> 4], code[byte & 15])
  __shared__ __attribute__((aligned(16))) int tslot[kLora ? kBM : 1];
  __shared__ int list[kLora ? kMaxList + 1 : 1];
  __shared__ int order[kLora ? kBM : 1];  // z producer: tile rows sorted by slot
  __shared__ uint32_t zmissing[2];        // producers of the tile whose flag never came
  __shared__ int mrank[kLora ? kMaxList + 1 : 1];
  __shared__ int mstride[kLora ? kMaxList + 1 : 1];
  __shared__ float mscale[kLora ? kMaxList : 1];
  __shared__ int64_t mboff[kLora ? kMaxList : 1];
  const int tid = threadIdx.x;
  int b = blockIdx.x;
  uint32_t tag = 0;
  if constexpr (kLora) {
    tag = __builtin_amdgcn_readfirstlane(epoch_tag(p.ce));
    if (b < p.mtiles * p.zparts) {
      // (The slot metadata arrays double as the producer's sort counters; the
      // idle x ring holds the partial tiles.)
      produce_z(p, b / p.zparts, b % p.zparts, tag, tslot, list, order, mrank, mstride, reinterpret_cast<float*>(xring));
      depart(p, tag);
      return;
    }
    b -= p.mtiles * p.zparts;
  }
  const int mt = b % p.mtiles;
  const int nt = b / p.mtiles;
  const int m0 = mt * kBM;
  const int n0 = nt * kBN;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int wm = wave & 1;
  const int wn = wave >> 1;
  const int c = lane & 15;
  const int g = lane >> 4;
  const int nk = p.k / kBK;

  WLane wl;
#pragma unroll
  for (int i = 0; i < kDw; ++i) {
    const int nrow = min(tile_row<kSwiglu>(p, nt, (tid >> 3) + 64 * i), p.n - 1);
    wl.qoff[i] = uint32_t(int64_t(nrow) * (p.k >> 1) + (tid & 7) * 4);
    wl.soff[i] = uint32_t(int64_t(nrow) * (p.k / kNf4Block) * 4);
  }

  // Prologue in the loop's request order: W(0), x(0), W(1), x(1) (a single
  // step requests step 0 twice).
  Packed wa, wb;
  issue_w(p, 0, wl, wb);
  issue_x(p, xring, m0, 0, wave, lane);
  issue_w(p, min(1, nk - 1), wl, wa);
  issue_x(p, xring + kXBytes, m0, min(1, nk - 1), wave, lane);
  table[tid] = sload(p.code, (tid & 1) ? (tid >> 1) & 15 : tid >> 5);
  __syncthreads();  // codebook staged
  const uint32_t table_addr = lds_addr(table);
  // Decoded-W store address of this lane (slot 0): row tid >> 3, unit tid & 7.
  const uint32_t wdst = lds_addr(wdec) + uint32_t((tid >> 3) * 128 + (((tid & 7) ^ ((tid >> 3) & 7)) << 4));
  constexpr int kW = Packed::kLoads;
  wait_vm<kW + 2 * kXCopies>();
  tie_w(wb);
  {
    LookAddr la;
    Looked lk;
    lookup_addresses(wb, table_addr, la);
#pragma unroll
    for (int i = 0; i < kDw; ++i) lookup_dword(la, i, lk);
    wait_lgkm<0>();
    tie_lookups(lk);
    decode_store(wb, lk, wdst);
  }
  wait_vm<kW + kXCopies>();
  lds_barrier();
  if constexpr (kLora) {
    // The tile's routes and slot metadata, ahead of the k-loop.
    live_slots(p, m0, min(kBM, p.m - m0), tslot, list);
    for (int d = tid; d < list[kMaxList]; d += kThreads) {
      const int gg = list[d];
      mrank[d] = p.ranks[gg];
      mstride[d] = p.b_strides[gg];
      mscale[d] = p.lscales[gg];
      mboff[d] = p.b_offsets[gg];
    }
  }

  f32x4 acc[8][kJ];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < kJ; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // Fragment addresses (stage 0) for k halves 0 and 1. Rows of a lane differ
  // by multiples of 16, so its fragments share the swizzle (row & 7) = (c & 7)
  // and differ by immediate offsets.
  const uint32_t xa0 = lds_addr(xring) + uint32_t((wm * 128 + c) * 128 + ((g ^ (c & 7)) << 4));
  const uint32_t xa1 = lds_addr(xring) + uint32_t((wm * 128 + c) * 128 + (((4 + g) ^ (c & 7)) << 4));
  const uint32_t wa0 = lds_addr(wdec) + uint32_t((wn * 48 + c) * 128 + ((g ^ (c & 7)) << 4));
  const uint32_t wa1 = lds_addr(wdec) + uint32_t((wn * 48 + c) * 128 + (((4 + g) ^ (c & 7)) << 4));

  // Fragment reads: k half h of stage kt (x ring slot kt % 3, decoded-W
  // slot kt & 1); 8 A and kJ B reads of 16 bytes, untracked.
  auto read_half = [&](int kt, int h, u32x4 (&a)[8], u32x4 (&b)[kJ]) {
    const uint32_t ax = (h ? xa1 : xa0) + uint32_t((kt % kXD) * kXBytes);
    const uint32_t bx = (h ? wa1 : wa0) + uint32_t((kt & 1) * kWBytes);
    a[0] = ldsr128<0 * 2048>(ax);
    a[1] = ldsr128<1 * 2048>(ax);
    a[2] = ldsr128<2 * 2048>(ax);
    a[3] = ldsr128<3 * 2048>(ax);
    a[4] = ldsr128<4 * 2048>(ax);
    a[5] = ldsr128<5 * 2048>(ax);
    a[6] = ldsr128<6 * 2048>(ax);
    a[7] = ldsr128<7 * 2048>(ax);
    b[0] = ldsr128<0 * 2048>(bx);
    b[1] = ldsr128<1 * 2048>(bx);
    b[2] = ldsr128<2 * 2048>(bx);
  };
  constexpr int kHalfReads = 8 + kJ;

  // One k-step, entered with the k-half-0 fragments of stage kt requested:
  // request step kt + 2 (W into `ld`; past the end the last step again, into
  // buffers nothing reads), decode W(kt + 1) from `dec` into the other
  // decoded-W slot over the k-half-0 MFMAs, meet the other waves once x(kt + 1)
  // landed, then request the next step's k-half-0 fragments and contract
  // k half 1.
  u32x4 a0[8], b0[kJ];
  read_half(0, 0, a0, b0);
  auto step = [&](int kt, Packed& dec, Packed& ld) {
    const int kr = min(kt + 2, nk - 1);
    issue_w(p, kr, wl, ld);
    issue_x(p, xring + ((kt + 2) % kXD) * kXBytes, m0, kr, wave, lane);
    u32x4 a1[8], b1[kJ];
    // W(kt + 1) was requested before x(kt + 1) and this step's requests.
    wait_vm<kW + 2 * kXCopies>();
    tie_w(dec);
    LookAddr la;
    lookup_addresses(dec, table_addr, la);
    wait_lgkm<0>();  // the k-half-0 fragments
#pragma unroll
    for (int i = 0; i < 8; ++i) tie(a0[i]);
#pragma unroll
    for (int j = 0; j < kJ; ++j) tie(b0[j]);
    __builtin_amdgcn_sched_barrier(0);
    // The lookups between the first k-half-0 MFMAs, then the k-half-1
    // fragment reads (queued behind the lookups; the barrier completes them).
    Looked lk;
#pragma unroll
    for (int i = 0; i < kDw; ++i) {
      lookup_dword(la, i, lk);
#pragma unroll
      for (int j = 0; j < kJ; ++j) acc[i][j] = mfma16(vec_bf16x8(b0[j]), vec_bf16x8(a0[i]), acc[i][j]);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int j = 0; j < kJ; ++j) acc[kDw][j] = mfma16(vec_bf16x8(b0[j]), vec_bf16x8(a0[kDw]), acc[kDw][j]);
    read_half(kt, 1, a1, b1);
    __builtin_amdgcn_sched_barrier(0);
    wait_lgkm<kHalfReads>();  // the lookups
    tie_lookups(lk);
#pragma unroll
    for (int i = kDw + 1; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < kJ; ++j) acc[i][j] = mfma16(vec_bf16x8(b0[j]), vec_bf16x8(a0[i]), acc[i][j]);
    decode_store(dec, lk, wdst + uint32_t(((kt + 1) & 1) * kWBytes));
#pragma unroll
    for (int q = 0; q < (8 - kDw - 1) * kJ; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // three VALU
    }
    __builtin_amdgcn_sched_barrier(0);
    // x(kt + 1) has landed once at most this step's requests are outstanding;
    // the barrier publishes it with the decoded W(kt + 1), completes this
    // wave's k-half-1 fragment reads and frees the slots read at kt - 1 for
    // the requests of step kt + 1.
    wait_vm<kW + kXCopies>();
    lds_barrier();
#pragma unroll
    for (int i = 0; i < 8; ++i) tie(a1[i]);
#pragma unroll
    for (int j = 0; j < kJ; ++j) tie(b1[j]);
    read_half(kt + 1, 0, a0, b0);
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < kJ; ++j) acc[i][j] = mfma16(vec_bf16x8(b1[j]), vec_bf16x8(a1[i]), acc[i][j]);
  };
  for (int kt = 0; kt < nk; kt += 2) {
    step(kt, wa, wb);
    if (kt + 1 < nk) step(kt + 1, wb, wa);
  }
  wait_lgkm<0>();  // the fragment reads past the end
  wait_vm<0>();  // the requests past the end

  // ---- epilogue: acc[i][j][e] = C[token m0 + wm*128 + 16i + c][feature n0 + wn*48 + 16j + 4g + e]
  // (W is the MFMA's A operand, so a lane holds four consecutive features of
  // one token: one 8-byte store per fragment).
  const int wn0 = tile_row<kSwiglu>(p, nt, wn * 48);
  if constexpr (kLora) {
    // z rows of slice 0 and the B fragments of the first slot are requested
    // before the base rounding, so their latency overlaps it.
    const int nd = list[kMaxList];
    const int zw = p.slices * kZSlice;
    constexpr int kZq = kBM * 8 / kThreads;  // 16-byte z units per thread and slice
    u32x4 zr[kZq];
    // Every lane loads (rows past M read row M - 1, base-only rows are
    // zeroed after the wait): no branch around the untracked loads.
    auto load_zs = [&](int s) {
#pragma unroll
      for (int q = 0; q < kZq; ++q) {
        const int row = min(m0 + (tid >> 3) + (kThreads / 8) * q, p.m - 1);
        zr[q] = load_z16(p.zpad + int64_t(row) * zw + s * kZSlice + (tid & 7) * 8);
      }
    };
    // B fragments of slot d as the MFMA's A operand: feature wn0 + 16j + c,
    // k-group g of ranks 0..31 (b0) and 32..63 (b1). Requested raw from
    // clamped, readable places (a select on a load result would wait for it)
    // and masked where used: past the row stride or the rank, and past N.
    auto request_b = [&](int d, uint4 (&b0)[kJ], uint4 (&b1)[kJ]) {
      const int br = mstride[d];
      const uint16_t* bg = p.b_store + mboff[d];
      const bool two = mrank[d] > 32;
#pragma unroll
      for (int j = 0; j < kJ; ++j) {
        const uint16_t* row = bg + int64_t(min(wn0 + j * 16 + c, p.n - 1)) * br;
        b0[j] = b_raw(row, br, g * 8);
        if (two) b1[j] = b_raw(row, br, 32 + g * 8);
      }
    };
    auto b_frag = [&](const uint4& raw, int d, int kk, int j) {
      const int keep = (wn0 + j * 16 + c < p.n) ? min(mstride[d], mrank[d]) - kk : 0;
      return as_bf16x8(keep_first(raw, keep));
    };
    // Routes of this lane's eight tokens.
    int rslot[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) rslot[i] = tslot[wm * 128 + i * 16 + c];
    // The next distinct slot after d taken by any of this wave's tokens (nd: none).
    auto next_live = [&](int d) {
      for (++d; d < nd; ++d) {
        const int gd = list[d];
        bool any = false;
#pragma unroll
        for (int i = 0; i < 8; ++i) any |= rslot[i] == gd;
        if (__ballot(any) != 0) break;
      }
      return d;
    };
    const int first = next_live(-1);
    // B of the slot being applied (index 0) and of the next kAhead live slots,
    // requested that far ahead: with dozens of slots in a tile (retained-rank
    // batches under Zipf routing) each slot would otherwise cost one memory
    // round trip.
    constexpr int kAhead = 2;
    int dq[kAhead + 1];
    uint4 bq0[kAhead + 1][kJ], bq1[kAhead + 1][kJ];
    wait_z(p, mt, tag, tslot, list, order, mrank, mstride, mscale, mboff, reinterpret_cast<float*>(xring), zmissing);
    // Every slice's z rows are staged at once (slice s at unit s * kBM * 8 of
    // the idle x ring: [token][8 units] with the x swizzle), so after one
    // barrier each wave applies exactly the slices its 48 columns touch,
    // without waiting at a barrier through the expand of a slice it does not
    // take (a SwiGLU tile's gate and up waves take different slices).
    static_assert(3 * kBM * 8 * 16 <= kXD * kXBytes, "the z rows of three slices (the most a call has) fit the x ring");
    uint4* zs_all = reinterpret_cast<uint4*>(xring);
    for (int s = 0; s < p.slices; ++s) {
      // The slice's z rows (the one place these untracked loads are made), and
      // with slice 0 the first slot's B, requested before the base rounding.
      load_zs(s);
      if (s == 0) {
        if (first < nd) request_b(first, bq0[0], bq1[0]);
        round_bias(p, acc, wn0, g);
      }
      wait_vm<0>();  // the z loads (and anything requested after them)
#pragma unroll
      for (int q = 0; q < kZq; ++q) tie(zr[q]);
#pragma unroll
      for (int q = 0; q < kZq; ++q) {
        const int row = (tid >> 3) + (kThreads / 8) * q;
        zs_all[s * kBM * 8 + swz(row, tid & 7)] =
            tslot[row] >= 0 ? make_uint4(zr[q].x, zr[q].y, zr[q].z, zr[q].w) : make_uint4(0, 0, 0, 0);
      }
    }
    __syncthreads();
    bool b_first_ready = true;  // the B of `first` requested above is still unused
    for (int s = 0; s < p.slices; ++s) {
      const int lo = p.slice_offsets[s];
      const int hi = p.slice_offsets[s + 1];
      if (hi <= wn0 || lo >= wn0 + 48) continue;  // this wave's 48 columns miss the slice
      const bool inside = lo <= wn0 && wn0 + 48 <= hi;
      const uint4* zs = zs_all + s * kBM * 8;
      // delta[n][m] = sum_j B_g[n][j] z[m][j] for the wave's 128 tokens x 48
      // features, added with the reference's two roundings to the tokens
      // routed to g and the features of slice s. The B of the next kAhead
      // live slots is in flight while this slot's MFMAs run.
      if (!b_first_ready && first < nd) request_b(first, bq0[0], bq1[0]);
      b_first_ready = false;
      dq[0] = first;
#pragma unroll
      for (int a = 1; a <= kAhead; ++a) {
        dq[a] = dq[a - 1] < nd ? next_live(dq[a - 1]) : nd;
        if (dq[a] < nd) request_b(dq[a], bq0[a], bq1[a]);
      }
      while (dq[0] < nd) {
        const int d = dq[0];
        const int gd = list[d];
        const bool two = mrank[d] > 32;
        const float scale = mscale[d];
        bf16x8 l0[kJ], l1[kJ];
#pragma unroll
        for (int j = 0; j < kJ; ++j) {
          l0[j] = b_frag(bq0[0][j], d, g * 8, j);
          l1[j] = two ? b_frag(bq1[0][j], d, 32 + g * 8, j) : as_bf16x8(make_uint4(0, 0, 0, 0));
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const bool mine = rslot[i] == gd;
          if (__ballot(mine) == 0) continue;  // no token of this 16-row block takes gd
          const int arow = wm * 128 + i * 16 + c;
          const bf16x8 z0 = as_bf16x8(zs[swz(arow, g)]);
          const bf16x8 z1 = as_bf16x8(zs[swz(arow, 4 + g)]);
#pragma unroll
          for (int j = 0; j < kJ; ++j) {
            f32x4 dacc = {0.f, 0.f, 0.f, 0.f};
            dacc = mfma16(l0[j], z0, dacc);
            if (two) dacc = mfma16(l1[j], z1, dacc);
            if (!mine) continue;
            // bf16(scale * delta) for the four features at once; the sum with
            // the rounded base is rounded once more by the output store.
            const uint32_t t01 = pack_bf16x2(dacc[0] * scale, dacc[1] * scale);
            const uint32_t t23 = pack_bf16x2(dacc[2] * scale, dacc[3] * scale);
            const float t[4] = {bf16_lo(t01), bf16_hi(t01), bf16_lo(t23), bf16_hi(t23)};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int n = wn0 + j * 16 + 4 * g + e;
              if (inside || (n >= lo && n < hi)) acc[i][j][e] += t[e];
            }
          }
        }
        // Rotate, then request the slot kAhead places on.
#pragma unroll
        for (int a = 0; a < kAhead; ++a) {
          dq[a] = dq[a + 1];
#pragma unroll
          for (int j = 0; j < kJ; ++j) {
            bq0[a][j] = bq0[a + 1][j];
            bq1[a][j] = bq1[a + 1][j];
          }
        }
        dq[kAhead] = dq[kAhead - 1] < nd ? next_live(dq[kAhead - 1]) : nd;
        if (dq[kAhead] < nd) request_b(dq[kAhead], bq0[kAhead], bq1[kAhead]);
      }
    }
  } else {
    round_bias(p, acc, wn0, g);
  }
  if (kSwiglu || p.y_vec == 2) {
    // 16-byte aligned rows (always so with the SwiGLU output): the tile goes through LDS (the idle x ring, rows
    // of 384 bytes, 16-byte chunks XOR-swizzled by row & 7) and leaves as
    // whole rows, so each 128-byte line of y is written by one request.
    static_assert(kBN * 2 == 384 && kBM * 384 <= kXD * kXBytes, "output staging fits the x ring");
    __syncthreads();  // every wave is done with the ring
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = wm * 128 + i * 16 + c;
#pragma unroll
      for (int j = 0; j < kJ; ++j) {
        const int q = wn * 6 + 2 * j + (g >> 1);  // 16-byte chunk of the row
        const uint32_t lo = pack_bf16x2(acc[i][j][0], acc[i][j][1]);
        const uint32_t hi = pack_bf16x2(acc[i][j][2], acc[i][j][3]);
        *reinterpret_cast<uint2*>(xring + row * 384 + ((q ^ (row & 7)) << 4) + (g & 1) * 8) = make_uint2(lo, hi);
      }
    }
    __syncthreads();
    if constexpr (kSwiglu) {
      // Activation chunk q (8 columns) of a row: gate chunk q and up chunk
      // q + 12 of the staged row, bf16(bf16(silu(g)) * u) as lf_swiglu.
#pragma unroll
      for (int r = 0; r < kBM * 12 / kThreads; ++r) {
        const int id = tid + r * kThreads;
        const int row = id / 12;
        const int q = id - row * 12;
        const int m = m0 + row;
        const int n = nt * (kBN / 2) + q * 8;
        if (m < p.m && n < (p.n >> 1)) {
          const uint4 gv = *reinterpret_cast<const uint4*>(xring + row * 384 + ((q ^ (row & 7)) << 4));
          const uint4 uv = *reinterpret_cast<const uint4*>(xring + row * 384 + (((q + 12) ^ (row & 7)) << 4));
          const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
          const uint32_t uw[4] = {uv.x, uv.y, uv.z, uv.w};
          uint32_t o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            o[e] = pack_bf16x2(silu_times(bf16_lo(gw[e]), bf16_lo(uw[e])),
                               silu_times(bf16_hi(gw[e]), bf16_hi(uw[e])));
          *reinterpret_cast<uint4*>(p.y + int64_t(m) * p.y_stride + n) = make_uint4(o[0], o[1], o[2], o[3]);
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < kBM * 24 / kThreads; ++r) {
        const int id = tid + r * kThreads;
        const int row = id / 24;
        const int q = id - row * 24;
        const int m = m0 + row;
        const int n = n0 + q * 8;
        if (m < p.m && n < p.n)
          *reinterpret_cast<uint4*>(p.y + int64_t(m) * p.y_stride + n) =
              *reinterpret_cast<const uint4*>(xring + row * 384 + ((q ^ (row & 7)) << 4));
      }
    }
  } else if constexpr (!kSwiglu) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int m = m0 + wm * 128 + i * 16 + c;
      if (m >= p.m) continue;
#pragma unroll
      for (int j = 0; j < kJ; ++j) {
        const int n = wn0 + j * 16 + 4 * g;  // N % 64 == 0: n < N covers n + 3
        if (n >= p.n) continue;
        uint16_t* dst = p.y + int64_t(m) * p.y_stride + n;
        const uint32_t lo = pack_bf16x2(acc[i][j][0], acc[i][j][1]);
        const uint32_t hi = pack_bf16x2(acc[i][j][2], acc[i][j][3]);
        if (p.y_vec) {
          *reinterpret_cast<uint2*>(dst) = make_uint2(lo, hi);
        } else {
          dst[0] = uint16_t(lo);
          dst[1] = uint16_t(lo >> 16);
          dst[2] = uint16_t(hi);
          dst[3] = uint16_t(hi >> 16);
        }
      }
    }
  }
  if constexpr (kLora) depart(p, tag);
}

}  // namespace wide

}  // namespace

namespace {
int64_t align256(int64_t v) { return (v + 255) / 256 * 256; }
}  // namespace

int device_cus();

// Workspace: the control header (call epoch), the z flags (one per producer,
// zparts per 256-token tile) at a fixed place (so a flag word only ever holds
// tags, whatever the shapes of earlier calls on the workspace), the z rows
// (m x slices x 64 bf16), then room for the fp32 block scales of a
// double-quant weight.
constexpr int64_t kMaxFlags = kFlagRegion / 4;
constexpr int kMaxZParts = 64;

// z producers per M-tile. Producers run first and hold a CU each (one
// workgroup per CU), so they take CUs from the GEMM tiles, except where the
// tiles' last round leaves CUs idle anyway: c5's 464 tiles on 256 CUs leave 48
// idle in the second round, and 48 producers that start on those CUs delay no
// tile, while 128 producers of one unit each (16 tokens) held half the CUs
// for the first 22 us. So the producers fill the last round's slack (at most
// 64 per tile, within the flag region), and never fall below 4 per tile, so
// that no producer has more than a few units (each about 11 us at c5's
// shape) to finish before its tile's consumers reach their epilogue.
constexpr int kMinZParts = 4;
int zparts_for(int64_t mtiles, int64_t tiles, int64_t cus) {
  const int64_t rem = tiles % cus;
  const int64_t slack = rem == 0 ? 0 : cus - rem;
  const int64_t most = std::min<int64_t>(kMaxZParts, kMaxFlags / mtiles);
  return int(std::max<int64_t>(1, std::min<int64_t>(most, std::max<int64_t>(kMinZParts, slack / mtiles))));
}

int64_t prefill_workspace_bytes(int64_t m, int64_t n, int64_t k, int slices, int) {
  return kWorkspaceHeader + kFlagRegion + align256(m * slices * kZSlice * 2) + align256(n * (k / kNf4Block) * 4);
}

int launch_nf4_lora_prefill(const uint16_t* x, int64_t m, int64_t x_stride, const lf_nf4_weight* w,
                            const uint16_t* bias, const lf_lora* lora, uint16_t* y, int64_t y_stride,
                            void* workspace, int64_t workspace_bytes, bool swiglu, bool withhold, void* stream) {
  const int slices = lora ? lora->num_slices : 1;
  const bool dq = w->scales == nullptr;
  const int64_t need = prefill_workspace_bytes(m, w->n, w->k, slices, lora ? lora->max_rank : 1);
  LF_REQUIRE(!(lora || dq) || (workspace && workspace_bytes >= need && aligned16(workspace)),
             "workspace too small: need %lld bytes", (long long)need);
  LF_REQUIRE((m - 1) * x_stride * 2 + w->k * 2 < (int64_t(1) << 32), "x spans 4 GiB or more");
  LF_REQUIRE((m + wide::kBM - 1) / wide::kBM <= kMaxFlags, "prefill handles at most %lld tokens per call",
             (long long)(kMaxFlags * wide::kBM));
  auto s = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  const float* scales = w->scales;
  if (dq) {
    // The GEMM streams fp32 block scales: rebuild them from the nested state
    // (the same reconstruction as the dequantisation kernel) after the z rows.
    const int64_t nblocks = w->n * (w->k / kNf4Block);
    float* rebuilt =
        reinterpret_cast<float*>(ws + kWorkspaceHeader + kFlagRegion + align256(m * slices * kZSlice * 2));
    const int rc = lf_nf4_prepare_scales_dq(w->absmax_q, w->absmax2, w->code2, w->offset, w->dq_block, rebuilt,
                                            nblocks, stream);
    if (rc != kOk) return rc;
    scales = rebuilt;
  }
  PrefillParams p{};
  p.x = x;
  p.x_stride = x_stride;
  p.m = int(m);
  p.q = w->qweight;
  p.src = ScaleSource{scales, nullptr, nullptr, nullptr, nullptr, 1};
  p.code = w->code;
  p.n = int(w->n);
  p.k = int(w->k);
  p.bias = bias;
  p.y = y;
  p.y_stride = y_stride;
  p.y_vec = (y_stride % 8 == 0 && (reinterpret_cast<uintptr_t>(y) & 15u) == 0) ? 2
            : (y_stride % 4 == 0 && (reinterpret_cast<uintptr_t>(y) & 7u) == 0)  ? 1
                                                                                 : 0;
  p.slices = slices;
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
    LF_REQUIRE(lora->num_slots >= 0, "num_slots must not be negative");
    p.num_slots = lora->num_slots;
    p.zflags = reinterpret_cast<uint32_t*>(ws + kWorkspaceHeader);  // after the decode header
    p.zpad = reinterpret_cast<uint16_t*>(ws + kWorkspaceHeader + kFlagRegion);
    p.ce = call_epoch_of(ws);
    p.status = reinterpret_cast<int*>(ws + kStatusOffset);
  }
  p.withhold = withhold ? 1 : 0;
  p.spin_limit = withhold ? 64 : (1 << 20);
  p.mtiles = int((m + wide::kBM - 1) / wide::kBM);
  // SwiGLU output: each tile takes kBN / 2 activation columns (their gate and
  // up rows) and stores 16-byte chunks of them.
  LF_REQUIRE(!swiglu || p.y_vec == 2, "prefill SwiGLU output needs y 16-byte aligned with row stride %% 8 == 0");
  const int64_t cols = swiglu ? w->n / 2 : w->n;
  const int64_t bn = swiglu ? wide::kBN / 2 : wide::kBN;
  const int64_t tiles = p.mtiles * ((cols + bn - 1) / bn);
  p.zparts = zparts_for(p.mtiles, tiles, device_cus());
  // LoRA launches put the z producers ahead of the GEMM tiles.
  const dim3 grid(unsigned(tiles + (lora ? p.mtiles * p.zparts : 0)));
  if (swiglu) {
    if (lora) hipLaunchKernelGGL((wide::gemm_kernel<true, true>), grid, dim3(wide::kThreads), 0, s, p);
    else hipLaunchKernelGGL((wide::gemm_kernel<false, true>), grid, dim3(wide::kThreads), 0, s, p);
  } else {
    if (lora) hipLaunchKernelGGL((wide::gemm_kernel<true, false>), grid, dim3(wide::kThreads), 0, s, p);
    else hipLaunchKernelGGL((wide::gemm_kernel<false, false>), grid, dim3(wide::kThreads), 0, s, p);
  }
  LF_HIP(hipGetLastError());
  return kOk;
}

}  // namespace lf
