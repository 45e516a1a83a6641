// LoRA machinery shared by the decode kernels (nf4_gemv.hip, the narrow
// tiles up to 32 tokens and the residual form; nf4_decode_wide.hip, 32 rows x
// 32 tokens per workgroup over any batch): launch parameters, the shrink
// units with their tagged partials, the tile metadata, the z gather with its
// bounded waits and recompute, the B fragment helpers and the host-side plan.
#pragma once

#include <algorithm>
#include <type_traits>

#include "call_epoch.h"
#include "dq_scales.h"
#include "lds_pipeline.h"
#include "nf4_common.h"
#include "../../include/loraforge_amd.h"

namespace lf {
namespace {

// Global output row of local row j (0 .. R - 1) of a row group whose first
// R / 2 rows start at lo and the others at hi (hi = lo + R / 2 for a plain
// group; in SwiGLU-output mode lo is the group's first gate row and hi the
// matching up row, hi = lo + n / 2).
template <class TL>
__device__ __forceinline__ int grow(int lo, int hi, int j) {
  return j < TL::kR / 2 ? lo + j : hi + (j - TL::kR / 2);
}

struct GemvParams {
  const uint16_t* x;
  int64_t x_stride;
  int m;
  const uint8_t* q;
  const float* scales;
  const float* code;
  int n;
  int k;
  const uint16_t* bias;
  uint16_t* y;
  int64_t y_stride;
  int row_groups;  // n / R
  int tiles;       // wide kernel: 32-token tiles (ceil(m / 32))
  int gated_half;  // SwiGLU output: n / 2 (a group's rows: R / 2 gate rows and the matching up rows), else 0
  int sc_stride;  // floats per row of a wave's scale area (narrow kScPre tiles: odd; wide: a power of two)
  int sc_bytes;   // bytes of a wave's scale area in dynamic LDS (multiple of 256)
  uint32_t sc_magic;  // ceil(2^32 / sc_stride): pos / sc_stride as a high multiply (pos < 2^16; stride > 1)
  // Double-quant block scales (absmax_q non-null, scales null): each base wave
  // stages them into its scale area and converts them there (dq_scales.h).
  const uint8_t* absmax_q;
  const float* absmax2;
  const float* code2;
  const float* dq_offset;
  int dq_shift;   // log2(dq_block)
  int a2_len;     // entries of absmax2
  // LoRA (kLora variants only).
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
  int num_slots;  // entries of the per-slot arrays (0: not given)
  int zw;         // z row width: slices * max_rank
  int units;      // shrink units: m * usplit * kz
  int kz;         // k-slices per token
  int usplit;     // row ranges per token (unit u: token u / (usplit * kz), range (u / kz) % usplit, k-slice u % kz)
  int urows;      // A rows per range (a multiple of 16)
  uint32_t unit_inv;  // ceil(2^21 / (usplit * kz)): u / (usplit * kz) by a multiply (u <= 1024)
  int kz_len;     // k per slice (multiple of 64)
  int producers;  // workgroups b < producers make units b, b + producers, ...
  int resident;   // workgroups of the first dispatch round (b < resident run beside the producers)
  int contract_after;  // (wide kernel) the loop block after which producing waves contract their first unit
  int* status;    // set to 1 when a bounded wait for partials gave up (they were then recomputed)
  int spin_limit; // polls of a bounded wait for partials
  int withhold;   // test hook: producers publish nothing, so every wait gives up and recomputes
  CallEpoch ce;      // call tag: epoch + 1, moved on by the last workgroup
  uint64_t* zp;      // [units][zw] shrink partial sums as (tag << 32) | fp32 bits
};

constexpr int kSpinLimit = 1 << 20;

// ---------------------------------------------------------------------------
// LoRA (the last wave of every workgroup is the LoRA wave).
//
// Shrink: unit u = (token t, row range, k-slice) is computed early in
// workgroup u % producers: the contraction waves contract x[t] with the
// range's rows (up to urows of the slices * r rows of the token's adapter
// A_g) over the slice (MFMA, the token in row 0); a token of high rank is
// split over several units so that no producer streams a whole rank-64 A
// while the others wait; the LoRA wave sums their partial rows
// and stores zp[u][j] with device-scope 64-bit stores, each value paired
// with the call's tag. The fragments of a workgroup's first unit are
// requested between its first and second weight stages, so they are not
// queued behind the whole prologue.
// Call tag (call_epoch.h): every workgroup reads the epoch at its start and
// the LoRA wave counts the workgroup in when its work is done. An entry is
// valid for a call iff its tag is the call's: nothing is reset between calls.
// Expand: the LoRA wave of every workgroup lists its tile's tokens and
// distinct slots, then polls the partials of its routed tokens until all
// carry the call's tag and sums their k-slices into z = bf16(sum) in LDS.
// Meanwhile the other waves contract the base; then they compute the expand
// of the tile's slots on MFMA, and the epilogue adds
// bf16(scale_g * sum_j z[t][s r + j] * B_g[n][j]) to each routed token.
// Units are produced before any wait, by workgroups below min(grid, CUs)
// (one per CU, so all of them are running), and the plan keeps the units to
// about half of those: every wait is for a workgroup that is already running.
// ---------------------------------------------------------------------------

__device__ __forceinline__ void tagged_store(uint64_t* p, float v, uint32_t tag) {
  __hip_atomic_store(p, (uint64_t(tag) << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t tagged_load(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct Unit {
  int t;      // token
  int ks;     // k-slice
  int j0;     // first A row of the unit's range
  int rows;   // rows of the range (slices * rank - j0, at most urows)
  int kb;     // first k of the slice
  int steps;  // 32-k MFMA steps in the slice
  int64_t aoff;
};

// Token of unit u (u < 1024; the rounding error of the multiply stays below
// 1024 / 2^21 < 1 / (usplit * kz)).
__device__ __forceinline__ int unit_token(const GemvParams& p, int u) { return int((uint32_t(u) * p.unit_inv) >> 21); }

// Unit u's token, adapter rows and k-slice (scalar loads); false when the
// token has no adapter (base only) or its rows end before the unit's range,
// so nothing is produced.
// g: the token's slot, token_slots[unit_token(p, u)], loaded by the caller.
__device__ __forceinline__ bool unit_of_slot(const GemvParams& p, int u, int g, Unit& un) {
  un.t = unit_token(p, u);
  const int rest = u - un.t * p.usplit * p.kz;
  const int range = rest >> (31 - __builtin_clz(p.kz));  // kz is a power of two
  un.ks = rest - range * p.kz;
  const int ks = un.ks;
  if (g < 0 || (p.num_slots > 0 && g >= p.num_slots)) return false;
  const int r = sload(p.ranks, g);
  if (r <= 0 || r > p.max_rank) return false;
  un.j0 = range * p.urows;
  if (un.j0 >= p.slices * r) return false;
  un.aoff = sload(p.a_offsets, g) + int64_t(un.j0) * p.k;
  un.rows = min(p.urows, p.slices * r - un.j0);
  un.kb = ks * p.kz_len;
  un.steps = (min(p.k, un.kb + p.kz_len) - un.kb) >> 5;
  if (un.steps <= 0) {  // an empty trailing slice: zero partials, read at k = 0
    un.kb = 0;
    un.steps = 0;
  }
  return true;
}

__device__ __forceinline__ bool unit_of(const GemvParams& p, int u, Unit& un) {
  return unit_of_slot(p, u, sload(p.token_slots, unit_token(p, u)), un);
}

// Partial of row j of a unit's range (value j0 + j of token t, k-slice ks):
// entry (t * zw + j0 + j) * kz + ks, so the kz partials a consumer sums for
// one value are adjacent.
__device__ __forceinline__ int64_t partial_index(const GemvParams& p, const Unit& un, int j) {
  return (int64_t(un.t) * p.zw + un.j0 + j) * p.kz + un.ks;
}

// x and A fragments of the MFMA steps st0 + i * stride (i < NB) of rows
// j0 .. j0 + 15 of a unit. Loads are unconditional (steps past the slice
// read its last step and contribute zero x) so that they are not serialised
// by branches.
template <int NB>
struct UnitFragsN {
  u32x4 xv[NB];
  u32x4 av[NB];
};

template <bool kUntracked, int NB>
__device__ __forceinline__ void unit_frags(const GemvParams& p, const Unit& un, int j0, int st0, int stride, int lane,
                                           UnitFragsN<NB>& f) {
  const int jn = lane & 15;
  const int kg = lane >> 4;
  const uint16_t* xrow = p.x + int64_t(un.t) * p.x_stride + un.kb + 8 * kg;
  const int j = j0 + jn;
  const uint16_t* arow = p.a_store + un.aoff + int64_t(j < un.rows ? j : un.rows - 1) * p.k + un.kb + 8 * kg;
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int st = st0 + i * stride;
    const int sc = st < un.steps ? st : max(un.steps - 1, 0);
    if constexpr (kUntracked) {
      // Only MFMA row 0 needs the token's x (the other rows stay zero and
      // their results are ignored): 64 bytes per step instead of 1 KiB.
      f.xv[i] = global_load128_untracked_masked(xrow + 32 * sc, 0x0001000100010001ull);
      f.av[i] = global_load128_untracked(arow + 32 * sc);
    } else {
      f.xv[i] = *reinterpret_cast<const u32x4*>(xrow + 32 * sc);
      f.av[i] = *reinterpret_cast<const u32x4*>(arow + 32 * sc);
    }
  }
}

// The first batch of a workgroup's first unit, requested in the prologue
// (untracked loads). x is compact: lane 4 i + g (i < NB <= 16, g < 4) holds
// the 16 bytes of k-group g of step st0 + i * KP, one gathered load; the
// MFMA layout (row 0 only) is formed when used.
template <int NB>
struct FirstFragsN {
  static_assert(NB <= 16, "one compact x register");
  u32x4 xc;
  u32x4 av[NB];
};

template <int NB, int KP>
__device__ __forceinline__ void first_frags(const GemvParams& p, const Unit& un, int st0, int lane, FirstFragsN<NB>& f) {
  const int jn = lane & 15;
  const int kg = lane >> 4;
  {
    const int i = min(lane >> 2, NB - 1);
    const int st = st0 + i * KP;
    const int sc = st < un.steps ? st : max(un.steps - 1, 0);
    const uint16_t* xp = p.x + int64_t(un.t) * p.x_stride + un.kb + 32 * sc + 8 * (lane & 3);
    f.xc = global_load128_untracked_masked(xp, NB == 16 ? ~0ull : (uint64_t(1) << (4 * NB)) - 1);
  }
  const int j = jn;
  const uint16_t* arow = p.a_store + un.aoff + int64_t(j < un.rows ? j : un.rows - 1) * p.k + un.kb + 8 * kg;
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int st = st0 + i * KP;
    const int sc = st < un.steps ? st : max(un.steps - 1, 0);
    f.av[i] = global_load128_untracked(arow + 32 * sc);
  }
}

// Ties every fragment register to a wait already made (no use may be
// scheduled above it).
template <int NB>
__device__ __forceinline__ void tie_frags(FirstFragsN<NB>& f) {
  tie(f.xc);
#pragma unroll
  for (int i = 0; i < NB; ++i) tie(f.av[i]);
}

// MFMAs of the first batch: step i's x fragment for lane (row jn, k-group
// kg) comes from lane 4 i + kg of xc (row 0 only; other rows zero).
template <int NB, int KP>
__device__ __forceinline__ f32x4 first_mfma(const FirstFragsN<NB>& f, const Unit& un, int st0, int lane, f32x4 c) {
  const int kg = lane >> 4;
  const bool row0 = (lane & 15) == 0;
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int src = (4 * i + kg) << 2;
    u32x4 x;
    x.x = uint32_t(__builtin_amdgcn_ds_bpermute(src, int(f.xc.x)));
    x.y = uint32_t(__builtin_amdgcn_ds_bpermute(src, int(f.xc.y)));
    x.z = uint32_t(__builtin_amdgcn_ds_bpermute(src, int(f.xc.z)));
    x.w = uint32_t(__builtin_amdgcn_ds_bpermute(src, int(f.xc.w)));
    const u32x4 zero = {0u, 0u, 0u, 0u};
    c = mfma16(vec_bf16x8(row0 && st0 + i * KP < un.steps ? x : zero), vec_bf16x8(f.av[i]), c);
  }
  return c;
}

template <int NB>
__device__ __forceinline__ f32x4 unit_mfma(const UnitFragsN<NB>& f, const Unit& un, int st0, int stride, f32x4 c) {
  const u32x4 zero = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < NB; ++i)
    c = mfma16(vec_bf16x8(st0 + i * stride < un.steps ? f.xv[i] : zero), vec_bf16x8(f.av[i]), c);
  return c;
}

// Contraction wave w (< KP, the producing waves) sums the MFMA steps w, w + KP, ... of
// every 16-row group of the workgroup's first unit into red[w][j] (j < rows;
// higher j are never read). pre holds the first batch of row group 0 (already
// landed); anything beyond it is loaded here. Then the wave counts itself
// in (LDS) so the LoRA wave can publish without a workgroup barrier.
template <int NB, int KP>
__device__ void first_unit_partials(const GemvParams& p, const Unit& un, FirstFragsN<NB>& pre, float* red, int* done,
                                    int wave, int lane) {
  tie_frags(pre);
  const int jn = lane & 15;
  const int kg = lane >> 4;
  for (int j0 = 0; j0 < un.rows; j0 += 16) {
    f32x4 c = {0.f, 0.f, 0.f, 0.f};
    int st0 = wave;
    if (j0 == 0) {
      c = first_mfma<NB, KP>(pre, un, st0, lane, c);
      st0 += NB * KP;
    }
    // Anything beyond the first batch (ranks above 16, long slices) in small
    // batches: this runs inside the base loop, where registers are scarce.
    for (; st0 < un.steps; st0 += 2 * KP) {
      UnitFragsN<2> f;
      unit_frags<false>(p, un, j0, st0, KP, lane, f);
      c = unit_mfma(f, un, st0, KP, c);
    }
    // Row 0 of C (lanes 0..15, element 0) holds this wave's partial of z[j].
    if (kg == 0) red[wave * 192 + j0 + jn] = c[0];
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the partial rows are in LDS
  if (lane == 0) __hip_atomic_fetch_add(done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// The LoRA wave: waits (LDS) until the contraction waves have written the
// first unit's partial rows, sums and stores them with the call's tag.
template <int KP>
__device__ void publish_first_unit(const GemvParams& p, const float* red, const int* done, const Unit& un,
                                   uint32_t tag, int lane) {
  const int rows = un.rows;
  for (int spins = 0; __hip_atomic_load(done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < KP; ++spins) {
    if (spins > kSpinLimit) {  // cannot happen (every contraction wave counts in); bounded all the same
      if (lane == 0) __hip_atomic_store(p.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    const int jj = q * 64 + lane;
    if (jj < rows) {
      float v = 0.f;
      for (int w = 0; w < KP; ++w) v += red[w * 192 + jj];
      if (!p.withhold) tagged_store(p.zp + partial_index(p, un, jj), v, tag);
    }
  }
}

// The LoRA wave alone: the workgroup's other units (only when there are
// more units than producers, i.e. small grids), each contracted whole by
// this wave and stored with the call's tag.
template <int NB>
__device__ void produce_other_units(const GemvParams& p, uint32_t tag, int lane) {
  if (blockIdx.x >= unsigned(p.producers)) return;
  const int jn = lane & 15;
  const int kg = lane >> 4;
  for (int u = blockIdx.x + p.producers; u < p.units; u += p.producers) {
    Unit un;
    if (!unit_of(p, u, un)) continue;
    for (int j0 = 0; j0 < un.rows; j0 += 16) {
      f32x4 c = {0.f, 0.f, 0.f, 0.f};
      for (int st0 = 0; st0 < un.steps; st0 += NB) {
        UnitFragsN<NB> f;
        unit_frags<false, NB>(p, un, j0, st0, 1, lane, f);
        c = unit_mfma(f, un, st0, 1, c);
      }
      if (kg == 0 && j0 + jn < un.rows && !p.withhold) tagged_store(p.zp + partial_index(p, un, j0 + jn), c[0], tag);
    }
  }
}

// Token metadata of the tile, one entry per tile token (g = -1: base only),
// and the tile's distinct live slots (in order of first use).
struct TileMeta {
  int g[32];
  int r[32];
  int stride[32];
  float scale[32];
  int64_t boff[32];
  int dslot[32];
  int dr[32];
  int dstride[32];
  int64_t dboff[32];
  int start[33];  // z values the tile's tokens need (slices * r, 0 base only), exclusive prefix; start[32] = total
  int bounds[4];  // slice_offsets[0 .. slices] (the wide kernel's copy for its base waves)
  int nd;
  int ready;  // set once the fields above are written (cleared at launch start)
};

// Up to 8 B values (16 bytes) of B row n of an adapter (offset boff, row
// stride st, rank r) from rank j0, zero past the rank or when !live. One
// unconditional 16-byte load (branches here would serialize the callers'
// loads): rows of stride >= 8 are 16-byte aligned (offsets are multiples of
// 8 elements) and j0 + 8 <= stride whenever j0 < r; a row of stride 1, 2 or
// 4 lies inside the aligned 16 bytes that hold its first element (inside
// the adapter's N x stride region) and is shifted down by its position.
struct B8 {
  const uint16_t* src;  // aligned 16 bytes to load
  int off;              // elements to shift down
  int cnt;              // elements to keep
};

__device__ __forceinline__ B8 b8_at(const GemvParams& p, int64_t boff, int st, int r, int n, int j0, bool live) {
  const int64_t e = boff + int64_t(n) * st + j0;
  B8 b;
  b.off = st >= 8 ? 0 : int(e & 7);
  b.cnt = live ? min(8, r - j0) : 0;
  // Nothing to keep (past the rank or dead): read the store's first 16
  // bytes instead, which always exist.
  b.src = p.b_store + (b.cnt > 0 ? e - b.off : 0);
  return b;
}

// The first cnt bf16 elements of v, the rest zero.
__device__ __forceinline__ uint4 keep_first(const uint4& v, int cnt) {
  uint32_t o[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int k = 0; k < 4; ++k) o[k] = 2 * k >= cnt ? 0u : 2 * k + 1 >= cnt ? (o[k] & 0xffffu) : o[k];
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// Dword i of v (0 past the end), by selects: a runtime-indexed array would
// live in scratch.
__device__ __forceinline__ uint32_t dword_at(const uint4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : i == 3 ? v.w : 0u;
}

__device__ __forceinline__ uint4 b8_fix(const uint4& v, const B8& b) {
  const int d = b.off >> 1;
  uint32_t out[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t a = dword_at(v, k + d);
    const uint32_t c = dword_at(v, k + d + 1);
    uint32_t o = (b.off & 1) ? ((a >> 16) | (c << 16)) : a;
    if (2 * k >= b.cnt) o = 0u;
    else if (2 * k + 1 >= b.cnt) o &= 0xffffu;
    out[k] = o;
  }
  return make_uint4(out[0], out[1], out[2], out[3]);
}

// z row stride in LDS (elements): a tile shape may set kZRow (a multiple
// of 8, at least 192); otherwise 192 (three slices of 64).
template <class TL, class = void>
struct ZRow {
  static constexpr int value = 192;
};
template <class TL>
struct ZRow<TL, std::void_t<decltype(TL::kZRow)>> {
  static constexpr int value = TL::kZRow;
};

// LDS of the LoRA stages, an array that never receives direct copies (so
// stores into it do not wait for copies in flight): the tile metadata and z
// (token i's slice s at i * kZRow + 64 s).
template <class TL>
struct LoraLds {
  static constexpr int kMeta = 0;
  static constexpr int kZ = 2048;  // z: [tile token][kZRow] bf16
  static constexpr int kZRow = ZRow<TL>::value;
  static constexpr int kBytes = kZ + TL::kXR * kZRow * 2;
  static_assert(sizeof(TileMeta) <= 2048, "tile metadata");
  static_assert(kZRow >= 192 && kZRow % 8 == 0, "z rows hold three 64-value slices, 16-byte aligned");
};

// The LoRA wave, part 1a (before the workgroup's table barrier, while
// nothing else is outstanding in this wave): the slot of tile token `lane`
// and its adapter's metadata, two round trips. Base-only tokens and lanes
// past the tile read the slice bounds instead (at least 8 valid bytes; the
// values are discarded), since the table may hold no slot at all.
struct TokenMeta {
  int g;
  int r;
  int stride;
  float scale;
  int64_t boff;
};

// g: token_slots[t0 + min(lane, mt - 1)], loaded by the caller.
__device__ __forceinline__ TokenMeta token_meta(const GemvParams& p, int g, int mt, int lane) {
  TokenMeta m;
  m.g = lane < mt && (p.num_slots == 0 || g < p.num_slots) ? g : -1;
  const bool live = m.g >= 0;
  const void* fb = p.slice_offsets;
  m.r = *(live ? p.ranks + m.g : static_cast<const int32_t*>(fb));
  m.stride = *(live ? p.b_strides + m.g : static_cast<const int32_t*>(fb));
  m.scale = *(live ? p.lscales + m.g : static_cast<const float*>(fb));
  m.boff = *(live ? p.b_offsets + m.g : static_cast<const int64_t*>(fb));
  if (!live || m.r <= 0 || m.r > p.max_rank) {
    m.g = -1;
    m.r = 0;
    m.stride = 1;
    m.scale = 0.f;
    m.boff = 0;
  }
  return m;
}

// The per-slot metadata of up to 256 slots in registers (lane l holds
// slots l, l + 64, l + 128, l + 192), requested by a LoRA wave at its start:
// these loads do not wait for the tile's token slots, so they can go out
// before the workgroup's copies. Token metadata then comes from lane
// shuffles (token_meta_from).
constexpr int kSlotTableMax = 256;
struct SlotTable {
  int r[4];
  int stride[4];
  float scale[4];
  int64_t boff[4];
};

__device__ __forceinline__ bool slot_table_usable(const GemvParams& p) {
  return p.num_slots > 0 && p.num_slots <= kSlotTableMax;
}

__device__ __forceinline__ void slot_table_load(const GemvParams& p, int lane, SlotTable& t) {
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    t.r[c] = 0;
    t.stride[c] = 1;
    t.scale[c] = 0.f;
    t.boff[c] = 0;
    if (64 * c < p.num_slots) {  // uniform
      const int s = min(64 * c + lane, p.num_slots - 1);
      t.r[c] = p.ranks[s];
      t.stride[c] = p.b_strides[s];
      t.scale[c] = p.lscales[s];
      t.boff[c] = p.b_offsets[s];
    }
  }
}

// token_meta from the slot table; slots past num_slots run base only.
__device__ __forceinline__ TokenMeta token_meta_from(const GemvParams& p, const SlotTable& t, int g, int mt,
                                                     int lane) {
  TokenMeta m;
  m.g = lane < mt && g >= 0 && g < p.num_slots ? g : -1;
  const int gs = max(m.g, 0);
  const int src = (gs & 63) << 2;
  const int c = gs >> 6;
  m.r = 0;
  m.stride = 1;
  m.scale = 0.f;
  m.boff = 0;
#pragma unroll
  for (int cc = 0; cc < 4; ++cc) {
    if (64 * cc >= p.num_slots) break;  // uniform
    const int r = __builtin_amdgcn_ds_bpermute(src, t.r[cc]);
    const int st = __builtin_amdgcn_ds_bpermute(src, t.stride[cc]);
    const float sc = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(t.scale[cc])));
    const uint32_t blo = uint32_t(__builtin_amdgcn_ds_bpermute(src, int(uint32_t(uint64_t(t.boff[cc])))));
    const uint32_t bhi = uint32_t(__builtin_amdgcn_ds_bpermute(src, int(uint32_t(uint64_t(t.boff[cc]) >> 32))));
    if (c == cc) {
      m.r = r;
      m.stride = st;
      m.scale = sc;
      m.boff = int64_t((uint64_t(bhi) << 32) | blo);
    }
  }
  if (m.g < 0 || m.r <= 0 || m.r > p.max_rank) {
    m.g = -1;
    m.r = 0;
    m.stride = 1;
    m.scale = 0.f;
    m.boff = 0;
  }
  return m;
}

// The LoRA wave, part 1b (after the table barrier): tile metadata and
// distinct slots into LDS, then the ready flag.
template <class TL>
__device__ void lora_meta(char* lds, const TokenMeta& m, int slices, int lane) {
  TileMeta* tm = reinterpret_cast<TileMeta*>(lds + LoraLds<TL>::kMeta);
  const int g = m.g, r = m.r, stride = m.stride;
  // Where each token's z values start in the tile's compact list of needed
  // values (a shuffle scan over the 32 token lanes).
  const int cnt = (lane < 32 && g >= 0) ? slices * r : 0;
  int incl = cnt;
#pragma unroll
  for (int d = 1; d < 32; d <<= 1) {
    const int v = __shfl_up(incl, d, 64);
    if (lane >= d) incl += v;
  }
  if (lane < 32) tm->start[lane] = incl - cnt;
  if (lane == 31) tm->start[32] = incl;
  const float scale = m.scale;
  const int64_t boff = m.boff;
  if (lane < 32) {
    tm->g[lane] = g;
    tm->r[lane] = r;
    tm->stride[lane] = stride;
    tm->scale[lane] = scale;
    tm->boff[lane] = boff;
  }
  // Distinct live slots: one ballot per slot.
  uint64_t left = __ballot(lane < 32 && g >= 0);
  int nd = 0;
  while (left) {
    const int f = __builtin_ctzll(left);
    const int gf = __builtin_amdgcn_readlane(g, f);
    if (lane == f) {
      tm->dslot[nd] = g;
      tm->dr[nd] = r;
      tm->dstride[nd] = stride;
      tm->dboff[nd] = boff;
    }
    left &= ~__ballot(g == gf);
    ++nd;
  }
  if (lane == 0) tm->nd = nd;
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the metadata is in LDS
  if (lane == 0) *(volatile __attribute__((address_space(3))) int*)(&tm->ready) = 1;
}


// The LoRA wave, part 2: z of the tile. Token i's value j has its KZ
// k-slice partials at ((t0 + i) * zw + j) * KZ .. + KZ. Only the values the
// routed tokens need (j < slices * r) are read: they are numbered in a
// compact list (token i's at start[i] .. start[i + 1]), each lane owns up to
// 16 / KZ of a batch of that list (its token found by a binary search over
// start), polls them until all carry the call's tag, sums each value in
// registers, z[i][j] = bf16(sum), and stores it slice padded into LDS (zero
// past the rank). A tile of 32 rank-64 tokens needs 2048 values, two
// batches; one whose ranks average 25 needs one. KZ (k-slices per token) is
// a power of two up to 16.
// z value j of token t (slot g) before rounding: sum over K of
// x[t][k] * A_g[j][k] (A rows packed at s * r, so value j is row j), in fp32.
__device__ __forceinline__ float full_dot(const GemvParams& p, int t, int g, int j) {
  const uint16_t* xr = p.x + int64_t(t) * p.x_stride;
  const uint16_t* ar = p.a_store + p.a_offsets[g] + int64_t(j) * p.k;
  float acc = 0.f;
  for (int k = 0; k < p.k; k += 8) {
    const uint4 xv = *reinterpret_cast<const uint4*>(xr + k);
    const uint4 av = *reinterpret_cast<const uint4*>(ar + k);
    const uint32_t xs[4] = {xv.x, xv.y, xv.z, xv.w};
    const uint32_t as[4] = {av.x, av.y, av.z, av.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc = __builtin_fmaf(bf16_lo(xs[e]), bf16_lo(as[e]), acc);
      acc = __builtin_fmaf(bf16_hi(xs[e]), bf16_hi(as[e]), acc);
    }
  }
  return acc;
}

// Tagged partials a lane polls per gather batch: a tile shape may set
// kGatherEntries; otherwise 16, or 8 for the narrow tiles of up to 8 tokens.
template <class TL, class = void>
struct GatherEntries {
  static constexpr int value = TL::kRT == 1 && TL::kXR <= 8 ? 8 : 16;
};
template <class TL>
struct GatherEntries<TL, std::void_t<decltype(TL::kGatherEntries)>> {
  static constexpr int value = TL::kGatherEntries;
};

template <class TL, int KZ>
__device__ bool lora_gather_kz(const GemvParams& p, char* lds, int t0, int mt, uint32_t tag, int lane) {
  using L = LoraLds<TL>;
  // Values per lane and batch (16 entries; 8 for the tiles of up to 8
  // tokens, which keeps them at two workgroups per CU, or a tile's own
  // kGatherEntries).
  constexpr int kEntries = GatherEntries<TL>::value;
  constexpr int kOut = kEntries / KZ > 0 ? kEntries / KZ : 1;
  const TileMeta* tm = reinterpret_cast<const TileMeta*>(lds + L::kMeta);
  uint16_t* zl = reinterpret_cast<uint16_t*>(lds + L::kZ);
  for (int e = lane; e < TL::kXR * L::kZRow / 8; e += 64) reinterpret_cast<uint4*>(zl)[e] = make_uint4(0, 0, 0, 0);
  const int total = tm->start[32];
  for (int o0 = 0; o0 < total; o0 += 64 * kOut) {
    const uint64_t* block = p.zp + int64_t(t0) * p.zw * KZ;
    int il[kOut], jv[kOut];
    bool need[kOut];
#pragma unroll
    for (int q = 0; q < kOut; ++q) {
      const int o = min(o0 + q * 64 + lane, total - 1);
      // The last token whose values start at or before o (tokens with none
      // share their successor's start and are passed over).
      int i = 0;
#pragma unroll
      for (int step = 16; step > 0; step >>= 1)
        if (tm->start[i + step] <= o) i += step;
      il[q] = i;
      jv[q] = o - tm->start[i];
      need[q] = o0 + q * 64 + lane < total;
    }
    uint64_t v[kOut][KZ];
    bool gave_up = false;
    for (int spins = 0;; ++spins) {
#pragma unroll
      for (int q = 0; q < kOut; ++q)
#pragma unroll
        for (int ks = 0; ks < KZ; ++ks)  // unconditional: no per-load branch
          v[q][ks] = tagged_load(block + (int64_t(il[q]) * p.zw + jv[q]) * KZ + ks);
      bool ok = true;
#pragma unroll
      for (int q = 0; q < kOut; ++q)
#pragma unroll
        for (int ks = 0; ks < KZ; ++ks) ok = ok && (!need[q] || uint32_t(v[q][ks] >> 32) == tag);
      if (__all(ok)) break;
      if (spins > p.spin_limit) {
        gave_up = true;  // (cannot happen while producers run: they wait for nothing)
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int q = 0; q < kOut; ++q) {
      float z = 0.f;
#pragma unroll
      for (int ks = 0; ks < KZ; ++ks) z += __uint_as_float(uint32_t(v[q][ks]));
      const int i = il[q];
      const int j = jv[q];
      const int ri = tm->r[i];
      const int s = int(j >= ri) + int(j >= 2 * ri) + int(j >= 3 * ri);  // slice of value j (3: past them)
      if (need[q] && s < p.slices) zl[i * L::kZRow + s * 64 + (j - s * ri)] = uint16_t(f32_to_bf16(z));
    }
    if (gave_up) return true;
  }
  return false;
}

// After a wait gave up: every z value of the tile is recomputed from x and A
// over the whole K (one compact loop, off the normal path; fp32 sums in
// another order than the partials', so z may differ by a bf16 rounding); the
// status word reports it.
template <class TL>
__device__ void lora_recompute(const GemvParams& p, char* lds, int t0, int mt, int lane) {
  using L = LoraLds<TL>;
  const TileMeta* tm = reinterpret_cast<const TileMeta*>(lds + L::kMeta);
  uint16_t* zl = reinterpret_cast<uint16_t*>(lds + L::kZ);
  if (lane == 0) __hip_atomic_store(p.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (int o = lane; o < mt * p.zw; o += 64) {
    const int i = o / p.zw;
    const int j = o - i * p.zw;
    const int ri = tm->r[i];
    if (tm->g[i] < 0 || j >= p.slices * ri) continue;
    const int s = j / ri;
    zl[i * L::kZRow + s * 64 + (j - s * ri)] = uint16_t(f32_to_bf16(full_dot(p, t0 + i, tm->g[i], j)));
  }
}

template <class TL>
__device__ void lora_gather(const GemvParams& p, char* lds, int t0, int mt, uint32_t tag, int lane) {
  bool gave_up;
  switch (p.kz) {
    case 1: gave_up = lora_gather_kz<TL, 1>(p, lds, t0, mt, tag, lane); break;
    case 2: gave_up = lora_gather_kz<TL, 2>(p, lds, t0, mt, tag, lane); break;
    case 4: gave_up = lora_gather_kz<TL, 4>(p, lds, t0, mt, tag, lane); break;
    case 8: gave_up = lora_gather_kz<TL, 8>(p, lds, t0, mt, tag, lane); break;
    default: gave_up = lora_gather_kz<TL, 16>(p, lds, t0, mt, tag, lane); break;
  }
  if (gave_up) lora_recompute<TL>(p, lds, t0, mt, lane);
}


// ---------------------------------------------------------------------------
// Host-side plan of the shrink units.
// ---------------------------------------------------------------------------
struct GemvPlan {
  int rows;
  int row_groups;
  int grid;
  int kz;
  int kz_len;
  int usplit;
  int urows;
  int units;
  int producers;
};

// Shrink units: m tokens x kz k-slices, kz chosen so that m * kz is about
// min(grid, CUs) (one unit per producing workgroup when m allows) and a
// consumer's partial reads fit one batch.
// Control header layout: the call-epoch words and the status word
// (call_epoch.h), then the tagged shrink partials (at most 64 tokens x 192
// values x 8 bytes).
constexpr int64_t kPartialsOffset = 2048;

GemvPlan gemv_plan(int64_t m, int64_t n, int64_t k, int cus, int zw) {
  GemvPlan pl;
  pl.rows = m > 32 ? 32 : 16;
  pl.row_groups = int(n / pl.rows);
  pl.grid = pl.row_groups * int((m + 31) / 32);
  const int64_t cap = std::min<int64_t>(pl.grid, cus);
  const int64_t nblk = k / 64;
  // A consumer reads tile tokens x zw x kz partials: keep that to one
  // 1024-value batch where the shape allows, and at most half of the
  // workgroups producing (production delays their contraction).
  const int64_t tile_tokens = std::min<int64_t>(m, 32);
  int64_t kz = std::max<int64_t>(
      1, std::min<int64_t>({nblk, cap / (2 * m), 16, 1024 / std::max<int64_t>(1, tile_tokens * zw)}));
  while (kz & (kz - 1)) kz &= kz - 1;  // a power of two (the consumer sums the slices unrolled)
  pl.kz_len = int((nblk + kz - 1) / kz) * 64;
  pl.kz = int(kz);  // trailing slices may be empty (their partials are zero)
  // The consumer holds 16 entries per lane and batch: one token's kz * zw
  // entries must fit 1024 (kz > 1 only when that holds; zw <= 192 at kz = 1).
  // Tokens of wide z (high ranks, several slices) split their rows over as
  // many units as the producers allow: a rank-64 token's whole A (512 KB at
  // K = 4096) in one workgroup held every consumer for about 30 us.
  const int64_t groups = (zw + 15) / 16;  // 16-row groups per token
  const int64_t split = std::max<int64_t>(1, std::min<int64_t>(groups, cap / (m * kz)));
  pl.urows = int((groups + split - 1) / split) * 16;
  pl.usplit = int((groups * 16 + pl.urows - 1) / pl.urows);
  pl.units = int(m) * pl.usplit * pl.kz;
  pl.producers = int(cap);
  return pl;
}

// The LoRA fields of the launch parameters (workspace control header, tagged
// partials and the unit plan), shared by both decode launchers.
// Block scales of a decode launch. fp32 scales are streamed as given. A
// nested state is read by the kernel itself (dq_scales.h) where the layout
// allows it: the codes' rows start on dwords (K % 256 == 0, the code pointer
// 4-byte aligned), dq_block is a power of two of at least 64, code2 16-byte aligned, a row
// half of `rows` rows spans at most 32 absmax2 entries, and the wave's
// staging fits its scale area (stage_fits). Otherwise the fp32 scales are
// rebuilt into the workspace (after the prefill's flag region, which holds
// only tags) by lf_nf4_prepare_scales_dq first.
inline int64_t decode_scales_offset() { return kWorkspaceHeader + kFlagRegion; }
inline int64_t decode_scales_bytes(int64_t n, int64_t k) { return (n * (k / 64) * 4 + 255) / 256 * 256; }

inline bool dq_layout_ok(const lf_nf4_weight* w, int rows) {
  if (w->scales || !w->absmax_q || !w->absmax2 || !w->code2 || !w->offset) return false;
  const int64_t nblk = w->k / 64, dq = w->dq_block;
  return w->k % 256 == 0 && (reinterpret_cast<uintptr_t>(w->absmax_q) & 3u) == 0 && aligned16(w->code2) && dq >= 64 &&
         (dq & (dq - 1)) == 0 && dq < (int64_t(1) << 30) && int64_t(rows / 2) * nblk / dq + 2 <= 32;
}

inline void fill_dq_params(GemvParams& p, const lf_nf4_weight* w) {
  p.absmax_q = w->absmax_q;
  p.absmax2 = w->absmax2;
  p.code2 = w->code2;
  p.dq_offset = w->offset;
  p.dq_shift = __builtin_ctzll(uint64_t(w->dq_block));
  const int64_t blocks = w->n * (w->k / 64);
  p.a2_len = int((blocks + w->dq_block - 1) / w->dq_block);
}

// (Stride 1 has no 32-bit magic: the kernels take pos itself.)
inline uint32_t stride_magic(int stride) {
  return stride <= 1 ? 0u : uint32_t(((uint64_t(1) << 32) + uint64_t(stride) - 1) / uint64_t(stride));
}

// fp32 scales of a nested state rebuilt into the workspace (the decode
// kernels' fallback).
inline int rebuild_scales(const lf_nf4_weight* w, void* workspace, int64_t workspace_bytes, void* stream,
                          const float** scales) {
  const int64_t need = decode_scales_offset() + decode_scales_bytes(w->n, w->k);
  LF_REQUIRE(workspace && workspace_bytes >= need && aligned16(workspace),
             "workspace too small for the rebuilt scales: need %lld bytes", (long long)need);
  float* out = reinterpret_cast<float*>(static_cast<char*>(workspace) + decode_scales_offset());
  const int rc = lf_nf4_prepare_scales_dq(w->absmax_q, w->absmax2, w->code2, w->offset, w->dq_block, out,
                                          w->n * (w->k / 64), stream);
  if (rc != kOk) return rc;
  *scales = out;
  return kOk;
}

inline int fill_lora_params(GemvParams& p, const GemvPlan& pl, const lf_lora* lora, int64_t m, void* workspace,
                            int64_t workspace_bytes, bool withhold) {
  LF_REQUIRE(workspace && workspace_bytes >= kWorkspaceHeader, "workspace too small: need %lld bytes",
             (long long)kWorkspaceHeader);
  LF_REQUIRE(kPartialsOffset + m * pl.kz * lora->num_slices * lora->max_rank * 8 <= kWorkspaceHeader,
             "shrink partials exceed the control header");
  LF_REQUIRE(aligned16(workspace), "workspace must be 16-byte aligned");
  p.a_store = lora->a_store;
  p.a_offsets = lora->a_offsets;
  p.b_store = lora->b_store;
  p.b_offsets = lora->b_offsets;
  p.b_strides = lora->b_strides;
  p.ranks = lora->ranks;
  p.lscales = lora->scales;
  p.token_slots = lora->token_slots;
  p.slice_offsets = lora->slice_offsets;
  p.slices = lora->num_slices;
  p.max_rank = lora->max_rank;
  LF_REQUIRE(lora->num_slots >= 0, "num_slots must not be negative");
  p.num_slots = lora->num_slots;
  p.zw = lora->num_slices * lora->max_rank;
  p.units = pl.units;
  p.kz = pl.kz;
  p.usplit = pl.usplit;
  p.urows = pl.urows;
  p.unit_inv = ((1u << 21) + uint32_t(pl.usplit * pl.kz) - 1) / uint32_t(pl.usplit * pl.kz);
  LF_REQUIRE(pl.units <= 1024, "too many shrink units");
  p.kz_len = pl.kz_len;
  p.producers = pl.producers;
  char* ws = static_cast<char*>(workspace);
  p.ce = call_epoch_of(ws);
  p.status = reinterpret_cast<int*>(ws + kStatusOffset);
  p.withhold = withhold ? 1 : 0;
  p.spin_limit = withhold ? 64 : kSpinLimit;
  p.zp = reinterpret_cast<uint64_t*>(ws + kPartialsOffset);
  return kOk;
}

}  // namespace
}  // namespace lf
