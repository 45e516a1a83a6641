// Decode NF4 linear (M <= 64 tokens) without split-K.
//
// Reference chain (integrations/_sglang_nf4_linear.py:116-129):
//   y = bf16(x @ dequant(W)^T) (+ bias, rounded again).
//
// Each workgroup owns R = 16 * RT output rows and a tile of up to 32 tokens
// over the whole K, so no partial sums cross workgroups. Its eight waves split
// the NF4 blocks of K between them; each wave streams its own blocks through
// a private LDS ring (W bytes, x rows, block scales) filled by direct
// global -> LDS copies, waits only on its own copy counter, and contracts
// each block on bf16 MFMA (16 tokens x 16 rows x 32 k). Two waves per SIMD
// keep two such chains in flight. The eight partial tiles are summed through
// LDS once at the end.
//
// Per-CU traffic is R * K / 2 bytes of W plus T * K * 2 bytes of x; the x
// rows are shared by every workgroup and come from L2. With N = 4096:
// M <= 16 uses 16 rows x 16 tokens (256 workgroups), M <= 32 16 x 32, and
// M <= 64 32 x 32 (128 row groups x 2 token tiles, both on one XCD so W is
// read from HBM once).
#include <algorithm>

#include "call_epoch.h"
#include "lds_pipeline.h"
#include "nf4_common.h"
#include "../../include/loraforge_amd.h"

namespace lf {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kCopies = 16;  // pair-table copies (lane l reads copy l % 16)

// RT: 16-row output tiles; XR: staged token rows (2, 8, 16 or 32).
// SP (scales in LDS; the launch uses it wherever the scale areas fit): each
// contraction wave copies the block scales of its whole k range into LDS
// once, ahead of its first stage, and the tile of up to 2 tokens stages 4
// blocks (a full 128-byte line of every row) at a time. Otherwise each stage
// carries its own scales. Measured read patterns on MI355X (no arithmetic,
// 7 streaming waves, B = 1 x rows, per-stage scales and 2-block stages ->
// scales once and 4-block stages): 24576 x 4096 18.9 -> 12.9 us, 4096 x 12288
// 11.6 -> 7.8 us, 4096 x 4096 5.0 -> 4.0 us.
template <int RT, int XR, bool SP>
struct Tile {
  static constexpr int kRT = RT;
  static constexpr int kR = 16 * RT;
  static constexpr int kXR = XR;
  static constexpr int kTT = XR > 16 ? 2 : 1;                  // 16-token MFMA tiles
  static constexpr bool kScPre = SP;
  static constexpr int kSB = (kScPre && XR <= 2) ? 4 : (RT == 1 && XR <= 16) ? 2 : 1;  // NF4 blocks per stage
  static constexpr int kWBytes = kR * kSB * 32 < 1024 ? 1024 : kR * kSB * 32;
  static constexpr int kWDma = kWBytes / 1024;
  static constexpr int kXBytes = XR * kSB * 128 < 1024 ? 1024 : XR * kSB * 128;
  static constexpr int kXDma = kXBytes / 1024;
  static constexpr int kScBytes = kScPre ? 0 : 256;  // one dword copy: kR * kSB scales used
  static constexpr int kStage = kWBytes + kXBytes + kScBytes;
  static constexpr int kDma = kWDma + kXDma + (kScPre ? 0 : 1);  // copies per stage
  // Scales in LDS: two stages, both streaming (against three: north-star
  // B = 64 18.1 -> 17.8 us, B = 32 16.5 -> 16.1 us, c3 B = 64 gate/up
  // 85.4 -> 81.1 us). Per-stage scales: three stages (Tile<1, 8>: two, for
  // two workgroups per CU in LDS).
  static constexpr int kDepth = (SP || (RT == 1 && XR == 8)) ? 2 : 3;
  static_assert(kR * kSB * 32 <= kWBytes && (kScPre || kR * kSB <= 64), "stage sizes");
  static_assert(kDma * (kDepth - 1) < 64, "vmcnt range");
};

// LDS scale area of one contraction wave (kScPre tiles): the group's rows
// over its k range at a row stride of `stride` floats (odd: the 16 rows a
// fragment read covers fall in distinct banks), rounded up to whole 64-lane
// dword copies.
struct ScaleArea {
  int stride;  // floats per row: (max blocks per wave) | 1
  int bytes;   // per wave: multiple of 256
};
inline ScaleArea scale_area(int nblk, int waves, int rows) {
  ScaleArea a;
  a.stride = ((nblk + waves - 1) / waves) | 1;
  a.bytes = int((int64_t(rows) * a.stride * 4 + 255) / 256 * 256);
  return a;
}

// bf16(silu(g)) * u in fp32 (the caller's store rounds the product): silu
// as g / (1 + e^-g), the form of the reference's activation.
__device__ __forceinline__ float silu_times(float g, float u) {
  const float act = g / (1.0f + expf(-g));
  return round_bf16(act) * u;
}

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
  int gated_half;  // SwiGLU output: n / 2 (a group's rows: R / 2 gate rows and the matching up rows), else 0
  int sc_stride;  // kScPre tiles: floats per row of a wave's scale area (odd)
  int sc_bytes;   // kScPre tiles: bytes of a wave's scale area in dynamic LDS (multiple of 256)
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
  int zw;         // z row width: slices * max_rank
  int units;      // shrink units: m * usplit * kz
  int kz;         // k-slices per token
  int usplit;     // row ranges per token (unit u: token u / (usplit * kz), range (u / kz) % usplit, k-slice u % kz)
  int urows;      // A rows per range (a multiple of 16)
  uint32_t unit_inv;  // ceil(2^21 / (usplit * kz)): u / (usplit * kz) by a multiply (u <= 1024)
  int kz_len;     // k per slice (multiple of 64)
  int producers;  // workgroups b < producers make units b, b + producers, ...
  int resident;   // workgroups of the first dispatch round (b < resident run beside the producers)
  int* status;    // set to 1 when a bounded wait for partials gave up (they were then recomputed)
  int spin_limit; // polls of a bounded wait for partials
  int withhold;   // test hook: producers publish nothing, so every wait gives up and recomputes
  CallEpoch ce;      // call tag: epoch + 1, moved on by the last workgroup
  uint64_t* zp;      // [units][zw] shrink partial sums as (tag << 32) | fp32 bits
};

constexpr int kSpinLimit = 1 << 20;

// vmcnt(n) for n = c * kDma, c < kDepth (runtime c).
template <class TL>
__device__ __forceinline__ void wait_stages(int c) {
  switch (c) {
    case 0: wait_vm<0>(); break;
    case 1: wait_vm<TL::kDma>(); break;
    case 2: wait_vm<2 * TL::kDma>(); break;
    case 3: wait_vm<3 * TL::kDma>(); break;
    case 4: wait_vm<4 * TL::kDma>(); break;
    case 5: wait_vm<(TL::kDepth > 5 ? 5 : 0) * TL::kDma>(); break;
    case 6: wait_vm<(TL::kDepth > 6 ? 6 : 0) * TL::kDma>(); break;
    default: wait_vm<(TL::kDepth > 7 ? 7 : 0) * TL::kDma>(); break;
  }
}

template <int kC>
__device__ __forceinline__ uint4 codes_dword(uint32_t d, const uint32_t* ptl) {
  uint4 r;
  r.x = ptl[(d & 0xffu) * kC];
  r.y = ptl[__builtin_amdgcn_ubfe(d, 8, 8) * kC];
  r.z = ptl[__builtin_amdgcn_ubfe(d, 16, 8) * kC];
  r.w = ptl[(d >> 24) * kC];
  return r;
}

// Lane (n = l & 15, g = l >> 4) holds W[row n][16g .. 16g + 16) of an NF4
// block (8 bytes) and x[token][same k]; MFMA step j covers k = 16g + 8j .. +8.
// Default: bf16(code) contracted, the fp32 block scale applied to the block
// sum; exact: bf16_rne(code * scale) weights (the reference's dequantised W).
// Ring fragments of one stage for this lane: W bytes (8 per block and row
// tile), block scales, and x fragments (2 x 16 bytes per block and token tile).
template <class TL>
struct Frags {
  u32x2 q[TL::kSB][TL::kRT];
  float sc[TL::kSB][TL::kRT];
  u32x4 xf[TL::kSB][TL::kTT][2];
};

// scb: the scales of the stage's first block (kScPre: in the wave's scale
// area, rows srs bytes apart; else the stage's own scale slot).
template <class TL>
__device__ __forceinline__ void read_frags(Frags<TL>& f, uint32_t wbase, uint32_t scb, uint32_t srs, int n, int g) {
  const uint32_t xbase = wbase + TL::kWBytes;
#pragma unroll
  for (int b = 0; b < TL::kSB; ++b) {
#pragma unroll
    for (int r = 0; r < TL::kRT; ++r) {
      const int row = r * 16 + n;
      f.q[b][r] = lds_read64(wbase + (b * TL::kR + row) * 32 + 8 * g);
      if constexpr (TL::kScPre) f.sc[b][r] = lds_read32f(scb + row * srs + b * 4);
      else f.sc[b][r] = lds_read32f(scb + (b * TL::kR + row) * 4);
    }
#pragma unroll
    for (int t = 0; t < TL::kTT; ++t) {
      const int xr = (t * 16 + n) % TL::kXR;
#pragma unroll
      for (int j = 0; j < 2; ++j)
        f.xf[b][t][j] = lds_read128(xbase + (xr * TL::kSB + b) * 128 + (((2 * g + j) ^ (xr & 7)) << 4));
    }
  }
}

// Waits for the untracked ring reads and ties their results to the wait.
template <class TL>
__device__ __forceinline__ void settle(Frags<TL>& f) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int b = 0; b < TL::kSB; ++b) {
#pragma unroll
    for (int r = 0; r < TL::kRT; ++r) {
      tie(f.q[b][r]);
      tie(f.sc[b][r]);
    }
#pragma unroll
    for (int t = 0; t < TL::kTT; ++t) {
      tie(f.xf[b][t][0]);
      tie(f.xf[b][t][1]);
    }
  }
}

// Decodes every W fragment of the stage first (all codebook lookups in
// flight together), then runs the MFMAs. Blocks past the wave's range get
// scale 0.
template <class TL, bool kExact>
__device__ __forceinline__ void contract(const Frags<TL>& f, int kb, int kend, f32x4 (&acc)[TL::kRT][TL::kTT],
                                         const float* table, const uint32_t* ptl) {
  uint4 w[TL::kSB][TL::kRT][2];
  float sc[TL::kSB][TL::kRT];
#pragma unroll
  for (int b = 0; b < TL::kSB; ++b)
#pragma unroll
    for (int r = 0; r < TL::kRT; ++r) {
      sc[b][r] = kb + b < kend ? f.sc[b][r] : 0.f;
      if constexpr (kExact) {
        w[b][r][0] = decode_dword(f.q[b][r].x, sc[b][r], table);
        w[b][r][1] = decode_dword(f.q[b][r].y, sc[b][r], table);
      } else {
        w[b][r][0] = codes_dword<kCopies>(f.q[b][r].x, ptl);
        w[b][r][1] = codes_dword<kCopies>(f.q[b][r].y, ptl);
      }
    }
#pragma unroll
  for (int b = 0; b < TL::kSB; ++b)
#pragma unroll
    for (int r = 0; r < TL::kRT; ++r)
#pragma unroll
      for (int t = 0; t < TL::kTT; ++t) {
        if constexpr (kExact) {
          acc[r][t] = mfma16(vec_bf16x8(f.xf[b][t][0]), as_bf16x8(w[b][r][0]), acc[r][t]);
          acc[r][t] = mfma16(vec_bf16x8(f.xf[b][t][1]), as_bf16x8(w[b][r][1]), acc[r][t]);
        } else {
          const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
          f32x4 d = mfma16(vec_bf16x8(f.xf[b][t][0]), as_bf16x8(w[b][r][0]), zero);
          d = mfma16(vec_bf16x8(f.xf[b][t][1]), as_bf16x8(w[b][r][1]), d);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[r][t][e] = __builtin_fmaf(sc[b][r], d[e], acc[r][t][e]);
        }
      }
}


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
constexpr int kProd = kWaves - 1;  // contraction waves: they compute the shrink partials
constexpr int kBatch = 10;         // MFMA steps per wave and batch (kProd * kBatch >= 64 steps)

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
  if (g < 0) return false;
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

// x and A fragments of the MFMA steps st0 + i * stride (i < kBatch) of rows
// j0 .. j0 + 15 of a unit. Loads are unconditional (steps past the slice
// read its last step and contribute zero x) so that they are not serialised
// by branches.
template <int NB>
struct UnitFragsN {
  u32x4 xv[NB];
  u32x4 av[NB];
};

// A 16-byte global load the compiler does not track. While direct LDS copies
// are in flight, the compiler waits for every outstanding memory operation
// before using any tracked load result; these fragments are requested
// between the first and second weight stages and are known to have landed
// once the second stage has (loads complete in order).
__device__ __forceinline__ u32x4 global_load128_untracked(const void* ptr) {
  u32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(ptr) : "memory");
  return v;
}

// The same for the lanes of `lanes` only (the others keep zero and issue no
// memory request): the whole exec change stays inside the statement.
__device__ __forceinline__ u32x4 global_load128_untracked_masked(const void* ptr, uint64_t lanes) {
  u32x4 v = {0u, 0u, 0u, 0u};
  uint64_t saved;
  asm volatile(
      "s_and_saveexec_b64 %1, %3\n\t"
      "global_load_dwordx4 %0, %2, off\n\t"
      "s_mov_b64 exec, %1"
      : "+v"(v), "=&s"(saved)
      : "v"(ptr), "s"(lanes)
      : "memory", "exec");
  return v;
}

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
// the 16 bytes of k-group g of step st0 + i * kProd, one gathered load; the
// MFMA layout (row 0 only) is formed when used.
template <int NB>
struct FirstFragsN {
  static_assert(NB <= 16, "one compact x register");
  u32x4 xc;
  u32x4 av[NB];
};

template <int NB>
__device__ __forceinline__ void first_frags(const GemvParams& p, const Unit& un, int st0, int lane, FirstFragsN<NB>& f) {
  const int jn = lane & 15;
  const int kg = lane >> 4;
  {
    const int i = min(lane >> 2, NB - 1);
    const int st = st0 + i * kProd;
    const int sc = st < un.steps ? st : max(un.steps - 1, 0);
    const uint16_t* xp = p.x + int64_t(un.t) * p.x_stride + un.kb + 32 * sc + 8 * (lane & 3);
    f.xc = global_load128_untracked_masked(xp, NB == 16 ? ~0ull : (uint64_t(1) << (4 * NB)) - 1);
  }
  const int j = jn;
  const uint16_t* arow = p.a_store + un.aoff + int64_t(j < un.rows ? j : un.rows - 1) * p.k + un.kb + 8 * kg;
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int st = st0 + i * kProd;
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
template <int NB>
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
    c = mfma16(vec_bf16x8(row0 && st0 + i * kProd < un.steps ? x : zero), vec_bf16x8(f.av[i]), c);
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

// Contraction wave w (< kProd) sums the MFMA steps w, w + kProd, ... of
// every 16-row group of the workgroup's first unit into red[w][j] (j < rows;
// higher j are never read). pre holds the first batch of row group 0 (already
// landed); anything beyond it is loaded here. Then the wave counts itself
// in (LDS) so the LoRA wave can publish without a workgroup barrier.
template <int NB>
__device__ void first_unit_partials(const GemvParams& p, const Unit& un, FirstFragsN<NB>& pre, float* red, int* done,
                                    int wave, int lane) {
  tie_frags(pre);
  const int jn = lane & 15;
  const int kg = lane >> 4;
  for (int j0 = 0; j0 < un.rows; j0 += 16) {
    f32x4 c = {0.f, 0.f, 0.f, 0.f};
    int st0 = wave;
    if (j0 == 0) {
      c = first_mfma(pre, un, st0, lane, c);
      st0 += NB * kProd;
    }
    // Anything beyond the first batch (ranks above 16, long slices) in small
    // batches: this runs inside the base loop, where registers are scarce.
    for (; st0 < un.steps; st0 += 2 * kProd) {
      UnitFragsN<2> f;
      unit_frags<false>(p, un, j0, st0, kProd, lane, f);
      c = unit_mfma(f, un, st0, kProd, c);
    }
    // Row 0 of C (lanes 0..15, element 0) holds this wave's partial of z[j].
    if (kg == 0) red[wave * 192 + j0 + jn] = c[0];
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the partial rows are in LDS
  if (lane == 0) __hip_atomic_fetch_add(done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// The LoRA wave: waits (LDS) until the contraction waves have written the
// first unit's partial rows, sums and stores them with the call's tag.
__device__ void publish_first_unit(const GemvParams& p, const float* red, const int* done, const Unit& un,
                                   uint32_t tag, int lane) {
  const int rows = un.rows;
  for (int spins = 0; __hip_atomic_load(done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < kProd; ++spins) {
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
      for (int w = 0; w < kProd; ++w) v += red[w * 192 + jj];
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

// LDS of the LoRA stages, an array that never receives direct copies (so
// stores into it do not wait for copies in flight): the tile metadata and z.
template <class TL>
struct LoraLds {
  static constexpr int kMeta = 0;
  static constexpr int kZ = 2048;  // z: [tile token][3 slices][64] bf16
  static constexpr int kBytes = kZ + TL::kXR * 192 * 2;
  static_assert(sizeof(TileMeta) <= 2048, "tile metadata");
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
  m.g = lane < mt ? g : -1;
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

template <class TL, int KZ>
__device__ bool lora_gather_kz(const GemvParams& p, char* lds, int t0, int mt, uint32_t tag, int lane) {
  using L = LoraLds<TL>;
  // Values per lane and batch (16 entries; 8 for the tiles of up to 8
  // tokens, which keeps them at two workgroups per CU).
  constexpr int kEntries = TL::kRT == 1 && TL::kXR <= 8 ? 8 : 16;
  constexpr int kOut = kEntries / KZ > 0 ? kEntries / KZ : 1;
  const TileMeta* tm = reinterpret_cast<const TileMeta*>(lds + L::kMeta);
  uint16_t* zl = reinterpret_cast<uint16_t*>(lds + L::kZ);
  for (int e = lane; e < TL::kXR * 192 / 8; e += 64) reinterpret_cast<uint4*>(zl)[e] = make_uint4(0, 0, 0, 0);
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
      if (need[q] && s < p.slices) zl[(i * 3 + s) * 64 + (j - s * ri)] = uint16_t(f32_to_bf16(z));
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
    zl[(i * 3 + s) * 64 + (j - s * ri)] = uint16_t(f32_to_bf16(full_dot(p, t0 + i, tm->g[i], j)));
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

// Expand on MFMA, by the contraction waves (the LoRA wave finishes z last):
// wave w takes the tile's distinct slots w, w + 7, ...; for each, delta[token][column] += z[token][s*64 + j] * B_g[column][j]
// over ranks in steps of 32, with z rows of other slots' tokens masked to
// zero, into tiles of the base layout (token rows x 16 columns). Columns of
// other slices are masked on the B side. B fragments go kSlotBatch slots
// at a time, so one batch covers the distinct slots of a tile; it is
// requested as soon as the wave has finished its contraction and is
// shifted and masked (expand_b_fix) before the wait for z, so both its
// latency and that VALU work overlap the wait.
constexpr int kExpandWaves = kWaves - 1;
// Slots per wave and batch: enough for one batch to cover the at most
// min(tile tokens, 32) distinct slots of a tile, and no more (every slot of a
// batch is unrolled code that each workgroup runs once, after its weight
// stream; c1 10.6 -> 10.2 us with one slot per wave instead of five).
template <class TL>
constexpr int kSlotBatch = (TL::kXR + kExpandWaves - 1) / kExpandWaves;

template <class TL>
struct ExpandB {
  uint4 bf[kSlotBatch<TL>][TL::kRT];  // ranks 0..31 (ranks 32..63 are loaded where used)
};

template <class TL>
__device__ __forceinline__ void expand_b_batch(const GemvParams& p, const TileMeta* tm, ExpandB<TL>& b, int d0,
                                               int lo, int hi, int lane) {
  const int n = lane & 15;
  const int kg = lane >> 4;
  const int nd = tm->nd;
#pragma unroll
  for (int q = 0; q < kSlotBatch<TL>; ++q) {
    const int d = d0 + q * kExpandWaves;
    const bool live = d < nd;
    const int dd = live ? d : 0;
#pragma unroll
    for (int r = 0; r < TL::kRT; ++r)
      // Raw 16 bytes only: the shift/mask (b8_fix) is applied where the
      // fragments are used, so nothing waits for these loads here.
      b.bf[q][r] = *reinterpret_cast<const uint4*>(
          b8_at(p, tm->dboff[dd], tm->dstride[dd], tm->dr[dd], grow<TL>(lo, hi, r * 16 + n), 8 * kg, live).src);
  }
}

// Shifts and masks a landed batch in place (b8_fix with the addresses the
// loads used): ranks 0..31 of each slot, ready for the MFMAs. The contraction
// waves do this before waiting for z, so the VALU work is off the path.
template <class TL>
__device__ __forceinline__ void expand_b_fix(const GemvParams& p, const TileMeta* tm, ExpandB<TL>& b, int d0,
                                             int lo, int hi, int lane) {
  const int n = lane & 15;
  const int kg = lane >> 4;
  const int nd = tm->nd;
#pragma unroll
  for (int q = 0; q < kSlotBatch<TL>; ++q) {
    const int d = d0 + q * kExpandWaves;
    if (d >= nd) break;  // uniform
    const int st = tm->dstride[d];
    const int cnt = min(8, tm->dr[d] - 8 * kg);  // elements kept (<= 0: none)
    if (st >= 8) {
      // Aligned rows (the common case): only the elements past the rank go.
#pragma unroll
      for (int r = 0; r < TL::kRT; ++r) b.bf[q][r] = keep_first(b.bf[q][r], cnt);
    } else {
      const int boff = int(tm->dboff[d] & 7);
#pragma unroll
      for (int r = 0; r < TL::kRT; ++r)
        b.bf[q][r] = b8_fix(b.bf[q][r], B8{nullptr, (boff + grow<TL>(lo, hi, r * 16 + n) * st + 8 * kg) & 7, cnt});
    }
  }
}

// Waits (LDS flag) for the LoRA wave's slot list, then requests this wave's
// first batch of B fragments.
template <class TL>
__device__ __forceinline__ void expand_b_first(const GemvParams& p, const char* lds7, ExpandB<TL>& b, int lo,
                                               int hi, int wave, int lane) {
  const TileMeta* tm = reinterpret_cast<const TileMeta*>(lds7 + LoraLds<TL>::kMeta);
  while (*(const volatile __attribute__((address_space(3))) int*)(&tm->ready) == 0) __builtin_amdgcn_s_sleep(1);
  expand_b_batch<TL>(p, tm, b, wave, lo, hi, lane);
}

template <class TL>
__device__ void expand_mfma(const GemvParams& p, const char* lds7, ExpandB<TL>& b, const int (&bounds)[4],
                            f32x4 (&dacc)[TL::kRT][TL::kTT], int lo, int hi, int wave, int lane) {
  using L = LoraLds<TL>;
  constexpr int RT = TL::kRT;
  constexpr int TT = TL::kTT;
  const TileMeta* tm = reinterpret_cast<const TileMeta*>(lds7 + L::kMeta);
  const uint16_t* zl = reinterpret_cast<const uint16_t*>(lds7 + L::kZ);
  const int n = lane & 15;
  const int kg = lane >> 4;
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int t = 0; t < TT; ++t) dacc[r][t] = (f32x4){0.f, 0.f, 0.f, 0.f};
  const int nd = tm->nd;
  int cs[RT];  // slice of this lane's column in each row tile
  auto slice_of = [&](int col) { return int(p.slices > 1 && col >= bounds[1]) + int(p.slices > 2 && col >= bounds[2]); };
#pragma unroll
  for (int r = 0; r < RT; ++r) cs[r] = slice_of(grow<TL>(lo, hi, r * 16 + n));
  // Slices the group's rows touch: its smallest row is lo, its largest hi + R / 2 - 1.
  const int top = hi + TL::kR / 2 - 1;
  const int s_lo = int(p.slices > 1 && lo >= bounds[1]) + int(p.slices > 2 && lo >= bounds[2]);
  const int s_hi = int(p.slices > 1 && top >= bounds[1]) + int(p.slices > 2 && top >= bounds[2]);
  for (int d0 = wave; d0 < nd; d0 += kSlotBatch<TL> * kExpandWaves) {
    if (d0 != wave) {
      expand_b_batch<TL>(p, tm, b, d0, lo, hi, lane);
      expand_b_fix<TL>(p, tm, b, d0, lo, hi, lane);
    }
#pragma unroll
    for (int q = 0; q < kSlotBatch<TL>; ++q) {
      const int d = d0 + q * kExpandWaves;
      if (d >= nd) break;  // uniform
      const int g = tm->dslot[d];
      const int rk = tm->dr[d];
      for (int s = s_lo; s <= s_hi; ++s) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          if (32 * h >= rk) break;  // uniform
          uint4 zf[TT];
#pragma unroll
          for (int t = 0; t < TT; ++t) {
            const int tok = t * 16 + n;
            const int tz = min(tok, TL::kXR - 1);
            const uint4 v = *reinterpret_cast<const uint4*>(zl + (tz * 3 + s) * 64 + 32 * h + 8 * kg);
            zf[t] = tm->g[tok] == g ? v : make_uint4(0, 0, 0, 0);
          }
#pragma unroll
          for (int r = 0; r < RT; ++r) {
            uint4 fixed = b.bf[q][r];  // ranks 0..31: shifted and masked already
            if (h == 1) {
              const B8 b8 = b8_at(p, tm->dboff[d], tm->dstride[d], rk, grow<TL>(lo, hi, r * 16 + n), 32 + 8 * kg, true);
              fixed = b8_fix(*reinterpret_cast<const uint4*>(b8.src), b8);
            }
            const uint4 bb = cs[r] == s ? fixed : make_uint4(0, 0, 0, 0);
#pragma unroll
            for (int t = 0; t < TT; ++t) dacc[r][t] = mfma16(as_bf16x8(zf[t]), as_bf16x8(bb), dacc[r][t]);
          }
        }
      }
    }
  }
}

// Copies of one stage (kSB blocks starting at block kb) into a ring slot.
// W: position p -> block p / (2R), row (p / 2) % R, 16-byte half p % 2, so a
// block's rows are 32 contiguous bytes each. x: position p -> token row
// p / (8 kSB), block (p / 8) % kSB, unit slot p % 8 holding 16-byte unit
// (p % 8) ^ (row & 7) (conflict-free fragment reads). Scales (tiles without
// kScPre): position p -> block p / R, row p % R. Positions past the stage and
// blocks past the wave's range read valid addresses of block kb (their scale
// is zeroed when used). kb must be a valid block.
template <class TL>
__device__ __forceinline__ void issue_stage(const GemvParams& p, char* slot, int lo, int hi, int t0, int mt, int kb,
                                            int kend, int lane) {
  const int nblk = p.k >> 6;
#pragma unroll
  for (int d = 0; d < TL::kWDma; ++d) {
    const int pos = d * 64 + lane;
    const int b = pos / (2 * TL::kR);
    const int r = (pos >> 1) % TL::kR;
    const int blk = (pos < 2 * TL::kR * TL::kSB && kb + b < kend) ? kb + b : kb;
    copy16(p.q + int64_t(grow<TL>(lo, hi, r)) * (p.k >> 1) + blk * 32 + (lane & 1) * 16, slot + d * 1024);
  }
#pragma unroll
  for (int d = 0; d < TL::kXDma; ++d) {
    const int pos = d * 64 + lane;
    int row = pos / (8 * TL::kSB);
    const int b = (pos / 8) % TL::kSB;
    const int u = (pos & 7) ^ (row & 7);
    int blk = kb + b < kend ? kb + b : kb;
    if (row >= TL::kXR) row = 0;
    const int tok = t0 + (row < mt ? row : mt - 1);
    copy16(p.x + int64_t(tok) * p.x_stride + blk * 64 + u * 8, slot + TL::kWBytes + d * 1024);
  }
  if constexpr (!TL::kScPre) {
    const int b = lane / TL::kR;
    const int r = lane % TL::kR;
    const int blk = (lane < TL::kR * TL::kSB && kb + b < kend) ? kb + b : kb;
    copy4(p.scales + int64_t(grow<TL>(lo, hi, r)) * nblk + (blk < nblk ? blk : 0), slot + TL::kWBytes + TL::kXBytes);
  }
}

// kScPre: the block scales of the group's 16 rows over the wave's blocks
// kb0 .. kb0 + nbw - 1 into its scale area (row j at j * stride floats), as
// dword copies of 64 consecutive floats. Padding positions read a valid scale
// of the range (never used). kb0 must be a valid block.
template <class TL>
__device__ __forceinline__ void issue_scales(const GemvParams& p, char* area, int lo, int hi, int kb0, int nbw,
                                             int lane) {
  const int nblk = p.k >> 6;
  for (int i = 0; i < p.sc_bytes / 256; ++i) {
    const int pos = i * 64 + lane;
    int row = pos / p.sc_stride;
    int col = pos - row * p.sc_stride;
    if (row > TL::kR - 1) row = TL::kR - 1;
    if (col >= nbw) col = 0;
    copy4(p.scales + int64_t(grow<TL>(lo, hi, row)) * nblk + kb0 + col, area + i * 256);
  }
}

// kResidual (with kLora): no weight. The base of each output is its current
// value in y, which the call updates in place with the LoRA delta
// (y = bf16(bf16(y) + bf16(scale * z B^T)), the row_shrink + row_expand chain
// in one launch); no weight stream, no bias.
// Tile<1, 2> fits two workgroups per CU in LDS; its launch bounds ask for
// the registers of two (four waves per SIMD), so one workgroup's prologue
// and epilogue overlap the other's weight stream when N spans several rounds
// of workgroups.
template <int RT, int XR>
constexpr int kMinWavesPerSimd = (RT == 1 && XR <= 8) ? 4 : 2;

template <int RT, int XR, bool kExact, bool kLora, bool kResidual, bool kSP>
__global__ __launch_bounds__(kThreads, (kMinWavesPerSimd<RT, XR>)) void nf4_gemv_kernel(GemvParams p) {
  using TL = Tile<RT, XR, kSP>;
  constexpr int TT = TL::kTT;
  constexpr int D = TL::kDepth;
  constexpr int kBase = kLora ? kWaves - 1 : kWaves;  // waves on the base contraction (ring owners)
  static_assert(D * TL::kStage >= 2 * RT * TT * 1024, "base and expand tiles fit a ring region");
  __shared__ __attribute__((aligned(16))) char ring[kBase * D * TL::kStage];
  __shared__ __attribute__((aligned(16))) char lora_lds[kLora ? LoraLds<TL>::kBytes : 16];
  __shared__ float table[16];
  __shared__ __attribute__((aligned(16))) uint32_t pt[kExact ? 4 : 256 * kCopies];
  __shared__ float red[kLora ? kProd * 192 : 1];
  __shared__ int prod_done;  // contraction waves that have written their first-unit partials
  __shared__ f32x4 up_vals[RT == 2 ? TL::kTT * 64 : 1];  // SwiGLU output: the up tile's final values
  extern __shared__ __attribute__((aligned(16))) char scale_lds[];  // kScPre: kBase * p.sc_bytes (+16)

  const int rg = blockIdx.x % p.row_groups;
  const int tile = blockIdx.x / p.row_groups;
  // The group's rows: R contiguous rows, or in SwiGLU-output mode R / 2 gate
  // rows and the R / 2 up rows of the same features.
  const int lo = p.gated_half ? rg * (TL::kR / 2) : rg * TL::kR;
  const int hi = p.gated_half ? p.gated_half + lo : lo + TL::kR / 2;
  const int t0 = tile * 32;
  const int mt = min(32, p.m - t0);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int nblk = p.k >> 6;
  const int kb0 = wave < kBase ? nblk * wave / kBase : 0;
  const int kend = wave < kBase ? nblk * (wave + 1) / kBase : 0;
  const int nst = kResidual ? 0 : (kend - kb0 + TL::kSB - 1) / TL::kSB;
  char* myring = ring + wave * D * TL::kStage;  // waves below kBase only
  char* myscales = scale_lds + wave * p.sc_bytes;  // kScPre, waves below kBase only
  static_assert(!kResidual || (kLora && !kExact), "the residual form is a LoRA-only variant");

  // Codebook (and the LoRA slice bounds) through scalar loads: no vector
  // load may wait behind the copies.
  float cb[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) cb[i] = kResidual ? 0.f : sload(p.code, i);
  int bounds[4] = {0, 0, 0, 0};
  if constexpr (kLora) {
#pragma unroll
    for (int q = 0; q < 4; ++q) bounds[q] = q <= p.slices ? sload(p.slice_offsets, q) : 0;
  }

  // Weight stages (the contraction waves; blocks clamped into range, so all
  // D stages are always requested). A producing workgroup requests its first
  // shrink unit's fragments ahead of the stages (untracked loads): at small
  // batches the D stages are most of the weight stream, and fragments queued
  // behind them would land only near its end. The contraction waves compute
  // the unit's partials before their first stage.
  Unit un0{};
  bool has0 = false;
  // Fragments of the first unit's first batch: ten steps per wave, four for
  // the smallest tile (B <= 2, whose units span at most 28 steps at K up to
  // 14336), which keeps that tile at two workgroups per CU.
  constexpr int kFirst = (RT == 1 && XR <= 8) ? 4 : kBatch;
  FirstFragsN<kFirst> pre;
  TokenMeta tmeta{};
  uint32_t epoch = 0;
  int g_tile = -1;  // the LoRA wave: token slots loaded in the prologue
  if (wave < kBase) {
    auto stage_kb = [&](int s) { return min(kb0 + s * TL::kSB, nblk - 1); };
    // kScPre: the wave's scales first (the wait for its first stage covers
    // them, and the unit's fragments are not queued behind them for long).
    if constexpr (TL::kScPre && !kResidual) issue_scales<TL>(p, myscales, lo, hi, kb0, kend - kb0, lane);
    if constexpr (kLora) {
      has0 = int(blockIdx.x) < p.producers && int(blockIdx.x) < p.units && unit_of(p, blockIdx.x, un0);
      if (has0) first_frags(p, un0, wave, lane, pre);
    }
    if constexpr (kLora && !kResidual) {
      // Workgroups that produce no unit hold their weight stream back by
      // about a microsecond (32 x 64 cycles), so the producers' unit
      // fragments are ahead of it in the memory queues; producers hold
      // their own stages back by half that, behind their fragments. The
      // tiles of up to 8 tokens hold back 24 x 64 cycles (12 for producers):
      // with the block scales in LDS, c1 9.78 / 9.80 / 9.86 / 9.99 us for
      // 24 / 32 / 48 / 64 x 64 (B = 64: 18.2 / 17.9 / 18.1 / 18.4 / 19.0 us
      // for no delay / 32 / 48 / 64 / 96 x 64, measured on an older stage
      // layout).
      // Workgroups of later dispatch rounds start after the producers have
      // published and do not wait.
      if (int(blockIdx.x) < p.resident) {
        if (kMinWavesPerSimd<RT, XR> > 2) {
          if (!has0) __builtin_amdgcn_s_sleep(24);
          else __builtin_amdgcn_s_sleep(12);
        } else {
          if (!has0) __builtin_amdgcn_s_sleep(32);
          else __builtin_amdgcn_s_sleep(16);
        }
      }
    }
    if constexpr (!kResidual) {
#pragma unroll
      for (int s = 0; s < D; ++s) issue_stage<TL>(p, myring + s * TL::kStage, lo, hi, t0, mt, stage_kb(s), kend, lane);
    }
  } else if constexpr (kLora) {
    // The LoRA wave: the epoch and the first loads of its metadata chains
    // (vector loads: the barriers below wait only for scalar loads and LDS,
    // so the whole workgroup does not wait for these round trips); the
    // dependent loads follow the barriers.
    epoch = __hip_atomic_load(p.ce.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    g_tile = p.token_slots[t0 + min(lane, mt - 1)];
  }
  // Residual form: the summing waves (one per 16 x 16 tile) fetch the outputs
  // they will update now; nothing uses them before the end.
  float yold[4] = {0.f, 0.f, 0.f, 0.f};
  if constexpr (kResidual) {
    if (wave < RT * TL::kTT) {
      const int col = grow<TL>(lo, hi, (wave / TL::kTT) * 16 + (lane & 15));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = (wave % TL::kTT) * 16 + 4 * (lane >> 4) + e;
        yold[e] = bf16_to_f32(p.y[int64_t(t0 + min(i, mt - 1)) * p.y_stride + col]);
      }
    }
  }

  if (threadIdx.x == 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) table[i] = cb[i];
    if constexpr (kLora) {
      reinterpret_cast<TileMeta*>(lora_lds + LoraLds<TL>::kMeta)->ready = 0;
      prod_done = 0;
    }
  }
  if constexpr (!kExact) {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    barrier_only();
    if (threadIdx.x < 256) {
      const uint32_t v = pack_bf16x2(table[threadIdx.x >> 4], table[threadIdx.x & 15]);
      uint4* dst = reinterpret_cast<uint4*>(pt + threadIdx.x * kCopies);
#pragma unroll
      for (int c = 0; c < kCopies / 4; ++c) dst[c] = make_uint4(v, v, v, v);
    }
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);
  barrier_only();
  const uint32_t* ptl = pt + (lane % kCopies);
  // The LoRA wave: the first unit (found through scalar loads and published
  // as soon as the contraction waves have counted in), then the tile
  // metadata (its loads are requested first and land meanwhile), the other
  // units, then z.
  if constexpr (kLora) {
    if (wave == kBase) {
      tmeta = token_meta(p, g_tile, mt, lane);
      has0 = int(blockIdx.x) < p.producers && int(blockIdx.x) < p.units && unit_of(p, blockIdx.x, un0);
      const uint32_t tag = __builtin_amdgcn_readfirstlane(epoch) + 1u;
      if (has0) publish_first_unit(p, red, &prod_done, un0, tag, lane);
      lora_meta<TL>(lora_lds, tmeta, p.slices, lane);
      produce_other_units<kFirst>(p, tag, lane);
    }
  }

  f32x4 acc[RT][TT];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[r][t] = (f32x4){0.f, 0.f, 0.f, 0.f};

  const int n = lane & 15;
  const int g = lane >> 4;
  const uint32_t ring_base = lds_addr(myring);
  // Fragments of stage s + 1 are read from the ring while stage s is decoded
  // and contracted; the slot of stage s is refilled as soon as its fragments
  // are in registers.
  Frags<TL> cur, nxt;
  ExpandB<TL> eb;
  static_assert(D * TL::kDma < 64, "vmcnt range");
  if constexpr (kLora) {
    // The unit's fragments were requested before the D stages: they have
    // landed once only the stages are outstanding.
    if (wave < kBase && has0) {
      wait_vm<kResidual ? 0 : D * TL::kDma>();
      first_unit_partials(p, un0, pre, red, &prod_done, wave, lane);
    }
  }
  // Scales of stage s: kScPre tiles read the wave's scale area (block
  // kb0 + s kSB onwards), the others the stage's slot.
  const uint32_t sc_base = lds_addr(myscales);
  const uint32_t sc_rs = uint32_t(p.sc_stride) * 4;
  auto scb_of = [&](int s) -> uint32_t {
    if constexpr (TL::kScPre) return sc_base + uint32_t(s * TL::kSB) * 4;
    else return ring_base + (s % D) * TL::kStage + TL::kWBytes + TL::kXBytes;
  };
  // kAhead: stage s + 1's fragments are read while stage s is contracted
  // (D - 1 stages stream meanwhile); otherwise each stage's fragments are read
  // at the top of its step and its slot refilled at once (D stages stream).
  // With the scales in LDS every stage streams (the 4-block stages would not
  // fit two fragment sets in registers either): c3 down projection
  // 17.2 -> 14.6 us at B = 1, 20.2 -> 17.9 us at B = 8; north-star B = 64
  // 18.4 -> 18.1 us (base only 11.8 -> 10.9 us).
  constexpr bool kAhead = !TL::kScPre;
  if constexpr (kAhead) {
    if (nst > 0) {
      wait_stages<TL>(min(D - 1, nst - 1));
      read_frags<TL>(cur, ring_base, scb_of(0), sc_rs, n, g);
      settle(cur);
    }
    // One ring stage: read the next stage's fragments, refill, contract this
    // one.
    auto step = [&](int s) {
      const bool more = s + 1 < nst;
      if (more) {
        wait_stages<TL>(min(D - 2, nst - 2 - s));
        read_frags<TL>(nxt, ring_base + ((s + 1) % D) * TL::kStage, scb_of(s + 1), sc_rs, n, g);
      }
      if (s + D < nst)
        issue_stage<TL>(p, myring + (s % D) * TL::kStage, lo, hi, t0, mt, kb0 + (s + D) * TL::kSB, kend, lane);
      contract<TL, kExact>(cur, kb0 + s * TL::kSB, kend, acc, table, ptl);
      if (more) {
        settle(nxt);
        cur = nxt;
      }
    };
    for (int s = 0; s < nst; ++s) step(s);
  } else {
    for (int s = 0; s < nst; ++s) {
      wait_stages<TL>(min(D - 1, nst - 1 - s));
      read_frags<TL>(cur, ring_base + (s % D) * TL::kStage, scb_of(s), sc_rs, n, g);
      settle(cur);
      if (s + D < nst)
        issue_stage<TL>(p, myring + (s % D) * TL::kStage, lo, hi, t0, mt, kb0 + (s + D) * TL::kSB, kend, lane);
      contract<TL, kExact>(cur, kb0 + s * TL::kSB, kend, acc, table, ptl);
    }
  }

  // Sum the waves' partial tiles: wave w writes its tiles into its own ring
  // (all of its copies have landed), then tile c = wave is summed by wave c.
  // With LoRA the last wave prepares z meanwhile, then every contraction
  // wave adds its share of the expand into a second tile set after its base
  // tiles.
  constexpr int kTiles = RT * TT;
  char* lora7 = lora_lds;
  uint32_t departed = 0;
  auto delta_tiles = [&](int w) { return reinterpret_cast<f32x4*>(ring + w * D * TL::kStage + kTiles * 1024); };
  if constexpr (kLora) {
    // The LoRA wave finishes z while the others request their first B
    // fragments; after the barrier (LDS only: a full fence would wait for the
    // B loads) the contraction waves compute the expand in registers.
    f32x4 dacc[RT][TT];
    if (wave == kBase) {
      lora_gather<TL>(p, lora7, t0, mt, __builtin_amdgcn_readfirstlane(epoch) + 1u, lane);
      departed = depart_issue(p.ce, lane);  // after the last partial load: nothing waits for it until the end
    } else {
      expand_b_first<TL>(p, lora7, eb, lo, hi, wave, lane);
      expand_b_fix<TL>(p, reinterpret_cast<const TileMeta*>(lora7 + LoraLds<TL>::kMeta), eb, wave, lo, hi, lane);
    }
    lds_barrier();  // z and the tile metadata are in LDS
    if (wave < kBase) expand_mfma<TL>(p, lora7, eb, bounds, dacc, lo, hi, wave, lane);
    if (wave < kBase) {
      wait_vm<0>();  // stages past the wave's blocks (short K) may still be landing in the ring
      f32x4* base_tiles = reinterpret_cast<f32x4*>(myring);
      f32x4* dt = delta_tiles(wave);
#pragma unroll
      for (int r = 0; r < RT; ++r)
#pragma unroll
        for (int t = 0; t < TT; ++t) {
          base_tiles[(r * TT + t) * 64 + lane] = acc[r][t];
          dt[(r * TT + t) * 64 + lane] = dacc[r][t];
        }
    }
  } else {
    wait_vm<0>();  // stages past the wave's blocks (short K) may still be landing in the ring
    f32x4* base_tiles = reinterpret_cast<f32x4*>(myring);
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int t = 0; t < TT; ++t) base_tiles[(r * TT + t) * 64 + lane] = acc[r][t];
  }
  lds_barrier();
  const bool summer = wave < kTiles;  // wave c sums tile (r, t) = (c / TT, c % TT)
  const int r = summer ? wave / TT : 0;
  const int t = summer ? wave % TT : 0;
  f32x4 out = {0.f, 0.f, 0.f, 0.f};  // the tile's final values (bf16, as stored)
  if (summer) {
    f32x4 sum = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kBase; ++w) {
      const f32x4 v = reinterpret_cast<const f32x4*>(ring + w * D * TL::kStage)[wave * 64 + lane];
#pragma unroll
      for (int e = 0; e < 4; ++e) sum[e] += v[e];
    }
    f32x4 dsum = {0.f, 0.f, 0.f, 0.f};
    if constexpr (kLora) {
#pragma unroll
      for (int w = 0; w < kBase; ++w) {
        const f32x4 v = delta_tiles(w)[wave * 64 + lane];
#pragma unroll
        for (int e = 0; e < 4; ++e) dsum[e] += v[e];
      }
    }
    const TileMeta* tm = reinterpret_cast<const TileMeta*>(lora7 + LoraLds<TL>::kMeta);
    const int col = grow<TL>(lo, hi, r * 16 + n);
    const float bias = p.bias ? bf16_to_f32(p.bias[col]) : 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int i = t * 16 + 4 * g + e;  // tile token
      float v = kResidual ? yold[e] : round_bf16(sum[e]);
      if (!kResidual && p.bias) v = round_bf16(v + bias);
      if constexpr (kLora) {
        if (i < mt && tm->g[i] >= 0) v += round_bf16(dsum[e] * tm->scale[i]);
      }
      out[e] = round_bf16(v);
      if (!p.gated_half && i < mt) p.y[int64_t(t0 + i) * p.y_stride + col] = uint16_t(f32_to_bf16(v));
    }
  }
  if (p.gated_half) {
    // SwiGLU output h[token][f] = bf16(bf16(silu(gate)) * up) for the group's
    // features f = lo .. lo + R / 2 (the reference's activation after both
    // LoRA adds, benchmarks/qwen35_decode_silu.py:60-61).
    f32x4 up = {0.f, 0.f, 0.f, 0.f};
    bool gate = false;
    if constexpr (RT == 1) {
      // Lanes n < 8 hold gate rows lo + n, lanes n + 8 the matching up rows.
#pragma unroll
      for (int e = 0; e < 4; ++e) up[e] = __shfl_xor(out[e], 8, 64);
      gate = summer && n < 8;
    } else {
      // Tile r = 0 holds the gate rows lo .. lo + 15, tile r = 1 the up rows.
      if (summer && r == 1) up_vals[t * 64 + lane] = out;
      lds_barrier();
      if (summer && r == 0) up = up_vals[t * 64 + lane];
      gate = summer && r == 0;
    }
    if (gate) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = t * 16 + 4 * g + e;
        if (i < mt) p.y[int64_t(t0 + i) * p.y_stride + lo + n] = uint16_t(f32_to_bf16(silu_times(out[e], up[e])));
      }
    }
  }
  if (kLora && wave == kBase) depart_finish(p.ce, departed, __builtin_amdgcn_readfirstlane(epoch), lane);
}

constexpr int64_t kLdsBytes = 160 * 1024;  // LDS of one workgroup on gfx950

// Static LDS bytes of a kernel (queried once per kernel).
template <class K>
int64_t static_lds_of(K fn, int64_t& cache) {
  if (cache < 0) {
    hipFuncAttributes at{};
    if (hipFuncGetAttributes(&at, reinterpret_cast<const void*>(fn)) != hipSuccess) return -1;
    cache = int64_t(at.sharedSizeBytes);
  }
  return cache;
}

// Launches the variant with the block scales in LDS (each contraction wave's
// area in dynamic LDS, 16 trailing bytes: the last area's stage reads may run
// up to 3 floats past it) when its static LDS and the areas fit, else the
// variant that stages the scales with the weights (very long K).
template <int RT, int XR, bool kExact, bool kLora>
int launch_scaled(dim3 grid, hipStream_t s, GemvParams p) {
  constexpr int kBase = kLora ? kWaves - 1 : kWaves;
  const ScaleArea a = scale_area(p.k >> 6, kBase, 16 * RT);
  const int64_t dyn = int64_t(kBase) * a.bytes + 16;
  static int64_t static_lds = -1;
  auto fn = nf4_gemv_kernel<RT, XR, kExact, kLora, false, true>;
  const int64_t st = static_lds_of(fn, static_lds);
  if (st >= 0 && st + dyn <= kLdsBytes) {
    p.sc_stride = a.stride;
    p.sc_bytes = a.bytes;
    hipLaunchKernelGGL(fn, grid, dim3(kThreads), size_t(dyn), s, p);
  } else {
    hipLaunchKernelGGL((nf4_gemv_kernel<RT, XR, kExact, kLora, false, false>), grid, dim3(kThreads), 0, s, p);
  }
  return kOk;
}

template <int RT, int XR>
int launch_tile(bool exact, bool lora, bool residual, dim3 grid, hipStream_t s, const GemvParams& p) {
  if (residual) {
    hipLaunchKernelGGL((nf4_gemv_kernel<RT, XR, false, true, true, false>), grid, dim3(kThreads), 0, s, p);
    return kOk;
  }
  if (lora) return exact ? launch_scaled<RT, XR, true, true>(grid, s, p) : launch_scaled<RT, XR, false, true>(grid, s, p);
  return exact ? launch_scaled<RT, XR, true, false>(grid, s, p) : launch_scaled<RT, XR, false, false>(grid, s, p);
}

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

}  // namespace

// Compute units of the current device (cached per device).
int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

int64_t gemv_workspace_bytes(int64_t, int64_t, int64_t, int, int) { return kWorkspaceHeader; }

// Fused NF4 + multi-LoRA linear for 1..64 tokens with fp32 block scales.
// residual: no weight (only w->n and w->k are read) and a LoRA batch: y is
// updated in place with each routed token's LoRA delta.
int launch_nf4_gemv(const uint16_t* x, int64_t m, int64_t x_stride, const lf_nf4_weight* w, const uint16_t* bias,
                    const lf_lora* lora, uint16_t* y, int64_t y_stride, void* workspace, int64_t workspace_bytes,
                    bool exact, bool swiglu, bool withhold, void* stream, bool residual) {
  LF_REQUIRE(m >= 1 && m <= 64, "decode path handles 1..64 tokens");
  LF_REQUIRE(residual || w->scales != nullptr, "decode takes fp32 block scales (prepare double-quant scales first)");
  LF_REQUIRE(!residual || (lora && !bias && !swiglu && !exact), "the residual form takes a LoRA batch and nothing else");
  const GemvPlan pl = gemv_plan(m, w->n, w->k, device_cus(), lora ? lora->num_slices * lora->max_rank : 1);
  LF_REQUIRE(w->n % pl.rows == 0, "output width must be a multiple of %d", pl.rows);
  GemvParams p{};
  p.x = x;
  p.x_stride = x_stride;
  p.m = int(m);
  p.q = w->qweight;
  p.scales = w->scales;
  p.code = w->code;
  p.n = int(w->n);
  p.k = int(w->k);
  p.bias = bias;
  p.y = y;
  p.y_stride = y_stride;
  p.row_groups = pl.row_groups;
  p.gated_half = swiglu ? int(w->n / 2) : 0;  // n % 32 == 0: R / 2 divides n / 2
  if (lora) {
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
    p.zw = lora->num_slices * lora->max_rank;
    p.units = pl.units;
    p.kz = pl.kz;
    p.usplit = pl.usplit;
    p.urows = pl.urows;
    p.unit_inv = ((1u << 21) + uint32_t(pl.usplit * pl.kz) - 1) / uint32_t(pl.usplit * pl.kz);
    LF_REQUIRE(pl.units <= 1024, "too many shrink units");
    p.kz_len = pl.kz_len;
    p.producers = pl.producers;
    // Tiles of at most 8 tokens run two workgroups per CU.
    p.resident = std::min(pl.grid, device_cus() * (m <= 8 ? 2 : 1));
    char* ws = static_cast<char*>(workspace);
    p.ce = call_epoch_of(ws);
    p.status = reinterpret_cast<int*>(ws + kStatusOffset);
    p.withhold = withhold ? 1 : 0;
    p.spin_limit = withhold ? 64 : kSpinLimit;
    p.zp = reinterpret_cast<uint64_t*>(ws + kPartialsOffset);
  }
  const dim3 grid(unsigned(pl.grid));
  auto s = static_cast<hipStream_t>(stream);
  const bool lo = lora != nullptr;
  int rc;
  if (m <= 2) rc = launch_tile<1, 2>(exact, lo, residual, grid, s, p);
  else if (m <= 8) rc = launch_tile<1, 8>(exact, lo, residual, grid, s, p);
  else if (m <= 16) rc = launch_tile<1, 16>(exact, lo, residual, grid, s, p);
  else if (m <= 32) rc = launch_tile<1, 32>(exact, lo, residual, grid, s, p);
  else rc = launch_tile<2, 32>(exact, lo, residual, grid, s, p);
  if (rc != kOk) return rc;
  LF_HIP(hipGetLastError());
  return kOk;
}

}  // namespace lf
