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

#include "decode_lora.h"

namespace lf {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kCopies = 16;  // pair-table copies (lane l reads copy l % 16)
constexpr int kProd = kWaves - 1;  // contraction waves: they compute the shrink partials
constexpr int kBatch = 10;         // MFMA steps per wave and batch (kProd * kBatch >= 64 steps)

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

// Double quant: columns of its row a lane converts, at most (16-row groups
// take four lanes a row, 32-row groups two).
template <int RT>
constexpr int kDqCols = RT == 1 ? 8 : 16;

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
  __shared__ int dq_ready;  // double quant: wave 0's code2 copies have landed
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
  // Double quant (kScPre): code2 after the scale areas (1 KiB of dynamic LDS
  // that only those launches allocate).
  float* dq_table = reinterpret_cast<float*>(scale_lds + kBase * p.sc_bytes + 16);
  const bool dq = TL::kScPre && !kResidual && p.absmax_q != nullptr;
  float dq_off = 0.f;
  DqStage dqs{};
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
    if constexpr (TL::kScPre && !kResidual) {
      if (dq) {
        // Double quant: code2 (wave 0, ahead of everything), then the
        // wave's codes and absmax2 entries instead of fp32 scales.
        if (wave == 0) dq_issue_code2(p, dq_table, lane);
        dq_off = sload(p.dq_offset, 0);
        dqs = dq_stage(p, p.sc_bytes, TL::kR, lo, hi, kb0, kend - kb0);
        dq_issue(p, myscales, dqs, TL::kR, lo, hi, kb0, lane);
      } else {
        issue_scales<TL>(p, myscales, lo, hi, kb0, kend - kb0, lane);
      }
    }
    if constexpr (kLora) {
      has0 = int(blockIdx.x) < p.producers && int(blockIdx.x) < p.units && unit_of(p, blockIdx.x, un0);
      if (has0) first_frags<kFirst, kProd>(p, un0, wave, lane, pre);
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
    dq_ready = 0;  // set by wave 0 after the barrier below
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
      if (has0) publish_first_unit<kProd>(p, red, &prod_done, un0, tag, lane);
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
      first_unit_partials<kFirst, kProd>(p, un0, pre, red, &prod_done, wave, lane);
    }
  }
  if (dq && wave < kBase) {
    // The staging (and wave 0's code2 copies) came before the unit's
    // fragments and the D stages: it has landed once only the stages are
    // outstanding. Wave 0 then raises dq_ready; the others wait for it, with
    // a bound, before reading code2.
    wait_vm<D * TL::kDma>();
    if (wave == 0) {
      if (lane == 0) __hip_atomic_store(&dq_ready, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    } else {
      for (int spins = 0; spins < kSpinLimit &&
                          *(const volatile __attribute__((address_space(3))) int*)(&dq_ready) == 0;
           ++spins)
        __builtin_amdgcn_s_sleep(1);
    }
    dq_convert<kDqCols<RT>>(p, myscales, dqs, TL::kR, lo, hi, kb0, kend - kb0, dq_table, dq_off, lane);
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
  // Double quant: each area grows by the staging of the codes (past its fp32
  // entries), and the code2 table follows the areas.
  const int nbw = ((p.k >> 6) + kBase - 1) / kBase;
  const int area = a.bytes + (p.absmax_q ? dq_stage_bytes(16 * RT, nbw) : 0);
  const int64_t dyn = int64_t(kBase) * area + 16 + (p.absmax_q ? 1024 : 0);
  static int64_t static_lds = -1;
  auto fn = nf4_gemv_kernel<RT, XR, kExact, kLora, false, true>;
  const int64_t st = static_lds_of(fn, static_lds);
  if (st >= 0 && st + dyn <= kLdsBytes) {
    p.sc_stride = a.stride;
    p.sc_bytes = area;
    p.sc_magic = stride_magic(a.stride);
    hipLaunchKernelGGL(fn, grid, dim3(kThreads), size_t(dyn), s, p);
  } else {
    // (A nested state is only passed where the variant above fits.)
    LF_REQUIRE(p.absmax_q == nullptr, "decode: double-quant scales need the scales-in-LDS variant");
    hipLaunchKernelGGL((nf4_gemv_kernel<RT, XR, kExact, kLora, false, false>), grid, dim3(kThreads), 0, s, p);
  }
  return kOk;
}

// Whether the scales-in-LDS variant of a tile reads a nested state itself
// (dq_scales.h): the layout conditions, and the variant with its areas grown
// by the staging and the code2 table fitting LDS.
template <int RT, int XR, bool kExact, bool kLora>
bool dq_variant_ok(const lf_nf4_weight* w) {
  constexpr int kBase = kLora ? kWaves - 1 : kWaves;
  constexpr int kRows = 16 * RT;
  const int nblk = int(w->k >> 6);
  const ScaleArea a = scale_area(nblk, kBase, kRows);
  const int nbw = (nblk + kBase - 1) / kBase;
  if (!dq_layout_ok(w, kRows) || dq_cols_per_lane(kRows, a.stride) > kDqCols<RT>) return false;
  static int64_t static_lds = -1;
  const int64_t st = static_lds_of(nf4_gemv_kernel<RT, XR, kExact, kLora, false, true>, static_lds);
  return st >= 0 && st + int64_t(kBase) * (a.bytes + dq_stage_bytes(kRows, nbw)) + 16 + 1024 <= kLdsBytes;
}

template <int RT, int XR>
bool dq_tile_ok(const lf_nf4_weight* w, bool lora, bool exact) {
  if (lora) return exact ? dq_variant_ok<RT, XR, true, true>(w) : dq_variant_ok<RT, XR, false, true>(w);
  return exact ? dq_variant_ok<RT, XR, true, false>(w) : dq_variant_ok<RT, XR, false, false>(w);
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

// The control header with the tagged partials, then (after the prefill's flag
// region) room for fp32 scales rebuilt from a nested state.
int64_t gemv_workspace_bytes(int64_t, int64_t n, int64_t k, int, int) {
  return decode_scales_offset() + decode_scales_bytes(n, k);
}

int rebuild_decode_scales(const lf_nf4_weight* w, void* workspace, int64_t workspace_bytes, void* stream,
                          const float** scales) {
  return rebuild_scales(w, workspace, workspace_bytes, stream, scales);
}

// Whether the narrow kernel reads this nested state itself (the tile that
// launch_nf4_gemv picks for m tokens).
bool gemv_takes_dq(int64_t m, const lf_nf4_weight* w, const lf_lora* lora, bool exact) {
  const bool lo = lora != nullptr;
  if (m <= 2) return dq_tile_ok<1, 2>(w, lo, exact);
  if (m <= 8) return dq_tile_ok<1, 8>(w, lo, exact);
  if (m <= 16) return dq_tile_ok<1, 16>(w, lo, exact);
  if (m <= 32) return dq_tile_ok<1, 32>(w, lo, exact);
  return dq_tile_ok<2, 32>(w, lo, exact);
}

// Fused NF4 + multi-LoRA linear for 1..64 tokens with fp32 block scales.
// residual: no weight (only w->n and w->k are read) and a LoRA batch: y is
// updated in place with each routed token's LoRA delta.
int launch_nf4_gemv(const uint16_t* x, int64_t m, int64_t x_stride, const lf_nf4_weight* w, const uint16_t* bias,
                    const lf_lora* lora, uint16_t* y, int64_t y_stride, void* workspace, int64_t workspace_bytes,
                    bool exact, bool swiglu, bool withhold, void* stream, bool residual) {
  LF_REQUIRE(m >= 1 && m <= 64, "decode path handles 1..64 tokens");
  // A nested state: read by the kernel where its scales-in-LDS variant takes
  // it, else fp32 scales rebuilt into the workspace.
  const float* scales = w->scales;
  const bool dq_in = !residual && !scales && gemv_takes_dq(m, w, lora, exact);
  if (!residual && !scales && !dq_in) {
    const int rc = rebuild_scales(w, workspace, workspace_bytes, stream, &scales);
    if (rc != kOk) return rc;
  }
  LF_REQUIRE(!residual || (lora && !bias && !swiglu && !exact), "the residual form takes a LoRA batch and nothing else");
  const GemvPlan pl = gemv_plan(m, w->n, w->k, device_cus(), lora ? lora->num_slices * lora->max_rank : 1);
  LF_REQUIRE(w->n % pl.rows == 0, "output width must be a multiple of %d", pl.rows);
  GemvParams p{};
  p.x = x;
  p.x_stride = x_stride;
  p.m = int(m);
  p.q = w->qweight;
  p.scales = scales;
  p.code = w->code;
  p.n = int(w->n);
  p.k = int(w->k);
  p.bias = bias;
  p.y = y;
  p.y_stride = y_stride;
  p.row_groups = pl.row_groups;
  p.gated_half = swiglu ? int(w->n / 2) : 0;  // n % 32 == 0: R / 2 divides n / 2
  if (dq_in) fill_dq_params(p, w);
  if (lora) {
    const int rc = fill_lora_params(p, pl, lora, m, workspace, workspace_bytes, withhold);
    if (rc != kOk) return rc;
    // Tiles of at most 8 tokens run two workgroups per CU.
    p.resident = std::min(pl.grid, device_cus() * (m <= 8 ? 2 : 1));
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
