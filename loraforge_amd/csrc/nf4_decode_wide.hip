// Wide-batch NF4 decode linear with per-token multi-LoRA (more than 32 tokens,
// one launch for any batch whose 32-token tiles the chip can take in a few
// rounds).
//
// Reference chain (integrations/_sglang_nf4_linear.py:116-129, then the row
// operators ops/lora_rows.py:51-239):
//   y = bf16(x @ dequant(W)^T) (+ bias, rounded again),
//   z = bf16(A_g x), y = bf16(y + bf16(scale_g * B_g z)) per routed token.
//
// A workgroup owns 32 output rows and 32 tokens over the whole K. Its eight
// base waves split the NF4 blocks of K into contiguous ranges; each wave
//   - requests the block scales of its whole range and the packed weight bytes
//     of its first kDWG groups of four blocks (32 rows x 128 bytes: a full
//     cache line of every row) at once, as direct global -> LDS copies that
//     each read eight full lines, so the weight stream is in flight from the
//     start; a group's slot is refilled as soon as its fourth block is read,
//   - streams the 32 token rows of x block by block through a private
//     two-slot LDS ring (4 KiB per block: 32 tokens x 64 k),
//   - contracts each block on v_mfma_f32_32x32x16_bf16 (tokens as A, the
//     block's weights as B: lane l takes the 16 packed bytes of half l/32 of
//     row l%32, i.e. 32 consecutive k, so the four MFMA steps of a block stay
//     inside one NF4 block and one scale),
// and the eight 32x32 partial tiles are summed through LDS once at the end.
// In LDS both streams keep rows of 128 bytes whose 16-byte units are
// XOR-swizzled by the row (unit u of row r at u ^ (r & 7)), so the global
// reads stay whole lines and the fragment reads are conflict-free. Waits are
// per wave: vmcnt over its own copies (which complete in issue order); with a
// two-slot x ring and four-block weight groups the copies outstanding after
// the ones a block needs are 0, 4 or 8 (wait_count); no workgroup barrier runs
// in the loop.
//
// LoRA (kLora, a ninth wave): the shrink units, their tagged partials, the
// tile metadata and the z gather are those of the narrow decode kernel
// (decode_lora.h). A producing workgroup requests its first unit's A and x
// fragments before its weight copies; the base waves contract them (MFMA,
// eight steps each) as soon as they land and the LoRA wave publishes the
// unit, then builds the tile metadata and gathers z while the base waves
// stream. After the loop each base wave takes the tile's distinct slots
// wave, wave + 8, ... and computes z_g B_g^T on the same 32x32 MFMA (z as A,
// tokens of other slots masked; B_g^T as B, columns of other slices masked),
// so the delta tiles share the base tiles' layout and are summed with them.
//
// The epilogue gives each thread a gate column and the column 16 rows up of
// one token, so the SwiGLU output (gate rows lo .. lo + 15 and the matching
// up rows in the group) is formed at the store.
//
// Why this shape (read-pattern probes on MI355X, 64-token batch, 4096 x 4096,
// weights rotated over 64 copies, no arithmetic): whole weight shares in
// flight at once with x streamed beside them take 3.5 us above an empty
// launch, against about 8.8 us for the 32-row tile of the narrow decode
// kernel, whose per-wave rings carry W and x together and keep about 1 KiB of
// W per stage in flight. Splitting K instead (x resident, fp32 partials
// exchanged between workgroups) loads 0.6 us faster but the exchange costs
// 1-4 us. Weight copies of 16 bytes per lane from 32 rows (a quarter line per
// row and request) took 7.8 us for the weight stream alone.
//
// Block order: workgroup b runs on XCD b % 8 (checked on the device: the
// dispatcher deals workgroups round-robin over the XCDs), so the token tiles
// of one row group are placed at b, b + 8, ... and read its weight bytes
// from HBM once, through one L2.
#include "decode_lora.h"

namespace lf {
namespace {

constexpr int kBase = 8;     // base (contraction) waves
constexpr int kRows = 32;    // output rows per workgroup
constexpr int kTokens = 32;  // tokens per workgroup
constexpr int kDX = 2;       // x ring slots per wave
constexpr int kXSlot = kTokens * 128;  // one x block: 32 tokens x 64 bf16
constexpr int kWGroup = kRows * 128;   // one weight group: 32 rows x 4 blocks x 32 packed bytes
constexpr int kFirstSteps = 8;         // first-unit MFMA steps per base wave (8 x 8 covers a 2048-k slice)
constexpr int kSlotsPerWave = kTokens / kBase;  // expand: the tile's distinct slots, one batch per wave

// Tile shape for the shared LoRA helpers (z staged for 32 tokens).
struct WideTile {
  static constexpr int kXR = kTokens;
  static constexpr int kRT = 2;
  static constexpr int kR = kRows;
  static constexpr int kTT = 1;
  // Eight polled partials per lane and batch: sixteen need more registers
  // than a ninth wave leaves (three waves on one SIMD, 168 VGPRs each).
  static constexpr int kGatherEntries = 8;
};
using WL = LoraLds<WideTile>;

// Global row of local row r: a plain group's rows are contiguous; in
// SwiGLU-output mode rows 0..15 are gate rows from lo, 16..31 the up rows
// from hi.
__device__ __forceinline__ int wrow(int lo, int hi, int r) { return r < 16 ? lo + r : hi + (r - 16); }

// vmcnt(n) for a runtime n (used once per launch; anything above 31 waits
// for everything, which is always safe).
__device__ __forceinline__ void wait_vm_any(int n) {
  switch (n) {
#define LF_WAIT_CASE(c) \
  case c: wait_vm<c>(); break;
    LF_WAIT_CASE(1) LF_WAIT_CASE(2) LF_WAIT_CASE(3) LF_WAIT_CASE(4) LF_WAIT_CASE(5) LF_WAIT_CASE(6)
    LF_WAIT_CASE(7) LF_WAIT_CASE(8) LF_WAIT_CASE(9) LF_WAIT_CASE(10) LF_WAIT_CASE(11) LF_WAIT_CASE(12)
    LF_WAIT_CASE(13) LF_WAIT_CASE(14) LF_WAIT_CASE(15) LF_WAIT_CASE(16) LF_WAIT_CASE(17) LF_WAIT_CASE(18)
    LF_WAIT_CASE(19) LF_WAIT_CASE(20) LF_WAIT_CASE(21) LF_WAIT_CASE(22) LF_WAIT_CASE(23) LF_WAIT_CASE(24)
    LF_WAIT_CASE(25) LF_WAIT_CASE(26) LF_WAIT_CASE(27) LF_WAIT_CASE(28) LF_WAIT_CASE(29) LF_WAIT_CASE(30)
    LF_WAIT_CASE(31)
#undef LF_WAIT_CASE
    default: wait_vm<0>(); break;
  }
}

// The block scales of the group's 32 rows over blocks kb0 .. kb0 + nb - 1 into
// the wave's scale area: row j at j * sc_stride floats (sc_stride a power of
// two, at least 4 and at least nb), as dword copies of 64 consecutive floats.
// Padding positions read a valid scale of the range (never used). Returns the
// number of copies.
__device__ __forceinline__ int issue_scales(const GemvParams& p, char* area, int lo, int hi, int kb0, int nb,
                                            int lane) {
  const int nblk = p.k >> 6;
  const int shift = __builtin_ctz(p.sc_stride);
  const int copies = p.sc_bytes / 256;
  for (int i = 0; i < copies; ++i) {
    const int pos = i * 64 + lane;
    const int row = min(pos >> shift, kRows - 1);
    const int col = pos & (p.sc_stride - 1);
    copy4(p.scales + int64_t(wrow(lo, hi, row)) * nblk + kb0 + (col < nb ? col : 0), area + i * 256);
  }
  return copies;
}

template <int kC>
__device__ __forceinline__ uint4 codes_of(uint32_t d, const uint32_t* ptl) {
  uint4 r;
  r.x = ptl[(d & 0xffu) * kC];
  r.y = ptl[__builtin_amdgcn_ubfe(d, 8, 8) * kC];
  r.z = ptl[__builtin_amdgcn_ubfe(d, 16, 8) * kC];
  r.w = ptl[(d >> 24) * kC];
  return r;
}

// Copies of a base wave, in issue order: its scale copies, weight groups
// 0 .. kDWG - 1 (4 copies each), x blocks 0 and 1 (4 each); then in
// iteration i, once block i's fragments are read, the weight group
// i / 4 + kDWG when i is the fourth block of its group, and x block i + 2,
// each while in range. Copies complete in issue order, so block i may start
// once no more than wait_count(i) copies are outstanding: those issued after
// x block i (the weight group of iteration i - 1, x block i + 1), or, with a
// single weight slot, after weight group i / 4 when that was issued later
// (at iteration i - 1).
template <int kDWG>
__device__ __forceinline__ int wait_count(int i, int nb, int groups) {
  const bool w_prev = i >= 4 && (i & 3) == 0 && ((i - 1) >> 2) + kDWG < groups;  // weight refill at i - 1
  const int x_next = i + 1 < nb ? 4 : 0;
  if (kDWG == 1 && w_prev) return x_next;
  return (w_prev ? 4 : 0) + x_next;
}

// Expand B fragments of one wave: for each of its slots (wave + kBase * q),
// ranks 0..15 of this lane's B row (row wrow(lane % 32), ranks 8 (lane / 32)
// .. + 8), raw 16 bytes (shifted and masked by expand_fix).
struct WideB {
  uint4 bf[kSlotsPerWave];
};

__device__ __forceinline__ void expand_request(const GemvParams& p, const TileMeta* tm, WideB& b, int lo, int hi,
                                               int wave, int lane) {
  const int nd = tm->nd;
  const int row = wrow(lo, hi, lane & 31);
  const int j0 = 8 * (lane >> 5);
#pragma unroll
  for (int q = 0; q < kSlotsPerWave; ++q) {
    const int d = wave + kBase * q;
    const bool live = d < nd;
    const int dd = live ? d : 0;
    b.bf[q] = *reinterpret_cast<const uint4*>(b8_at(p, tm->dboff[dd], tm->dstride[dd], tm->dr[dd], row, j0, live).src);
  }
}

__device__ __forceinline__ void expand_fix(const TileMeta* tm, WideB& b, int lo, int hi, int wave, int lane) {
  const int nd = tm->nd;
  const int row = wrow(lo, hi, lane & 31);
  const int j0 = 8 * (lane >> 5);
#pragma unroll
  for (int q = 0; q < kSlotsPerWave; ++q) {
    const int d = wave + kBase * q;
    if (d >= nd) break;  // uniform
    const int st = tm->dstride[d];
    const int cnt = min(8, tm->dr[d] - j0);
    if (st >= 8) b.bf[q] = keep_first(b.bf[q], cnt);
    else b.bf[q] = b8_fix(b.bf[q], B8{nullptr, int((tm->dboff[d] + int64_t(row) * st + j0) & 7), cnt});
  }
}

// delta[token][row] = sum over this wave's slots g of z_g[token] . B_g[row] for
// the tokens routed to g and the rows of the slice the z values belong to.
__device__ __forceinline__ f32x16 expand_wide(const GemvParams& p, const char* lds, const WideB& b,
                                              const int (&bounds)[4], int lo, int hi, int wave, int lane) {
  const TileMeta* tm = reinterpret_cast<const TileMeta*>(lds + WL::kMeta);
  const uint16_t* zl = reinterpret_cast<const uint16_t*>(lds + WL::kZ);
  f32x16 dacc;
#pragma unroll
  for (int e = 0; e < 16; ++e) dacc[e] = 0.f;
  const int nd = tm->nd;
  const int i = lane & 31;  // token (A row) and local row (B column) of this lane
  const int g8 = 8 * (lane >> 5);
  const int row = wrow(lo, hi, i);
  auto slice_of = [&](int r) { return int(p.slices > 1 && r >= bounds[1]) + int(p.slices > 2 && r >= bounds[2]); };
  const int cs = slice_of(row);
  const int s_lo = slice_of(lo);
  const int s_hi = slice_of(hi + 15);
  const int gi = tm->g[i];
#pragma unroll
  for (int q = 0; q < kSlotsPerWave; ++q) {
    const int d = wave + kBase * q;
    if (d >= nd) break;  // uniform
    const int g = tm->dslot[d];
    const int rk = tm->dr[d];
    for (int s = s_lo; s <= s_hi; ++s) {
      for (int h = 0; h < 4; ++h) {
        if (16 * h >= rk) break;  // uniform
        const uint4 zv = *reinterpret_cast<const uint4*>(zl + (i * 3 + s) * 64 + 16 * h + g8);
        const uint4 zf = gi == g ? zv : make_uint4(0, 0, 0, 0);
        uint4 bv = b.bf[q];
        if (h > 0) {
          const B8 b8 = b8_at(p, tm->dboff[d], tm->dstride[d], rk, row, 16 * h + g8, true);
          bv = b8_fix(*reinterpret_cast<const uint4*>(b8.src), b8);
        }
        const uint4 bb = cs == s ? bv : make_uint4(0, 0, 0, 0);
        dacc = mfma32(as_bf16x8(zf), as_bf16x8(bb), dacc);
      }
    }
  }
  return dacc;
}

// The LoRA wave of a wide workgroup: publishes the workgroup's first shrink
// unit as soon as the base waves have counted in, builds the tile metadata,
// produces the other units (small grids only), gathers z, and takes its part
// in the workgroup's two remaining barriers (z ready; partial tiles in LDS)
// before it counts the workgroup out of the call.
__device__ __forceinline__ void lora_wave(const GemvParams& p, char* lora_lds, float* red, int* prod_done, int g_tile,
                                       uint32_t epoch, int t0, int mt, int lane) {
  const TokenMeta tmeta = token_meta(p, g_tile, mt, lane);
  Unit un0{};
  const bool has0 = int(blockIdx.x) < p.producers && int(blockIdx.x) < p.units && unit_of(p, blockIdx.x, un0);
  const uint32_t tag = __builtin_amdgcn_readfirstlane(epoch) + 1u;
  if (has0) publish_first_unit<kBase>(p, red, prod_done, un0, tag, lane);
  lora_meta<WideTile>(lora_lds, tmeta, p.slices, lane);
  produce_other_units<kFirstSteps>(p, tag, lane);
  lora_gather<WideTile>(p, lora_lds, t0, mt, tag, lane);
  const uint32_t departed = depart_issue(p.ce, lane);  // after the last partial load
  lds_barrier();  // z and the tile metadata are in LDS
  lds_barrier();  // the partial tiles are in LDS
  depart_finish(p.ce, departed, __builtin_amdgcn_readfirstlane(epoch), lane);
}

// kDWG: weight group slots per wave (2, or 1 when a long K needs the LDS).
// kLora: a ninth wave and the LoRA stages (row groups must fill whole XCD
// octets, so every workgroup of the grid is a real one and counts in once).
template <bool kExact, int kDWG, bool kLora>
__global__ __launch_bounds__(64 * (kBase + (kLora ? 1 : 0)), 1) void nf4_decode_wide_kernel(GemvParams p) {
  constexpr int kCP = kLora ? 8 : 16;  // pair-table copies (lane l reads copy l % kCP); 8 leave LDS for LoRA
  __shared__ __attribute__((aligned(16))) char wring[kBase * kDWG * kWGroup];
  __shared__ __attribute__((aligned(16))) char xring[kBase * kDX * kXSlot];
  __shared__ float table[16];
  __shared__ __attribute__((aligned(16))) uint32_t pt[kExact ? 4 : 256 * kCP];
  __shared__ __attribute__((aligned(16))) char lora_lds[kLora ? WL::kBytes : 16];
  __shared__ int prod_done;  // base waves that have written their first-unit partials
  extern __shared__ __attribute__((aligned(16))) char scale_lds[];  // kBase * p.sc_bytes (+16)

  const int xcc = blockIdx.x & 7;
  const int jb = blockIdx.x >> 3;
  const int tile = jb % p.tiles;
  const int rg = (jb / p.tiles) * 8 + xcc;
  if (!kLora && rg >= p.row_groups) return;  // the grid rounds the row groups up to whole XCD octets
  const int lo = p.gated_half ? rg * (kRows / 2) : rg * kRows;
  const int hi = p.gated_half ? p.gated_half + lo : lo + kRows / 2;
  const int t0 = tile * kTokens;
  const int mt = min(kTokens, p.m - t0);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const bool base = wave < kBase;
  const int nblk = p.k >> 6;
  const int kb0 = base ? nblk * wave / kBase : 0;
  const int nb = base ? nblk * (wave + 1) / kBase - kb0 : 0;
  const int groups = (nb + 3) >> 2;
  char* myw = wring + (base ? wave : 0) * kDWG * kWGroup;
  char* myx = xring + (base ? wave : 0) * kDX * kXSlot;
  char* mysc = scale_lds + (base ? wave : 0) * p.sc_bytes;
  float* red = reinterpret_cast<float*>(lora_lds + WL::kZ);  // first-unit partials (before z is gathered there)

  // Copy addresses: a uniform base (scalar registers) plus a 32-bit per-lane
  // byte offset, so the copies take the scalar-base form and no 64-bit
  // pointers are held per lane.
  // x copy c: token row 8c + lane / 8, unit position lane % 8 holds unit
  // (lane % 8) ^ (row & 7) of the token's 64 bf16 of the block. Tokens past
  // the batch read the last token (their outputs are not stored).
  const char* xbase_g = reinterpret_cast<const char*>(p.x) + int64_t(kb0) * 128;
  uint32_t xo[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int i = 8 * c + (lane >> 3);
    const int tok = t0 + (i < mt ? i : mt - 1);
    xo[c] = uint32_t(tok) * uint32_t(p.x_stride) * 2u + uint32_t(((lane & 7) ^ (i & 7)) * 16);
  }
  // Weight copy c of a group: row 8c + lane / 8 (row & 7 = (lane / 8) & 7),
  // unit position lane % 8 holds 16-byte unit (lane % 8) ^ (row & 7) of the
  // row's 128 bytes of the group. The block of the group this lane's unit
  // belongs to is the same for every copy; in a wave's last group, units of
  // blocks past its range (nb not a multiple of 4) read the group's first
  // block instead, so no copy leaves the wave's blocks (or the weight, in the
  // last row); those positions are never read.
  const int row_bytes = p.k >> 1;
  const int wblk = ((lane & 7) ^ ((lane >> 3) & 7)) >> 1;
  const uint32_t wo = uint32_t((lane >> 3) * row_bytes + ((lane & 7) ^ ((lane >> 3) & 7)) * 16);
  const char* wrow_g[4];  // uniform: row 8c of the group, at the wave's first block
#pragma unroll
  for (int c = 0; c < 4; ++c)
    wrow_g[c] = reinterpret_cast<const char*>(p.q) + int64_t(wrow(lo, hi, 8 * c)) * row_bytes + int64_t(kb0) * 32;
  auto issue_w = [&](int grp, int slot) {
    const uint32_t off = wo - (4 * grp + wblk < nb ? 0u : uint32_t(wblk * 32));
#pragma unroll
    for (int c = 0; c < 4; ++c) copy16(wrow_g[c] + grp * 128 + off, myw + slot * kWGroup + c * 1024);
  };
  auto issue_x = [&](int blk, int slot) {
#pragma unroll
    for (int c = 0; c < 4; ++c) copy16(xbase_g + blk * 128 + xo[c], myx + slot * kXSlot + c * 1024);
  };

  // Codebook (and the LoRA slice bounds) through scalar loads: no vector
  // load waits behind the copies.
  float cb[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) cb[i] = sload(p.code, i);
  int bounds[4] = {0, 0, 0, 0};
  if constexpr (kLora) {
#pragma unroll
    for (int q = 0; q < 4; ++q) bounds[q] = q <= p.slices ? sload(p.slice_offsets, q) : 0;
  }

  // A producing workgroup's first shrink unit: its fragments are requested
  // ahead of the weight copies (untracked loads), so they are not queued
  // behind the weight stream; the base waves contract them once they land.
  Unit un0{};
  bool has0 = false;
  FirstFragsN<kFirstSteps> pre;
  uint32_t epoch = 0;
  int g_tile = -1;
  int after_unit = 0;  // copies issued after the unit's fragments
  if (base) {
    if constexpr (kLora) {
      has0 = int(blockIdx.x) < p.producers && int(blockIdx.x) < p.units && unit_of(p, blockIdx.x, un0);
      if (has0) first_frags<kFirstSteps, kBase>(p, un0, wave, lane, pre);
    }
    if (nb > 0) {
      after_unit += issue_scales(p, mysc, lo, hi, kb0, nb, lane);
#pragma unroll
      for (int g2 = 0; g2 < kDWG; ++g2)
        if (g2 < groups) {
          issue_w(g2, g2);
          after_unit += 4;
        }
#pragma unroll
      for (int s = 0; s < kDX; ++s)
        if (s < nb) {
          issue_x(s, s);
          after_unit += 4;
        }
    }
  } else if constexpr (kLora) {
    // The LoRA wave: the call epoch and the tile's token slots (vector loads;
    // the barriers below wait for scalar loads and LDS only).
    epoch = __hip_atomic_load(p.ce.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    g_tile = p.token_slots[t0 + min(lane, mt - 1)];
  }

  if (threadIdx.x == 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) table[i] = cb[i];
    if constexpr (kLora) {
      reinterpret_cast<TileMeta*>(lora_lds + WL::kMeta)->ready = 0;
      prod_done = 0;
    }
  }
  if constexpr (!kExact) {
    lds_barrier();
    if (threadIdx.x < 256) {
      const uint32_t v = pack_bf16x2(table[threadIdx.x >> 4], table[threadIdx.x & 15]);
      uint4* dst = reinterpret_cast<uint4*>(pt + threadIdx.x * kCP);
#pragma unroll
      for (int c = 0; c < kCP / 4; ++c) dst[c] = make_uint4(v, v, v, v);
    }
  }
  lds_barrier();
  const uint32_t* ptl = pt + (lane % kCP);

  // The base waves; the LoRA wave's code follows theirs (so nothing of the
  // streaming state is live across it).
  if (base) {
  if constexpr (kLora) {
    if (has0) {
      wait_vm_any(after_unit);  // the unit's fragments have landed (loads complete in order)
      first_unit_partials<kFirstSteps, kBase>(p, un0, pre, red, &prod_done, wave, lane);
    }
  }

  f32x16 acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
  const int rr = lane & 31;  // A row (token) and B column (weight row) of this lane
  const int g = lane >> 5;   // k half of the block (A and B)
  // Fragment offsets inside a slot: x units 4g + u of token rr; weight unit
  // 2 * (block % 4) + g of row rr.
  uint32_t xoff[4], woff[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    xoff[u] = uint32_t(rr * 128 + (((4 * g + u) ^ (rr & 7)) << 4));
    woff[u] = uint32_t(rr * 128 + (((2 * u + g) ^ (rr & 7)) << 4));
  }
  const uint32_t xbase = lds_addr(myx);
  const uint32_t wbase = lds_addr(myw);
  const uint32_t scb = lds_addr(mysc) + uint32_t(rr * p.sc_stride) * 4;
  // The loop runs eight blocks per pass (two weight groups), so every slot
  // index is a compile-time constant.
  for (int i0 = 0; i0 < nb; i0 += 8) {
    f32x4 sc4 = {0.f, 0.f, 0.f, 0.f};  // the scales of this lane's row for the current four blocks
#pragma unroll
    for (int bl = 0; bl < 8; ++bl) {
      const int i = i0 + bl;
      if (i >= nb) break;
      const int wc = wait_count<kDWG>(i, nb, groups);
      if (wc == 8) wait_vm<8>();
      else if (wc == 4) wait_vm<4>();
      else wait_vm<0>();
      const uint32_t xs = xbase + (bl % kDX) * kXSlot;
      u32x4 xf[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) xf[u] = lds_read128(xs + xoff[u]);
      u32x4 wq = lds_read128(wbase + ((bl >> 2) % kDWG) * kWGroup + woff[bl & 3]);
      if ((bl & 3) == 0) sc4 = __builtin_bit_cast(f32x4, lds_read128(scb + i * 4));
      lds_wait();
      tie(wq);
      tie(sc4);
#pragma unroll
      for (int u = 0; u < 4; ++u) tie(xf[u]);
      const float sc = sc4[bl & 3];
      // Refill what was just read: the weight group after its fourth block,
      // then the x slot.
      if ((bl & 3) == 3 && (i >> 2) + kDWG < groups) issue_w((i >> 2) + kDWG, ((i >> 2) + kDWG) % kDWG);
      if (i + kDX < nb) issue_x(i + kDX, bl % kDX);
      const uint32_t qd[4] = {wq.x, wq.y, wq.z, wq.w};
      uint4 wb[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) wb[u] = kExact ? decode_dword(qd[u], sc, table) : codes_of<kCP>(qd[u], ptl);
      if constexpr (kExact) {
#pragma unroll
        for (int u = 0; u < 4; ++u) acc = mfma32(vec_bf16x8(xf[u]), as_bf16x8(wb[u]), acc);
      } else {
        f32x16 d;
#pragma unroll
        for (int e = 0; e < 16; ++e) d[e] = 0.f;
#pragma unroll
        for (int u = 0; u < 4; ++u) d = mfma32(vec_bf16x8(xf[u]), as_bf16x8(wb[u]), d);
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[e] = __builtin_fmaf(sc, d[e], acc[e]);
      }
    }
  }
  wait_vm<0>();

  // With LoRA: the base waves request the B fragments of their slots once the
  // tile metadata is ready, the LoRA wave has gathered z, and after the
  // barrier (LDS only) each base wave computes its delta tile.
  f32x16 dacc;
#pragma unroll
  for (int e = 0; e < 16; ++e) dacc[e] = 0.f;
  if constexpr (kLora) {
    const TileMeta* tm = reinterpret_cast<const TileMeta*>(lora_lds + WL::kMeta);
    WideB eb;
    while (*(const volatile __attribute__((address_space(3))) int*)(&tm->ready) == 0) __builtin_amdgcn_s_sleep(1);
    expand_request(p, tm, eb, lo, hi, wave, lane);
    expand_fix(tm, eb, lo, hi, wave, lane);
    lds_barrier();  // z and the tile metadata are in LDS
    dacc = expand_wide(p, lora_lds, eb, bounds, lo, hi, wave, lane);
  }

  // Sum the partial tiles: base wave w writes its accumulators (and delta
  // tile) into its own x ring (all of its copies have landed and been read),
  // element r of lane l at r * 64 + l (the delta 1024 floats further).
  {
    float* mine = reinterpret_cast<float*>(myx);
#pragma unroll
    for (int e = 0; e < 16; ++e) mine[e * 64 + lane] = acc[e];
    if constexpr (kLora) {
#pragma unroll
      for (int e = 0; e < 16; ++e) mine[1024 + e * 64 + lane] = dacc[e];
    }
  }
  lds_barrier();
  {
    // Thread t: token t / 16 and the columns t % 16 (a gate row in SwiGLU
    // mode) and t % 16 + 16 (its up row). Output (token, column) of the 32x32
    // tile is element 4 (token / 8) + token % 4 of lane column + 32 ((token / 4) % 2).
    const int tok = threadIdx.x >> 4;
    const int jj = threadIdx.x & 15;
    const TileMeta* tm = reinterpret_cast<const TileMeta*>(lora_lds + WL::kMeta);
    const bool routed = kLora && tok < mt && tm->g[tok] >= 0;
    const float lscale = kLora && routed ? tm->scale[tok] : 0.f;
    float out[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int col = jj + 16 * h;
      const int o = (4 * (tok >> 3) + (tok & 3)) * 64 + col + 32 * ((tok >> 2) & 1);
      float sum = 0.f, dsum = 0.f;
#pragma unroll
      for (int w = 0; w < kBase; ++w) {
        const float* part = reinterpret_cast<const float*>(xring + w * kDX * kXSlot);
        sum += part[o];
        if constexpr (kLora) dsum += part[1024 + o];
      }
      const int row = wrow(lo, hi, col);
      float v = round_bf16(sum);
      if (p.bias) v = round_bf16(v + bf16_to_f32(p.bias[row]));
      if (routed) v += round_bf16(dsum * lscale);
      out[h] = round_bf16(v);
      if (!p.gated_half && tok < mt) p.y[int64_t(t0 + tok) * p.y_stride + row] = uint16_t(f32_to_bf16(v));
    }
    // SwiGLU output h = bf16(bf16(silu(gate)) * up) for feature lo + jj (the
    // reference's activation after both LoRA adds, benchmarks/qwen35_decode_silu.py:60-61).
    if (p.gated_half && tok < mt)
      p.y[int64_t(t0 + tok) * p.y_stride + lo + jj] = uint16_t(f32_to_bf16(silu_times(out[0], out[1])));
  }
  } else {
    if constexpr (kLora) lora_wave(p, lora_lds, red, &prod_done, g_tile, epoch, t0, mt, lane);
  }
}

constexpr int64_t kLdsBytes = 160 * 1024;

template <class K>
int64_t static_lds_of(K fn, int64_t& cache) {
  if (cache < 0) {
    hipFuncAttributes at{};
    if (hipFuncGetAttributes(&at, reinterpret_cast<const void*>(fn)) != hipSuccess) return -1;
    cache = int64_t(at.sharedSizeBytes);
  }
  return cache;
}

// Launches the variant whose static LDS and the waves' scale areas fit one
// workgroup; returns false when it does not fit.
template <bool kExact, int kDWG, bool kLora>
bool try_launch(dim3 grid, hipStream_t s, const GemvParams& p, int64_t dyn) {
  static int64_t static_lds = -1;
  auto fn = nf4_decode_wide_kernel<kExact, kDWG, kLora>;
  const int64_t st = static_lds_of(fn, static_lds);
  if (st < 0 || st + dyn > kLdsBytes) return false;
  hipLaunchKernelGGL(fn, grid, dim3(64 * (kBase + (kLora ? 1 : 0))), size_t(dyn), s, p);
  return true;
}

template <bool kExact, bool kLora>
bool launch_variant(dim3 grid, hipStream_t s, const GemvParams& p, int64_t dyn) {
  return try_launch<kExact, 2, kLora>(grid, s, p, dyn) || try_launch<kExact, 1, kLora>(grid, s, p, dyn);
}

// Floats per row of a wave's scale area: the wave's blocks rounded up to a
// power of two, at least 4 (scales are read four blocks at a time).
int64_t scale_stride(int64_t nblk) {
  const int64_t nbw = (nblk + kBase - 1) / kBase;
  int64_t s = 4;
  while (s < nbw) s *= 2;
  return s;
}

int64_t scale_area_bytes(int64_t nblk) { return (kRows * scale_stride(nblk) * 4 + 255) / 256 * 256; }

}  // namespace

int device_cus();

// Whether the wide decode kernel takes this call: more than 32 tokens, a K
// whose rings and scale areas fit LDS (the smallest variant), and with LoRA
// row groups that fill whole XCD octets (N a multiple of 256), shrink
// partials that fit the workspace header and at most 1024 units.
bool decode_wide_fits(int64_t m, int64_t n, int64_t k, const lf_lora* lora) {
  if (m <= 32 || n % kRows) return false;
  const int64_t nblk = k / 64;
  const int64_t area = scale_area_bytes(nblk);
  // Static LDS of the smallest variant: one weight group and two x blocks per
  // base wave, the pair table and (with LoRA) the z area.
  const int64_t smallest = int64_t(kBase) * (kWGroup + kDX * kXSlot) + 256 * 16 * 4 + 64 + (lora ? WL::kBytes : 0);
  if (smallest + kBase * area + 16 > kLdsBytes) return false;
  if (!lora) return true;
  if (n % (8 * kRows)) return false;
  const GemvPlan pl = gemv_plan(m, n, k, device_cus(), lora->num_slices * lora->max_rank);
  return pl.units <= 1024 && kPartialsOffset + m * pl.kz * lora->num_slices * lora->max_rank * 8 <= kWorkspaceHeader;
}

int launch_decode_wide(const uint16_t* x, int64_t m, int64_t x_stride, const lf_nf4_weight* w, const uint16_t* bias,
                       const lf_lora* lora, uint16_t* y, int64_t y_stride, void* workspace, int64_t workspace_bytes,
                       bool exact, bool swiglu, bool withhold, void* stream) {
  LF_REQUIRE(decode_wide_fits(m, w->n, w->k, lora) && w->scales != nullptr, "wide decode: call outside its range");
  LF_REQUIRE(!swiglu || w->n % 64 == 0, "SwiGLU output needs N a multiple of 64");
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
  p.row_groups = int(w->n / kRows);
  p.tiles = int((m + kTokens - 1) / kTokens);
  p.gated_half = swiglu ? int(w->n / 2) : 0;
  const int64_t nblk = w->k / 64;
  p.sc_stride = int(scale_stride(nblk));
  p.sc_bytes = int(scale_area_bytes(nblk));
  if (lora) {
    const GemvPlan pl = gemv_plan(m, w->n, w->k, device_cus(), lora->num_slices * lora->max_rank);
    const int rc = fill_lora_params(p, pl, lora, m, workspace, workspace_bytes, withhold);
    if (rc != kOk) return rc;
  }
  const int64_t dyn = int64_t(kBase) * p.sc_bytes + 16;
  const int64_t octets = (p.row_groups + 7) / 8;
  const int64_t grid = octets * 8 * p.tiles;
  LF_REQUIRE(grid < (int64_t(1) << 31), "wide decode: grid too large");
  auto s = static_cast<hipStream_t>(stream);
  const dim3 g3(static_cast<unsigned>(grid));
  bool ok;
  if (lora) ok = exact ? launch_variant<true, true>(g3, s, p, dyn) : launch_variant<false, true>(g3, s, p, dyn);
  else ok = exact ? launch_variant<true, false>(g3, s, p, dyn) : launch_variant<false, false>(g3, s, p, dyn);
  LF_REQUIRE(ok, "wide decode: the rings and scale areas do not fit LDS at K = %lld", (long long)w->k);
  LF_HIP(hipGetLastError());
  return kOk;
}

}  // namespace lf
