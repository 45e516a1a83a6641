// Wide-batch NF4 decode linear with per-token multi-LoRA (more than 8 tokens,
// more than 2 at N >= 8192, more than 16 at K > 8192; one launch for any batch whose 32-token tiles the chip can take in a few
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
//     of its first group of four blocks (32 rows x 128 bytes: a full cache
//     line of every row) at once, as direct global -> LDS copies that each
//     read eight full lines; the group's slot is refilled as soon as its
//     fourth block is read (the launcher takes one slot, kDWG = 1),
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
// The loop block after which a producing wave contracts the first unit
// (GemvParams::contract_after). The unit's pieces are requested behind the
// wave's first copies and, with the whole chip's first burst of copies ahead
// of them, land about 2 us after its first block: in a grid of one dispatch
// round, contracted after block 1 they held a producing wave's loop there.
// Measured on MI355X (north star B = 64, us per call, two rounds of
// alternating builds): after block 1 / 3 / 5 / 6 / 7 15.8 / 15.6 / 15.0 /
// 15.4 / 15.6 (exact weights 16.6 / 16.3 / 16.0 / 16.5 / 16.9). In grids of
// several rounds (c3's gate/up at B = 64) block 1 stays ahead (about 1 us
// per call), as the later rounds wait for nothing.
// One weight slot per wave (us per call, north star): a full round (B = 64,
// 256 workgroups) after block 3 / 4 / 5 / 6 14.5 / 14.3 / 14.1 / 14.4; a
// partial round (B = 32, 128 workgroups) 13.8 / 13.9 / 14.2 / 14.4.
constexpr int kContractAfterOneRound = 5;
constexpr int kContractAfterPartialRound = 3;
constexpr int kContractAfterRounds = 1;

// Tile shape for the shared LoRA helpers (z staged for 32 tokens).
struct WideTile {
  static constexpr int kXR = kTokens;
  static constexpr int kRT = 2;
  static constexpr int kR = kRows;
  static constexpr int kTT = 1;
  // Sixteen polled partials per lane and batch: a tile's partials in one
  // batch (the plan keeps 32 x zw x kz to 1024 where it can).
  static constexpr int kGatherEntries = 8;
  // z rows 400 bytes apart: the 32 token rows of an MFMA operand read start
  // on 16 different 4-bank groups (384 bytes apart, only two).
  static constexpr int kZRow = 200;
};
using WL = LoraLds<WideTile>;

// The launch parameters through a pointer the compiler cannot see through:
// fields read after this are loaded (scalar loads from the kernarg segment)
// where they are used, instead of being held in scalar registers from the
// kernel's start across the weight loop.
// (The kernels' only argument is the GemvParams, at offset 0 of the kernarg
// segment.)
__device__ __forceinline__ const GemvParams& reload() {
  auto q = (const __attribute__((address_space(4))) GemvParams*)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(q));
  return *(const GemvParams*)q;
}

// Global row of local row r: a plain group's rows are contiguous; in
// SwiGLU-output mode rows 0..15 are gate rows from lo, 16..31 the up rows
// from hi.
__device__ __forceinline__ int wrow(int lo, int hi, int r) { return r < 16 ? lo + r : hi + (r - 16); }

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

// The tile's distinct slots that this wave expands (wave + kBase q, q <
// kSlotsPerWave), in scalar registers: each lane reads one entry of the list
// (one batch of LDS reads and one wait), and the wave's entries are taken by
// lane reads, so the loops over slots, slices and rank groups branch on
// scalars. Entries at or past nd are not used.
struct WaveSlots {
  int nd;
  int g[kSlotsPerWave];
  int r[kSlotsPerWave];
  int stride[kSlotsPerWave];
  int64_t boff[kSlotsPerWave];
};

__device__ __forceinline__ WaveSlots wave_slots(const TileMeta* tm, int wave, int lane) {
  const int l = lane & 31;
  const int vg = tm->dslot[l];
  const int vr = tm->dr[l];
  const int vst = tm->dstride[l];
  const uint64_t vb = uint64_t(tm->dboff[l]);
  const int vnd = tm->nd;
  WaveSlots w;
  w.nd = __builtin_amdgcn_readfirstlane(vnd);
#pragma unroll
  for (int q = 0; q < kSlotsPerWave; ++q) {
    const int d = wave + kBase * q;
    w.g[q] = __builtin_amdgcn_readlane(vg, d);
    w.r[q] = __builtin_amdgcn_readlane(vr, d);
    w.stride[q] = __builtin_amdgcn_readlane(vst, d);
    w.boff[q] = int64_t((uint64_t(uint32_t(__builtin_amdgcn_readlane(int(uint32_t(vb >> 32)), d))) << 32) |
                        uint32_t(__builtin_amdgcn_readlane(int(uint32_t(vb)), d)));
  }
  return w;
}

__device__ __forceinline__ void expand_request(const GemvParams& p, const WaveSlots& ws, WideB& b, int lo, int hi,
                                               int wave, int lane) {
  const int row = wrow(lo, hi, lane & 31);
  const int j0 = 8 * (lane >> 5);
#pragma unroll
  for (int q = 0; q < kSlotsPerWave; ++q) {
    const bool live = wave + kBase * q < ws.nd;
    const int qq = live ? q : 0;
    b.bf[q] = *reinterpret_cast<const uint4*>(b8_at(p, ws.boff[qq], ws.stride[qq], ws.r[qq], row, j0, live).src);
  }
}

__device__ __forceinline__ void expand_fix(const WaveSlots& ws, WideB& b, int lo, int hi, int wave, int lane) {
  const int row = wrow(lo, hi, lane & 31);
  const int j0 = 8 * (lane >> 5);
#pragma unroll
  for (int q = 0; q < kSlotsPerWave; ++q) {
    if (wave + kBase * q >= ws.nd) break;
    const int cnt = min(8, ws.r[q] - j0);
    if (ws.stride[q] >= 8) b.bf[q] = keep_first(b.bf[q], cnt);
    else b.bf[q] = b8_fix(b.bf[q], B8{nullptr, int((ws.boff[q] + int64_t(row) * ws.stride[q] + j0) & 7), cnt});
  }
}

// delta[token][row] = sum over this wave's slots g of z_g[token] . B_g[row] for
// the tokens routed to g and the rows of the slice the z values belong to.
__device__ __forceinline__ f32x16 expand_wide(const GemvParams& p, const char* lds, const WaveSlots& ws,
                                              const WideB& b, int lo, int hi, int wave, int lane) {
  const TileMeta* tm = reinterpret_cast<const TileMeta*>(lds + WL::kMeta);
  const int bounds[3] = {0, __builtin_amdgcn_readfirstlane(tm->bounds[1]), __builtin_amdgcn_readfirstlane(tm->bounds[2])};
  const uint16_t* zl = reinterpret_cast<const uint16_t*>(lds + WL::kZ);
  f32x16 dacc;
#pragma unroll
  for (int e = 0; e < 16; ++e) dacc[e] = 0.f;
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
    if (wave + kBase * q >= ws.nd) break;
    for (int s = s_lo; s <= s_hi; ++s) {
      for (int h = 0; 16 * h < ws.r[q]; ++h) {
        const uint4 zv = *reinterpret_cast<const uint4*>(zl + i * WL::kZRow + s * 64 + 16 * h + g8);
        const uint4 zf = gi == ws.g[q] ? zv : make_uint4(0, 0, 0, 0);
        uint4 bv = b.bf[q];
        if (h > 0) {
          const B8 b8 = b8_at(p, ws.boff[q], ws.stride[q], ws.r[q], row, 16 * h + g8, true);
          bv = b8_fix(*reinterpret_cast<const uint4*>(b8.src), b8);
        }
        const uint4 bb = cs == s ? bv : make_uint4(0, 0, 0, 0);
        dacc = mfma32(as_bf16x8(zf), as_bf16x8(bb), dacc);
      }
    }
  }
  return dacc;
}

// A producing workgroup's first shrink unit, contracted on the VALU by the
// base waves. The unit is cut into pieces of one A row x 512 k (1 KiB, one
// load in which each 16-lane quarter reads 256 contiguous bytes). A pass
// covers rp rows from j0 over c k-chunks (c = 1, 2, 4 or 8, the slice's
// chunks rounded up to a power of two, at most 8; rp * c = 8 pw): wave w
// takes chunk c ub + w % c of rows j0 + (w / c) pw .. + pw (pw <= R), with
// the matching 1 KiB of x[t]. Lane l owns k = 512 chunk + 8 l; lanes past
// the slice read x as zero (their A loads stay inside the row). The first
// pass is requested before the x copies; further passes (more rows, slices
// longer than 8 chunks) run after it.
constexpr int kPieceK = 512;
// Rows per wave and pass (pw): R = 4 for a unit contracted inside the weight
// loop (fewer registers held across it), 8 otherwise.
template <int R>
struct UnitPieces {
  u32x4 x;    // as loaded (lanes past the slice read k = 0; masked when used)
  bool live;  // this lane's k is inside the slice
  u32x4 a[R];
};

struct PassShape {
  int c;   // k-chunks per pass
  int rp;  // rows per pass
  int pw;  // rows per wave
};

template <int R>
__device__ __forceinline__ PassShape pass_shape(const Unit& un, int j0) {
  const int chunks = (un.steps * 32 + kPieceK - 1) / kPieceK;
  PassShape ps;
  ps.c = chunks >= 8 ? 8 : chunks >= 4 ? (chunks == 4 ? 4 : 8) : chunks >= 2 ? (chunks == 2 ? 2 : 4) : 1;
  const int step = 8 / ps.c;  // rp is a multiple of 8 / c
  const int rest = (un.rows - j0 + step - 1) / step * step;
  ps.rp = min(rest, R * 8 / ps.c);
  ps.pw = ps.rp * ps.c / 8;
  return ps;
}

// Ordinary (tracked) loads: the compiler waits for them before their first
// use. Loads the compiler does not track must not be used here: the row
// count is a runtime value, and a branch around such a load lets the
// compiler copy its destination register before the data has arrived.
template <int R>
__device__ __forceinline__ void unit_pieces(const GemvParams& p, const Unit& un, int j0, int ub, const PassShape& ps,
                                            int wave, int lane, UnitPieces<R>& f) {
  const int len = un.steps * 32;
  const int kofs = (ps.c * ub + wave % ps.c) * kPieceK + 8 * lane;
  const bool live = kofs < len;
  const uint32_t voff = uint32_t(live ? kofs : 0) * 2u;
  // (No arithmetic on the loaded values here: it would make the compiler
  // wait for them before the copies that follow.)
  f.x = global_load128(uniform_ptr(p.x + int64_t(un.t) * p.x_stride + un.kb), voff);
  f.live = live;
  const int r0 = j0 + (wave / ps.c) * ps.pw;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    f.a[i] = u32x4{0u, 0u, 0u, 0u};
    if (i < ps.pw) {  // uniform
      const int row = min(r0 + i, un.rows - 1);
      f.a[i] = global_load128(uniform_ptr(p.a_store + un.aoff + int64_t(row) * p.k + un.kb), voff);
    }
  }
}

// v[i] += sum over this lane's 8 k of x * A[row i] (fp32, in k order), i < pw.
template <int R>
__device__ __forceinline__ void unit_dots(const UnitPieces<R>& f, int pw, float (&v)[8]) {
  const u32x4 x = f.live ? f.x : u32x4{0u, 0u, 0u, 0u};
  const uint32_t xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int i = 0; i < R; ++i) {
    if (i >= pw) continue;  // uniform
    const uint32_t as[4] = {f.a[i].x, f.a[i].y, f.a[i].z, f.a[i].w};
    float acc = v[i];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc = __builtin_fmaf(bf16_lo(xs[e]), bf16_lo(as[e]), acc);
      acc = __builtin_fmaf(bf16_hi(xs[e]), bf16_hi(as[e]), acc);
    }
    v[i] = acc;
  }
}

// Sums v[0..7] over the wave's 64 lanes in 10 exchanges (each step halves
// the values a lane keeps); lane l with l % 8 == 0 returns the sum of row
// 4 (l / 32 % 2) + 2 (l / 16 % 2) + (l / 8 % 2).
__device__ __forceinline__ float unit_reduce(float (&v)[8], int lane) {
  const bool b5 = lane & 32, b4 = lane & 16, b3 = lane & 8;
  float h4[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float keep = b5 ? v[i + 4] : v[i];
    const float give = b5 ? v[i] : v[i + 4];
    h4[i] = keep + __shfl_xor(give, 32, 64);
  }
  float h2[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const float keep = b4 ? h4[i + 2] : h4[i];
    const float give = b4 ? h4[i] : h4[i + 2];
    h2[i] = keep + __shfl_xor(give, 16, 64);
  }
  float s = (b3 ? h2[1] : h2[0]) + __shfl_xor(b3 ? h2[0] : h2[1], 8, 64);
  s += __shfl_xor(s, 4, 64);
  s += __shfl_xor(s, 2, 64);
  s += __shfl_xor(s, 1, 64);
  return s;
}

// The base waves' part of a first unit that takes several passes (contracted
// before the weight loop): every pass, then this wave's partial rows into red
// (the pass's other rows as zero), then the wave counts in.
__device__ void unit_contract(const GemvParams& p, const Unit& un, float* red, int* done, int wave, int lane) {
  const int len = un.steps * 32;
  const int rsel = 4 * ((lane >> 5) & 1) + 2 * ((lane >> 4) & 1) + ((lane >> 3) & 1);
  for (int j0 = 0; j0 < un.rows;) {
    const PassShape ps = pass_shape<8>(un, j0);
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = 0.f;
    for (int ub = 0; ub == 0 || ub * ps.c * kPieceK < len; ++ub) {
      UnitPieces<8> f;
      unit_pieces(p, un, j0, ub, ps, wave, lane, f);
      unit_dots(f, ps.pw, v);
    }
    const float s = unit_reduce(v, lane);
    if (lane < ps.rp) red[wave * 192 + j0 + lane] = 0.f;
    if ((lane & 7) == 0 && rsel < ps.pw) red[wave * 192 + j0 + (wave / ps.c) * ps.pw + rsel] = s;
    j0 += ps.rp;
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the partial rows are in LDS
  if (lane == 0) lds_count_in(done);
}

// A unit whose rows fit one pass and whose slice fits one group of c chunks
// is contracted from the first pass alone (inside the weight loop).
__device__ __forceinline__ bool unit_single_pass(const Unit& un, const PassShape& ps) {
  return un.rows <= ps.rp && un.steps * 32 <= ps.c * kPieceK;
}

__device__ __forceinline__ void unit_contract_single(const UnitPieces<4>& pre, const PassShape& ps, float* red,
                                                     int* done, int wave, int lane) {
  float v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = 0.f;
  unit_dots(pre, ps.pw, v);
  const float s = unit_reduce(v, lane);
  const int rsel = 4 * ((lane >> 5) & 1) + 2 * ((lane >> 4) & 1) + ((lane >> 3) & 1);
  if (lane < ps.rp) red[wave * 192 + lane] = 0.f;
  if ((lane & 7) == 0 && rsel < ps.pw) red[wave * 192 + (wave / ps.c) * ps.pw + rsel] = s;
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the partial rows are in LDS
  if (lane == 0) lds_count_in(done);
}

// Tile metadata of the wide kernel (the fields its base waves and the
// recompute read): per token g, r and scale; the distinct live slots in
// order of first use with their rank, B stride and B offset; the slice
// bounds; then the ready flag. One ballot per distinct slot records the
// slot's first token in a register lane; the slot fields come from that
// token's lane by shuffles after the loop (no LDS stores inside it).
__device__ void lora_meta_wide(char* lds, const TokenMeta& m, int sbound, int lane) {
  TileMeta* tm = reinterpret_cast<TileMeta*>(lds + WL::kMeta);
  if (lane < 32) {
    tm->g[lane] = m.g;
    tm->r[lane] = m.r;
    tm->scale[lane] = m.scale;
  }
  if (lane < 4) tm->bounds[lane] = sbound;
  uint64_t left = __ballot(m.g >= 0);  // (lanes past the tile hold g = -1)
  int nd = 0;
  int first = 0;  // lane d < nd: the first token of distinct slot d
  while (left) {
    const int f = __builtin_ctzll(left);
    const int gf = __builtin_amdgcn_readlane(m.g, f);
    first = lane == nd ? f : first;
    left &= ~__ballot(m.g == gf);
    ++nd;
  }
  const int src = first << 2;
  const int dg = __builtin_amdgcn_ds_bpermute(src, m.g);
  const int dr = __builtin_amdgcn_ds_bpermute(src, m.r);
  const int dst = __builtin_amdgcn_ds_bpermute(src, m.stride);
  const uint32_t blo = uint32_t(__builtin_amdgcn_ds_bpermute(src, int(uint32_t(uint64_t(m.boff)))));
  const uint32_t bhi = uint32_t(__builtin_amdgcn_ds_bpermute(src, int(uint32_t(uint64_t(m.boff) >> 32))));
  if (lane < nd) {
    tm->dslot[lane] = dg;
    tm->dr[lane] = dr;
    tm->dstride[lane] = dst;
    tm->dboff[lane] = int64_t((uint64_t(bhi) << 32) | blo);
  }
  if (lane == 0) tm->nd = nd;
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the metadata is in LDS
  if (lane == 0) *(volatile __attribute__((address_space(3))) int*)(&tm->ready) = 1;
}

// z of the tile into LDS, fixed layout. Lane-group q (one per lane and
// batch) owns vg = 8 / KZ consecutive values of one token and slice: token
// i = q / gt, slice s = (q % gt) / gs, positions j0 = vg (q % gs) .. + vg,
// where gs = pl / vg groups cover the part of a slice the expand reads (pl:
// max_rank rounded up to 16) and gt = slices * gs. A lane polls its vg x KZ
// tagged partials until every one it needs carries the call's tag, sums the
// k-slices in registers and writes its values as bf16 with one store (zero
// past the token's rank, for base-only tokens and tokens past the batch).
// Token i's rank comes from lane i of the token metadata by a shuffle; no
// list is searched. Returns true when a wait gave up (the caller recomputes).
template <int KZ>
__device__ bool gather_wide_kz(const GemvParams& p, char* lds, const TokenMeta& m, int t0, uint32_t tag, int lane) {
  constexpr int VG = 8 / KZ;
  char* zl = lds + WL::kZ;
  const int pl = (p.max_rank + 15) & ~15;
  const int gs = pl / VG;
  const int gt = p.slices * gs;
  const int total = kTokens * gt;
  const uint64_t* block = p.zp + int64_t(t0) * p.zw * KZ;
  bool gave_up = false;
  for (int q0 = 0; q0 < total; q0 += 64) {
    const int q = q0 + lane;
    const int i = min(q / gt, kTokens - 1);
    const int rem = q - i * gt;
    const int s = rem / gs;
    const int j0 = (rem - s * gs) * VG;
    const int ri = __builtin_amdgcn_ds_bpermute(i << 2, m.r);
    const int cnt = q < total ? max(0, min(VG, ri - j0)) : 0;
    const int64_t base = (int64_t(i) * p.zw + s * ri + j0) * KZ;
    uint64_t v[VG][KZ];
    for (int spins = 0;; ++spins) {
#pragma unroll
      for (int vv = 0; vv < VG; ++vv)
#pragma unroll
        for (int ks = 0; ks < KZ; ++ks)  // unconditional: no per-load branch
          v[vv][ks] = tagged_load(block + (vv < cnt ? base + vv * KZ + ks : 0));
      bool ok = true;
#pragma unroll
      for (int vv = 0; vv < VG; ++vv)
#pragma unroll
        for (int ks = 0; ks < KZ; ++ks) ok = ok && (vv >= cnt || uint32_t(v[vv][ks] >> 32) == tag);
      if (__all(ok)) break;
      if (spins > p.spin_limit) {
        gave_up = true;  // (cannot happen while producers run: they wait for nothing)
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    uint32_t w[(VG + 1) / 2];
#pragma unroll
    for (int h = 0; h < (VG + 1) / 2; ++h) {
      float z2[2] = {0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int vv = 2 * h + e;
        if (vv >= VG) break;
        float z = 0.f;
#pragma unroll
        for (int ks = 0; ks < KZ; ++ks) z += __uint_as_float(uint32_t(v[vv][ks]));
        z2[e] = vv < cnt ? z : 0.f;
      }
      w[h] = pack_bf16x2(z2[0], z2[1]);
    }
    if (q < total) {
      char* dst = zl + (i * WL::kZRow + s * 64 + j0) * 2;
      if constexpr (VG == 8) *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
      else if constexpr (VG == 4) *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
      else if constexpr (VG == 2) *reinterpret_cast<uint32_t*>(dst) = w[0];
      else *reinterpret_cast<uint16_t*>(dst) = uint16_t(w[0]);
    }
  }
  return gave_up;
}

__device__ void gather_wide(const GemvParams& p, char* lds, const TokenMeta& m, int t0, int mt, uint32_t tag,
                            int lane) {
  bool gave_up;
  switch (p.kz) {
    case 1: gave_up = gather_wide_kz<1>(p, lds, m, t0, tag, lane); break;
    case 2: gave_up = gather_wide_kz<2>(p, lds, m, t0, tag, lane); break;
    case 4: gave_up = gather_wide_kz<4>(p, lds, m, t0, tag, lane); break;
    default: gave_up = gather_wide_kz<8>(p, lds, m, t0, tag, lane); break;
  }
  if (gave_up) {
    // Every z value is recomputed from x and A (the status word reports it);
    // the area is cleared first, as batches after the one that gave up were
    // not written.
    uint4* z4 = reinterpret_cast<uint4*>(lds + WL::kZ);
    for (int e = lane; e < kTokens * WL::kZRow / 8; e += 64) z4[e] = make_uint4(0, 0, 0, 0);
    lora_recompute<WideTile>(p, lds, t0, mt, lane);
  }
}

// The LoRA wave of a wide workgroup: publishes the workgroup's first shrink
// unit as soon as the base waves have counted in, builds the tile metadata,
// produces the other units (small grids only), gathers z, and takes its part
// in the workgroup's two remaining barriers (z ready; partial tiles in LDS)
// before it counts the workgroup out of the call.
__device__ __forceinline__ void lora_wave(const GemvParams& p, char* lora_lds, float* red, int* prod_done, int g_tile,
                                       int sbound, const SlotTable& stab, uint32_t epoch, int t0, int mt, int lane) {
  // (At the base waves' issue priority: raised to 3, as an earlier form of
  // this chain was, c4 and c3's B = 64 MLP took about 0.9 us longer and the
  // headline the same.)
  const TokenMeta tmeta =
      slot_table_usable(p) ? token_meta_from(p, stab, g_tile, mt, lane) : token_meta(p, g_tile, mt, lane);
  Unit un0{};
  const bool has0 = int(blockIdx.x) < p.producers && int(blockIdx.x) < p.units && unit_of(p, blockIdx.x, un0);
  const uint32_t tag = __builtin_amdgcn_readfirstlane(epoch) + 1u;
  lora_meta_wide(lora_lds, tmeta, sbound, lane);  // first: the base waves request B with it before their loop
  if (has0) publish_first_unit<kBase>(p, red, prod_done, un0, tag, lane);
  produce_other_units<kFirstSteps>(p, tag, lane);
  gather_wide(p, lora_lds, tmeta, t0, mt, tag, lane);
  const uint32_t departed = depart_issue(p.ce, lane);  // after the last partial load
  lds_barrier();  // z and the tile metadata are in LDS
  lds_barrier();  // the partial tiles are in LDS
  depart_finish(p.ce, departed, __builtin_amdgcn_readfirstlane(epoch), lane);
}

// kDWG: weight group slots per wave (the launcher uses 1; the ring and its
// waits are written for 1 or 2).
// kLora: a ninth wave and the LoRA stages (row groups must fill whole XCD
// octets, so every workgroup of the grid is a real one and counts in once).
// kResidual (with kLora): no weight; y is the base and is updated in place
// with each routed token's LoRA delta (the one-launch shrink + expand).
// kDq: the launch passes a double-quant state (dq_scales.h), a variant of
// its own so that the fp32-scale kernels carry none of its registers.
template <bool kExact, int kDWG, bool kLora, bool kResidual = false, bool kDq = false>
__global__ __launch_bounds__(64 * (kBase + (kLora ? 1 : 0)), 1) void nf4_decode_wide_kernel(GemvParams p) {
  static_assert(!kResidual || (kLora && !kExact), "the residual form is a LoRA-only variant");
  static_assert(!(kResidual && kDq), "the residual form reads no weight");
  constexpr int kCP = 16;  // pair-table copies (lane l reads copy l % kCP)
  __shared__ __attribute__((aligned(16))) char wring[kBase * kDWG * kWGroup];
  __shared__ __attribute__((aligned(16))) char xring[kBase * kDX * kXSlot];
  __shared__ float table[16];
  __shared__ __attribute__((aligned(16))) uint32_t pt[kExact ? 4 : 256 * kCP];
  __shared__ __attribute__((aligned(16))) char lora_lds[kLora ? WL::kBytes : 16];
  __shared__ int prod_done;   // base waves that have written their first-unit partials
  __shared__ int table_done;  // (LoRA) base waves 0..3 that have written their part of the decode table
  __shared__ int dq_ready;    // double quant: wave 0's code2 copies have landed
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
  const int kb0 = base && !kResidual ? nblk * wave / kBase : 0;
  const int nb = base && !kResidual ? nblk * (wave + 1) / kBase - kb0 : 0;
  const int groups = (nb + 3) >> 2;
  char* myw = wring + (base ? wave : 0) * kDWG * kWGroup;
  char* myx = xring + (base ? wave : 0) * kDX * kXSlot;
  char* mysc = scale_lds + (base ? wave : 0) * p.sc_bytes;
  // Double quant: code2 after the scale areas (1 KiB of dynamic LDS that only
  // those launches allocate).
  float* dq_table = reinterpret_cast<float*>(scale_lds + kBase * p.sc_bytes + 16);
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
  // (With LoRA: base waves only, once their copies are out, so the LoRA
  // wave's early barrier does not wait for these loads and the values are
  // not held across the copy issue.)
  float cb[16];
  auto load_codebook = [&]() {
#pragma unroll
    for (int i = 0; i < 16; ++i) cb[i] = sload(p.code, i);
  };
  if constexpr (!kLora) load_codebook();

  // With LoRA, the LoRA wave clears the workgroup's flags and requests the
  // call epoch, its tile's token slots and the per-slot metadata before one
  // early barrier, so those loads are ahead of every copy of the workgroup; after
  // it the base waves build the decode table behind their copies and count
  // in on table_done, and the LoRA wave meets them again only at the z
  // barrier (a barrier after the copies would hold it until the base waves
  // had issued all of theirs).
  uint32_t epoch = 0;
  int g_tile = -1;
  int g0 = -1;  // slot of the token of this workgroup's first unit (base waves)
  int sbound = 0;  // (LoRA wave) slice_offsets[min(lane % 4, slices)]
  SlotTable stab;
  if constexpr (kLora) {
    if (base) {
      g0 = sload(p.token_slots, unit_token(p, min(int(blockIdx.x), p.units - 1)));
      barrier_only();  // (no wait: the base waves' scalar loads stay in flight)
    } else {
      if (lane == 0) {
        reinterpret_cast<TileMeta*>(lora_lds + WL::kMeta)->ready = 0;
        prod_done = 0;
        table_done = 0;
        dq_ready = 0;
      }
      epoch = __hip_atomic_load(p.ce.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      g_tile = p.token_slots[t0 + min(lane, mt - 1)];
      sbound = p.slice_offsets[min(lane & 3, p.slices)];
      if (slot_table_usable(p)) slot_table_load(p, lane, stab);
      lds_barrier();  // the flags are cleared
    }
  }

  // Copies: the block scales, the first weight groups and the first x
  // blocks, then (a producing workgroup) the first unit's A and x pieces.
  // The base waves contract the pieces once they land (ordinary loads: the
  // compiler waits for them, and as loads complete in issue order, for every
  // copy before them; the x blocks are therefore requested first).
  Unit un0{};
  bool has0 = false;
  bool single = false;  // the first unit is contracted inside the loop (from pre4)
  UnitPieces<4> pre4;
  // Double quant: the codes and absmax2 entries are staged instead of fp32
  // scales (code2 requested ahead of every copy) and converted before the loop.
  constexpr bool dq = kDq;
  float dq_off = 0.f;
  DqStage dqs{};
  if (base) {
    if constexpr (dq) {
      if (wave == 0) dq_issue_code2(p, dq_table, lane);  // ahead of wave 0's staging
    }
    if (nb > 0) {
      if constexpr (dq) {
        dq_off = sload(p.dq_offset, 0);
        dqs = dq_stage(p, p.sc_bytes, kRows, lo, hi, kb0, nb);
        dq_issue(p, mysc, dqs, kRows, lo, hi, kb0, lane);
      } else {
        issue_scales(p, mysc, lo, hi, kb0, nb, lane);
      }
#pragma unroll
      for (int g2 = 0; g2 < kDWG; ++g2)
        if (g2 < groups) issue_w(g2, g2);
    }
    if (nb > 0) {
#pragma unroll
      for (int s = 0; s < kDX; ++s)
        if (s < nb) issue_x(s, s);
    }
    if constexpr (kLora) {
      has0 = int(blockIdx.x) < p.producers && int(blockIdx.x) < p.units && unit_of_slot(p, blockIdx.x, g0, un0);
      if (has0) {
        single = unit_single_pass(un0, pass_shape<4>(un0, 0));
        if (single) unit_pieces(p, un0, 0, 0, pass_shape<4>(un0, 0), wave, lane, pre4);
      }
    }
  }

  // Residual form: thread t's two outputs of y (the base), requested now.
  uint32_t ybase[2] = {0u, 0u};
  if constexpr (kResidual) {
    const int tok = threadIdx.x >> 4;
    if (base && tok < mt) {
#pragma unroll
      for (int h = 0; h < 2; ++h) ybase[h] = p.y[int64_t(t0 + tok) * p.y_stride + wrow(lo, hi, (threadIdx.x & 15) + 16 * h)];
    }
  }

  if constexpr (kResidual) {
    // (no weight: no decode table)
  } else if constexpr (kLora) {
    // Waves 0..3: entry t = threadIdx.x of the pair table (and the codebook
    // for the exact decode), from the codebook in scalar registers.
    if (base && wave < 4) {
      load_codebook();
      const int t = threadIdx.x;
      float c_lo = cb[0], c_hi = cb[0];
#pragma unroll
      for (int q = 1; q < 16; ++q) {
        c_lo = (t >> 4) == q ? cb[q] : c_lo;
        c_hi = (t & 15) == q ? cb[q] : c_hi;
      }
      if (t < 16) table[t] = c_hi;
      if constexpr (!kExact) {
        const uint32_t v = pack_bf16x2(c_lo, c_hi);
        uint4* dst = reinterpret_cast<uint4*>(pt + t * kCP);
#pragma unroll
        for (int c = 0; c < kCP / 4; ++c) dst[c] = make_uint4(v, v, v, v);
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's entries are in LDS
      if (lane == 0) lds_count_in(&table_done);
    }
  } else {
    if (threadIdx.x == 0) {
#pragma unroll
      for (int i = 0; i < 16; ++i) table[i] = cb[i];
      dq_ready = 0;  // set by wave 0 after the barriers below
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
  }
  const uint32_t* ptl = pt + (lane % kCP);

  // The base waves; the LoRA wave's code follows theirs (so nothing of the
  // streaming state is live across it).
  if (base) {
  if constexpr (kLora && !kResidual) {
    while (*(const volatile __attribute__((address_space(3))) int*)(&table_done) < 4) __builtin_amdgcn_s_sleep(1);
  }
  // A producing wave contracts its part of a single-pass first unit inside
  // the loop, after block p.contract_after: the pieces were requested before
  // the refills of the blocks before it and have usually landed, and the loop
  // is not held back until they do (a wave with fewer blocks contracts after the
  // loop). Longer units are contracted here, before the loop, so their
  // partials are not late for the other workgroups.
  bool contract = false;
  PassShape ps0{};
  if constexpr (kLora) {
    if (has0) {
      ps0 = pass_shape<4>(un0, 0);
      if (single) contract = true;
      else unit_contract(p, un0, red, &prod_done, wave, lane);
    }
  }

  if constexpr (dq) {
    // The staging (and wave 0's code2 copies before it) was requested first:
    // it has landed once no more than the weight groups and x blocks
    // requested after it are outstanding (loads complete in issue order; a
    // producer's unit pieces came later still). Wave 0 raises dq_ready
    // whether or not it has blocks (short K); the others wait for it, with
    // a bound, before reading code2.
    const int after = nb > 0 ? 4 * (min(kDWG, groups) + min(kDX, nb)) : 0;
    switch (after) {
      case 16: wait_vm<16>(); break;
      case 12: wait_vm<12>(); break;
      case 8: wait_vm<8>(); break;
      default: wait_vm<0>(); break;
    }
    if (wave == 0) {
      if (lane == 0) __hip_atomic_store(&dq_ready, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    } else if (nb > 0) {
      for (int spins = 0; spins < kSpinLimit &&
                          *(const volatile __attribute__((address_space(3))) int*)(&dq_ready) == 0;
           ++spins)
        __builtin_amdgcn_s_sleep(1);
    }
    if (nb > 0) dq_convert<kDqEntries>(p, mysc, dqs, kRows, lo, hi, kb0, nb, dq_table, dq_off, lane);
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
      if constexpr (kLora) {
        if (contract && bl == p.contract_after) {
          unit_contract_single(pre4, ps0, red, &prod_done, wave, lane);
          contract = false;
        }
      }
    }
  }
  if constexpr (kLora) {
    if (contract) unit_contract_single(pre4, ps0, red, &prod_done, wave, lane);
  }
  wait_vm<0>();
  const GemvParams& pe = reload();  // the epilogue's parameters, read where used

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
    const WaveSlots ws = wave_slots(tm, wave, lane);
    expand_request(pe, ws, eb, lo, hi, wave, lane);
    expand_fix(ws, eb, lo, hi, wave, lane);
    lds_barrier();  // z and the tile metadata are in LDS
    dacc = expand_wide(pe, lora_lds, ws, eb, lo, hi, wave, lane);
  }

  // Sum the partial tiles: base wave w writes its accumulators (and delta
  // tile) into its own x ring (all of its copies have landed and been read),
  // element r of lane l at r * 64 + l (the delta 1024 floats further).
  {
    float* mine = reinterpret_cast<float*>(myx);
    if constexpr (!kResidual) {
#pragma unroll
      for (int e = 0; e < 16; ++e) mine[e * 64 + lane] = acc[e];
    }
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
        if constexpr (!kResidual) sum += part[o];
        if constexpr (kLora) dsum += part[1024 + o];
      }
      if constexpr (kResidual) sum = bf16_to_f32(ybase[h]);
      const int row = wrow(lo, hi, col);
      float v = round_bf16(sum);
      if (pe.bias) v = round_bf16(v + bf16_to_f32(pe.bias[row]));
      if (routed) v += round_bf16(dsum * lscale);
      out[h] = round_bf16(v);
      // (The residual form leaves base-only tokens' y untouched.)
      if (!pe.gated_half && tok < mt && (!kResidual || routed))
        pe.y[int64_t(t0 + tok) * pe.y_stride + row] = uint16_t(f32_to_bf16(v));
    }
    // SwiGLU output h = bf16(bf16(silu(gate)) * up) for feature lo + jj (the
    // reference's activation after both LoRA adds, benchmarks/qwen35_decode_silu.py:60-61).
    if (pe.gated_half && tok < mt)
      pe.y[int64_t(t0 + tok) * pe.y_stride + lo + jj] = uint16_t(f32_to_bf16(silu_times(out[0], out[1])));
  }
  } else {
    if constexpr (kLora) lora_wave(reload(), lora_lds, red, &prod_done, g_tile, sbound, stab, epoch, t0, mt, lane);
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
template <bool kExact, int kDWG, bool kLora, bool kResidual = false, bool kDq = false>
bool try_launch(dim3 grid, hipStream_t s, const GemvParams& p, int64_t dyn) {
  static int64_t static_lds = -1;
  auto fn = nf4_decode_wide_kernel<kExact, kDWG, kLora, kResidual, kDq>;
  const int64_t st = static_lds_of(fn, static_lds);
  if (st < 0 || st + dyn > kLdsBytes) return false;
  hipLaunchKernelGGL(fn, grid, dim3(64 * (kBase + (kLora ? 1 : 0))), size_t(dyn), s, p);
  return true;
}

template <bool kExact, bool kLora>
// One weight-group slot per wave at every K (the second group is requested
// after the first one's fourth block), which also leaves the LDS for 16
// pair-table copies with LoRA. Measured on MI355X against two slots (the
// whole W of a wave at K = 4096 requested up front) and 8 copies with LoRA:
// headline 15.5 -> 14.7 us, north star B = 16 / 32 / 64 14.2 / 14.6 / 15.1
// -> 13.5 / 14.2 / 14.3-14.8 us, base only B = 64 10.1 -> 9.8 us, exact
// weights B = 64 16.1 -> 15.7 us, c4 66.3 -> 64.4 us, c3 B = 64 98.5 -> 94.7
// us; with two slots and 8 copies the loop's LDS reads conflicted more and
// the up-front weight requests queued ahead of the x blocks. 32 copies were
// slower again (headline 15.1 us).
bool launch_variant(dim3 grid, hipStream_t s, const GemvParams& p, int64_t dyn) {
  if (p.absmax_q) return try_launch<kExact, 1, kLora, false, true>(grid, s, p, dyn);
  return try_launch<kExact, 1, kLora>(grid, s, p, dyn);
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

// Whether the wide kernel reads this nested state itself (dq_scales.h).
// (The code2 table's 1 KiB must fit beside the largest static LDS, that of
// the LoRA variant with one weight group per wave.)
bool wide_takes_dq(const lf_nf4_weight* w) {
  const int64_t nblk = w->k / 64;
  const int64_t nbw = (nblk + kBase - 1) / kBase;
  const int64_t smallest = int64_t(kBase) * (kWGroup + kDX * kXSlot) + 256 * 16 * 4 + 64 + WL::kBytes;
  return dq_layout_ok(w, kRows) && dq_cols_per_lane(kRows, int(scale_stride(nblk))) <= kDqEntries &&
         dq_stage_bytes(kRows, int(nbw)) <= scale_area_bytes(nblk) &&
         smallest + kBase * scale_area_bytes(nblk) + 16 + 1024 <= kLdsBytes;
}

int device_cus();

// Shrink units of the wide kernel: k-slices only as many as keep a tile's
// partials (32 tokens x zw x kz) to one gather batch of 512 entries (8 per
// lane of the LoRA wave) and leave a producer per unit, then 4-row ranges
// (the VALU contraction takes any number of rows) until every workgroup up
// to min(grid, CUs) produces one unit: no workgroup contracts a larger share
// of the adapters' A than the others and holds the call's end.
GemvPlan wide_plan(int64_t m, int64_t n, int64_t k, int cus, int zw) {
  GemvPlan pl;
  pl.rows = kRows;
  pl.row_groups = int(n / kRows);
  pl.grid = pl.row_groups * int((m + kTokens - 1) / kTokens);
  const int64_t cap = std::min<int64_t>(pl.grid, cus);
  const int64_t nblk = k / 64;
  int64_t kz = std::max<int64_t>(
      1, std::min<int64_t>({nblk, 8, 512 / (int64_t(kTokens) * zw), cap / std::max<int64_t>(1, m)}));
  while (kz & (kz - 1)) kz &= kz - 1;  // a power of two (the consumer sums the slices unrolled)
  pl.kz = int(kz);
  pl.kz_len = int((nblk + kz - 1) / kz) * 64;
  const int64_t groups = (zw + 3) / 4;  // 4-row groups per token
  // (Grids of several dispatch rounds: at most two units per token and
  // slice, c3's gate/up at B = 64 about 2 us faster; one round: as many as
  // the producers allow, B = 64 0.9 us faster than two.)
  const int64_t split = std::max<int64_t>(
      1, std::min<int64_t>({groups, cap / (m * kz), pl.grid > cus ? int64_t(2) : groups}));
  pl.urows = int((groups + split - 1) / split) * 4;
  pl.usplit = int((groups * 4 + pl.urows - 1) / pl.urows);
  pl.units = int(m) * pl.usplit * pl.kz;
  pl.producers = int(cap);
  return pl;
}

// Batches the wide kernel serves faster than the narrow one (measured on
// MI355X with one weight slot and 16 table copies, us per call with 32
// rank-16 adapters; narrow / wide):
//   4096 x 4096 at 2 / 4 / 8 / 12 / 16 / 24 tokens: 10.1 / 11.2 / 11.6 /
//     15.2 / 14.8 / 16.4 against 12.6 / 12.7 / 13.1 / 13.2 / 13.5 / 13.8;
//   N = 8192 / 12288 / 16384 / 24576 (K = 4096) at 2 tokens: 12.8 / 20.1 /
//     21.6 / 30.8 against 13.1 / 19.7 / 22.5 / 32.1; at 3: 13.4 / 21.9 /
//     23.8 / 33.4 against 13.3 / 19.9 / 22.7 / 32.2; at 8: 14.5 / 24.1 /
//     25.8 / 36.6 against 13.6 / 21.0 / 24.2 / 34.3 (the narrow kernel's
//     two workgroups per CU win while one round of them covers N);
//   4096 x 12288 at 4 / 8 / 12 / 16 / 24: 17.1 / 21.1 / 23.7 / 24.9 / 33.3
//     against 23.1 / 23.8 / 24.5 / 24.9 / 26.2 (128 workgroups with one
//     weight slot a wave: long K keeps the narrow kernel up to 16 tokens).
bool wide_takes_batch(int64_t m, int64_t n, int64_t k) {
  if (k > 8192) return m > 16;
  return m > 8 || (m > 2 && n >= 8192);
}

// Whether the wide decode kernel takes this call: a batch it serves faster
// (wide_takes_batch), a K whose rings and scale areas fit LDS (the smallest
// variant), and with LoRA row groups that fill whole XCD octets (N a multiple
// of 256), shrink partials that fit the workspace header and at most 1024
// units.
bool decode_wide_fits(int64_t m, int64_t n, int64_t k, const lf_lora* lora) {
  if (!wide_takes_batch(m, n, k) || n % kRows) return false;
  const int64_t nblk = k / 64;
  const int64_t area = scale_area_bytes(nblk);
  // Static LDS of the smallest variant: one weight group and two x blocks per
  // base wave, the pair table and (with LoRA) the z area.
  const int64_t smallest = int64_t(kBase) * (kWGroup + kDX * kXSlot) + 256 * 16 * 4 + 64 + (lora ? WL::kBytes : 0);
  if (smallest + kBase * area + 16 > kLdsBytes) return false;
  if (!lora) return true;
  if (n % (8 * kRows)) return false;
  const GemvPlan pl = wide_plan(m, n, k, device_cus(), lora->num_slices * lora->max_rank);
  return pl.units <= 1024 && kPartialsOffset + m * pl.kz * lora->num_slices * lora->max_rank * 8 <= kWorkspaceHeader;
}

// The residual form (one launch of shrink + expand onto y, no weight) for
// 33..64 tokens: N a multiple of 256 (whole XCD octets of 32-row groups) and
// the unit plan's limits.
bool lora_apply_wide_fits(int64_t m, int64_t n, int64_t k, const lf_lora* lora) {
  if (m <= 32 || m > 64 || n % (8 * kRows)) return false;
  const GemvPlan pl = wide_plan(m, n, k, device_cus(), lora->num_slices * lora->max_rank);
  return pl.units <= 1024 && kPartialsOffset + m * pl.kz * lora->num_slices * lora->max_rank * 8 <= kWorkspaceHeader;
}

int launch_lora_apply_wide(const uint16_t* x, int64_t m, int64_t x_stride, int64_t n, int64_t k, const lf_lora* lora,
                           uint16_t* y, int64_t y_stride, void* workspace, int64_t workspace_bytes, bool withhold,
                           void* stream) {
  LF_REQUIRE(lora && lora_apply_wide_fits(m, n, k, lora), "wide LoRA apply: call outside its range");
  GemvParams p{};
  p.x = x;
  p.x_stride = x_stride;
  p.m = int(m);
  p.n = int(n);
  p.k = int(k);
  p.y = y;
  p.y_stride = y_stride;
  p.row_groups = int(n / kRows);
  p.tiles = int((m + kTokens - 1) / kTokens);
  const GemvPlan pl = wide_plan(m, n, k, device_cus(), lora->num_slices * lora->max_rank);
  const int rc = fill_lora_params(p, pl, lora, m, workspace, workspace_bytes, withhold);
  if (rc != kOk) return rc;
  const dim3 g3(static_cast<unsigned>(int64_t(p.row_groups) * p.tiles));
  LF_REQUIRE((try_launch<false, 2, true, true>(g3, static_cast<hipStream_t>(stream), p, 16)),
             "wide LoRA apply: LDS does not fit");
  LF_HIP(hipGetLastError());
  return kOk;
}

int launch_decode_wide(const uint16_t* x, int64_t m, int64_t x_stride, const lf_nf4_weight* w, const uint16_t* bias,
                       const lf_lora* lora, uint16_t* y, int64_t y_stride, void* workspace, int64_t workspace_bytes,
                       bool exact, bool swiglu, bool withhold, void* stream) {
  LF_REQUIRE(decode_wide_fits(m, w->n, w->k, lora), "wide decode: call outside its range");
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
  p.sc_magic = stride_magic(p.sc_stride);
  if (!w->scales) {
    // A nested state: staged and converted by the kernel where its layout
    // allows (a wave's area rows x stride at most 16 entries per lane),
    // else fp32 scales rebuilt into the workspace.
    if (wide_takes_dq(w)) {
      fill_dq_params(p, w);
    } else {
      const int rc = rebuild_scales(w, workspace, workspace_bytes, stream, &p.scales);
      if (rc != kOk) return rc;
    }
  }
  if (lora) {
    const GemvPlan pl = wide_plan(m, w->n, w->k, device_cus(), lora->num_slices * lora->max_rank);
    const int rc = fill_lora_params(p, pl, lora, m, workspace, workspace_bytes, withhold);
    if (rc != kOk) return rc;
    const int64_t cus = device_cus();
    p.contract_after = pl.grid > cus    ? kContractAfterRounds
                       : pl.grid >= cus ? kContractAfterOneRound
                                        : kContractAfterPartialRound;
  }
  const int64_t dyn = int64_t(kBase) * p.sc_bytes + 16 + (p.absmax_q ? 1024 : 0);
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
