// Fused NF4 base linear + per-token multi-LoRA for decode batches (M <= 64),
// one kernel launch per call.
//
// Reference chain being fused:
//   integrations/_sglang_nf4_linear.py:116-129  y = bf16(x @ dequant(W)^T) (+bias)
//   ops/csrc/lora_rows.cu:35-65                 z = bf16(A_g @ x)
//   ops/csrc/lora_rows.cu:67-117                y = bf16(bf16(y) + bf16(scale * B_g @ z))
//
// Work split. A group owns 16*WAVES output rows (one 16-row MFMA tile per
// wave) and one K range of NSEG segments of 256 k; groups of one row range
// differ only in their K range ("splits").
//
// Memory path. Packed W bytes and x are copied HBM/L2 -> LDS with the gfx950
// direct copy (global_load_lds_dwordx4): every copy instruction moves 1 KiB of
// whole 128-byte lines, so the address unit handles 8 lines per instruction
// instead of 16 partial lines per fragment load. All segments are requested
// up front into separate LDS objects; segment s is consumed after an explicit
// vmcnt wait that covers only the copies issued before it, so the contraction
// of early segments overlaps the arrival of later ones. The copies permute
// 16-byte units within each row (XOR swizzle) so the MFMA fragment reads from
// LDS are bank-conflict free. Block scales of the group are staged once.
//
// Arithmetic. v_mfma_f32_16x16x32_bf16 with x as the A operand (tokens padded
// to 16 per tile) and W^T as the B operand. Default: B = bf16(code[nibble])
// from a byte -> bf16-pair table in LDS and the fp32 block scale applied to
// the per-block MFMA sums. Exact mode (LF_EXACT_WEIGHTS): B = bf16_rne(code *
// scale), the reference's dequantised weight bit for bit.
//
// Split-K. Each split stores its fp32 partial tile for real tokens; the last
// split to arrive sums them in split order (deterministic) and runs the
// epilogue from registers.
//
// LoRA, in the same launch:
//   shrink  - the distinct adapter slots of the batch are split into
//             (slot, k-slice) units; group g computes unit g (units are kept
//             <= 256 and below the grid size, so every producer is among the
//             first groups dispatched and none of them waits before
//             producing). fp32 partial z goes to the workspace.
//   expand  - slot d belongs to split (d mod splits) of every row range: that
//             group waits for all shrink units (bounded spin), stages
//             z = bf16(sum of partials) in LDS and runs one masked MFMA per
//             owned slot and slice against the slot's B rows, giving the fp32
//             delta sum of its tokens.
//   epilogue- v = bf16(acc); v = bf16(v + bias); v = bf16(v + bf16(delta * scale)).
// Slot metadata (rank, offsets, stride, scale) is read with scalar loads so
// it never queues behind the weight copies.
//
// Cross-workgroup exchange uses no cache-wide fences: values another
// workgroup reads (partials, z, counters) are written and read with
// device-coherent (agent-scope) relaxed atomic accesses; a producer's stores
// complete (the workgroup release inside __syncthreads waits for them) before
// its counter update is issued, and a consumer loads only after observing the
// counter. Counters are reset by their last user, so the workspace is left
// zeroed.
#include <algorithm>

#include "nf4_common.h"
#include "../../include/loraforge_amd.h"

namespace lf {
namespace {

constexpr int kSegK = 256;      // k per pipeline segment: 4 NF4 blocks
constexpr int kShrinkK = 1024;  // k per lane pass of the shrink dot products (2 x 8 per lane)
constexpr int kCtrlBytes = 512;
constexpr int kSpinLimit = 1 << 22;
constexpr int kMaxUnits = 256;
// Control words: groups finished, status, and one z-ready counter per distinct slot.
enum Ctrl { kDone = 1, kStatus = 2, kSlotDone = 64 };

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
  int splits;  // K ranges per row range
  int krange;  // k per split
  int kz;      // shrink k-slices per slot
  int kz_len;  // k per shrink slice (multiple of kShrinkK)
  int zw;      // z row width = slices * max_rank
  int* ctrl;
  int* tile_count;
  float* zpart;  // [kz][m][zw]
  float* dpart;  // [m][n]
  float* part;   // [groups][m][rows]
};

// XR: token rows of x staged per segment: 16 * TM, or 2 for one- and
// two-token batches (other MFMA rows then repeat those two; they are never stored).
template <int WAVES, int TM, int NSEG, int XR = 16 * TM>
struct Shape {
  static constexpr int kXRows = XR;
  static constexpr int kWaves = WAVES;
  static constexpr int kThreads = 64 * WAVES;
  static constexpr int kRows = 16 * WAVES;
  static constexpr int kTM = TM;
  static constexpr int kNSeg = NSEG;
  static constexpr int kBlk = 4 * NSEG;        // NF4 blocks per row per group
  static constexpr int kScStride = kBlk + 1;   // padded: conflict-free scale reads
  static constexpr int kWSeg = kRows * 128;    // packed W bytes per segment
  static constexpr int kXSeg = XR * 512;  // x bytes per segment
  static constexpr int kWDma = kWSeg / (1024 * WAVES);
  // x copies per wave; a segment smaller than one copy per wave is moved by
  // wave 0 while the other waves issue one dummy copy (keeps counts uniform).
  static constexpr int kXDma = kXSeg >= 1024 * WAVES ? kXSeg / (1024 * WAVES) : 1;
  static constexpr bool kXSmall = kXSeg < 1024 * WAVES;
  static constexpr int kDmaSeg = kWDma + kXDma;  // copies per wave per segment
  static constexpr int kCopies = TM == 1 ? 32 : 16;
  static constexpr int kZlBytes = TM * 16 * 3 * 64 * 2;  // staged z: [token][slice][64] bf16
  static_assert(kWSeg % (1024 * WAVES) == 0 && (kXSmall ? kXSeg == 1024 : kXSeg % (1024 * WAVES) == 0),
                "copy split");
  static_assert(kDmaSeg * NSEG < 64, "vmcnt range");
};

// ---------------------------------------------------------------------------
// Small helpers.
// ---------------------------------------------------------------------------
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

// Read-only metadata through the scalar path (wave-uniform index): these loads
// count on lgkmcnt, so they neither wait for nor delay the weight copies.
template <class T>
__device__ __forceinline__ T sload(const T* base, int idx) {
  typedef const __attribute__((address_space(4))) T* ConstPtr;
  return ((ConstPtr)base)[idx];
}

// s_waitcnt vmcnt(N) lgkmcnt(0).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}

// Workgroup barrier without the memory fence of __syncthreads (that fence
// would wait for every outstanding LDS copy). The clobber keeps the compiler
// from moving memory accesses across it; callers wait for their own LDS
// writes / copies first.
__device__ __forceinline__ void barrier_only() { asm volatile("s_barrier" ::: "memory"); }

__device__ __forceinline__ void lds_sync() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  barrier_only();
}

// Distinct LDS object per (ID, size): the compiler tracks outstanding direct
// copies per object, so reading segment s waits only for segment s.
template <int ID, int BYTES>
__device__ __forceinline__ char* lds_region() {
  __shared__ __attribute__((aligned(16))) char buf[BYTES];
  return buf;
}

__device__ __forceinline__ void copy16(const void* src, char* lds) {
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
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
// Prologue data. Anything the pipelined contraction uses must arrive through
// scalar loads or LDS copies: a vector-load result consumed while copies are
// in flight makes the compiler wait for every copy.
// ---------------------------------------------------------------------------
struct Codebook {
  float c[16];
};

__device__ __forceinline__ Codebook load_codebook(const float* code) {
  Codebook cb;
#pragma unroll
  for (int i = 0; i < 16; ++i) cb.c[i] = sload(code, i);
  return cb;
}

// fp32 codebook (lane 0 writes the 16 scalar values with constant indices),
// then the pair table: entry e (a packed byte) -> bf16(code[e >> 4]) |
// bf16(code[e & 15]) << 16, kCopies copies with copy c at dword e * kCopies + c
// so that lane l always reads bank l % kCopies.
template <bool kExact, int kCopies>
__device__ __forceinline__ void stage_tables(const Codebook& cb, float* table, uint32_t* pt) {
  if (threadIdx.x == 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) table[i] = cb.c[i];
  }
  if constexpr (!kExact) {
    lds_sync();
    if (threadIdx.x < 256) {
      const uint32_t v = pack_bf16x2(table[threadIdx.x >> 4], table[threadIdx.x & 15]);
      uint4* dst = reinterpret_cast<uint4*>(pt + threadIdx.x * kCopies);
#pragma unroll
      for (int c = 0; c < kCopies / 4; ++c) dst[c] = make_uint4(v, v, v, v);
    }
  }
}

// Staged block scales: [row][kBlk] fp32, the 16-byte group of segment s at
// slot s ^ h(row) so that the 16 rows of a wave read 16 distinct bank quads.
template <class S>
__device__ __forceinline__ int sc_pos(int row, int blk) {
  constexpr int kGroup = 16 / S::kNSeg;
  const int h = (row / kGroup) % S::kNSeg;
  return row * S::kBlk * 4 + (((blk >> 2) ^ h) << 4) + ((blk & 3) << 2);
}

template <class S>
__device__ __forceinline__ char* sc_lds() {
  return lds_region<8, S::kRows * S::kBlk * 4>();
}

// Plain fp32 scales copied straight into the staged layout. 16-byte units
// when a row's scales are 16-byte aligned (K % 256 == 0), dwords otherwise.
// Units past K read block 0 of the row (the contraction zeroes those blocks).
template <class S>
__device__ __forceinline__ void issue_scales(const DecodeParams& p, int row0, int kbase, int wave, int lane) {
  char* sc = sc_lds<S>();
  const int nbr = p.k >> 6;
  const int blk0 = kbase >> 6;
  constexpr int kGroup = 16 / S::kNSeg;
  if ((nbr & 3) == 0) {
    constexpr int kCopiesTotal = S::kRows * S::kNSeg / 64;
    if (wave < kCopiesTotal) {
      const int f = wave * 64 + lane;
      const int row = f / S::kNSeg;
      const int part = (f % S::kNSeg) ^ ((row / kGroup) % S::kNSeg);
      const int blk = blk0 + 4 * part;
      copy16(p.src.scales + int64_t(row0 + row) * nbr + (blk < nbr ? blk : 0), sc + wave * 1024);
    }
  } else {
#pragma unroll
    for (int i = 0; i < S::kNSeg; ++i) {
      const int ci = wave * S::kNSeg + i;
      const int f = ci * 64 + lane;
      const int row = f / S::kBlk;
      const int q = f % S::kBlk;
      const int blk = blk0 + ((((q >> 2) ^ ((row / kGroup) % S::kNSeg)) << 2) | (q & 3));
      __builtin_amdgcn_global_load_lds(p.src.scales + int64_t(row0 + row) * nbr + (blk < nbr ? blk : 0),
                                       (__attribute__((address_space(3))) void*)(sc + ci * 256), 4, 0, 0);
    }
  }
}

// Double quant: code2 (1 KiB), the uint8 absmax codes of the group ([row][kBlk]
// bytes, dword copies) and the second-level scales they use (<= 256 entries
// starting at j_lo) are copied; scales are rebuilt from LDS after the first
// segment barrier. Requires K % 256 == 0 (checked on the host).
template <class S>
__device__ __forceinline__ char* dq_code2_lds() { return lds_region<9, 1024>(); }
template <class S>
__device__ __forceinline__ char* dq_codes_lds() { return lds_region<10, S::kRows * S::kBlk>(); }
template <class S>
__device__ __forceinline__ char* dq_level2_lds() { return lds_region<11, 1024>(); }

template <class S>
__device__ __forceinline__ int dq_first(const DecodeParams& p, int row0, int kbase) {
  return int((int64_t(row0) * (p.k >> 6) + (kbase >> 6)) / p.src.dq_block);
}

template <class S>
__device__ __forceinline__ void issue_dq(const DecodeParams& p, int row0, int kbase, int wave, int lane) {
  const int nbr = p.k >> 6;
  const int blk0 = kbase >> 6;
  if (wave == 0) copy16(p.src.code2 + lane * 4, dq_code2_lds<S>());
  constexpr int kCodeCopies = S::kRows * S::kNSeg / 64;  // 4 codes (one dword) per lane
  if (wave < kCodeCopies) {
    const int f = wave * 64 + lane;
    const int row = f / S::kNSeg;
    const int blk = blk0 + 4 * (f % S::kNSeg);
    __builtin_amdgcn_global_load_lds(p.src.absmax_q + int64_t(row0 + row) * nbr + (blk < nbr ? blk : 0),
                                     (__attribute__((address_space(3))) void*)(dq_codes_lds<S>() + wave * 256), 4,
                                     0, 0);
  }
  const int j0 = dq_first<S>(p, row0, kbase);
  const int nlevel = (p.n * nbr + p.src.dq_block - 1) / p.src.dq_block;
  for (int c = wave; c < 4; c += S::kWaves) {
    const int j = j0 + c * 64 + lane;
    __builtin_amdgcn_global_load_lds(p.src.absmax2 + (j < nlevel ? j : nlevel - 1),
                                     (__attribute__((address_space(3))) void*)(dq_level2_lds<S>() + c * 256), 4, 0,
                                     0);
  }
}

// scale = fl32(fl32(code2[q] * absmax2[j / dq_block]) + offset), written into
// the staged layout (blocks past K: 0).
template <class S>
__device__ __forceinline__ void rebuild_dq_scales(const DecodeParams& p, int row0, int kbase, float offset) {
  const int nbr = p.k >> 6;
  const int blk0 = kbase >> 6;
  const int j0 = dq_first<S>(p, row0, kbase);
  const float* code2 = reinterpret_cast<const float*>(dq_code2_lds<S>());
  const uint8_t* codes = reinterpret_cast<const uint8_t*>(dq_codes_lds<S>());
  const float* level2 = reinterpret_cast<const float*>(dq_level2_lds<S>());
  char* sc = sc_lds<S>();
#pragma unroll
  for (int j = 0; j < S::kNSeg; ++j) {
    const int f = j * S::kThreads + threadIdx.x;
    const int row = f / S::kBlk;
    const int b = f % S::kBlk;
    float s = 0.f;
    if (blk0 + b < nbr) {
      const int64_t id = int64_t(row0 + row) * nbr + blk0 + b;
      s = code2[codes[row * S::kBlk + b]] * level2[int(id / p.src.dq_block) - j0] + offset;
    }
    *reinterpret_cast<float*>(sc + sc_pos<S>(row, b)) = s;
  }
}

// ---------------------------------------------------------------------------
// Direct copies of one segment. W: copy gi moves rows 8gi..8gi+7, 128 bytes
// (256 k) each; LDS slot (row, s) holds 16-byte unit s ^ ((row >> 1) & 7).
// x: copy gi moves token rows 2gi, 2gi+1, 512 bytes each; slot (row, s) holds
// unit s ^ (row & 15). Rows past M repeat the last token (never stored);
// k past K reads k = 0 (its block scale is 0).
// ---------------------------------------------------------------------------
template <class S, int SEG>
__device__ __forceinline__ void issue_segment(const DecodeParams& p, int row0, int kbase, int wave, int lane) {
  char* wb = lds_region<16 + SEG, S::kWSeg>();
  char* xb = lds_region<32 + SEG, S::kXSeg>();
  const int k0 = kbase + SEG * kSegK;
#pragma unroll
  for (int i = 0; i < S::kWDma; ++i) {
    const int gi = wave * S::kWDma + i;
    const int r = gi * 8 + (lane >> 3);
    const int u = (lane & 7) ^ ((r >> 1) & 7);
    const int kk = k0 + 32 * u;
    const int koff = kk < p.k ? kk : 0;
    copy16(p.q + int64_t(row0 + r) * (p.k >> 1) + (koff >> 1), wb + gi * 1024);
  }
#pragma unroll
  for (int i = 0; i < S::kXDma; ++i) {
    const int gi = S::kXSmall ? 0 : wave * S::kXDma + i;
    const int r = gi * 2 + (lane >> 5);
    const int u = (lane & 31) ^ (r & 15);
    const int t = r < p.m ? r : p.m - 1;
    const int kk = k0 + 8 * u;
    const int koff = kk < p.k ? kk : 0;
    char* dst = xb + gi * 1024;
    if (S::kXSmall && wave != 0) dst = lds_region<48, 1024>();  // dummy copy
    copy16(p.x + int64_t(t) * p.x_stride + koff, dst);
  }
}

template <class S, int SEG>
__device__ __forceinline__ void issue_all(const DecodeParams& p, int row0, int kbase, int wave, int lane) {
  issue_segment<S, SEG>(p, row0, kbase, wave, lane);
  if constexpr (SEG + 1 < S::kNSeg) {
    __builtin_amdgcn_sched_barrier(0);  // keep the copy order: waits count copies in issue order
    issue_all<S, SEG + 1>(p, row0, kbase, wave, lane);
  }
}

// ---------------------------------------------------------------------------
// Contraction of one NF4 block (64 k) for this wave's 16 rows: two MFMA steps.
// Lane (n = l & 15, gq = l >> 4) holds W[row n][k = 64b + 16gq .. +16) (8 bytes)
// and x[token][same k]; step j covers k = 64b + 16gq + 8j .. +8.
// ---------------------------------------------------------------------------
template <int kCopies>
__device__ __forceinline__ uint4 codes_dword(uint32_t d, const uint32_t* ptl) {
  uint4 r;
  r.x = ptl[(d & 0xffu) * kCopies];
  r.y = ptl[__builtin_amdgcn_ubfe(d, 8, 8) * kCopies];
  r.z = ptl[__builtin_amdgcn_ubfe(d, 16, 8) * kCopies];
  r.w = ptl[(d >> 24) * kCopies];
  return r;
}

template <int TM, bool kExact, int kCopies>
__device__ __forceinline__ void mfma_block(uint2 q, float s, const uint4 (&xf)[TM][2], f32x4 (&acc)[TM],
                                           const float* table, const uint32_t* ptl) {
  if constexpr (kExact) {
    const uint4 w0 = decode_dword(q.x, s, table);
    const uint4 w1 = decode_dword(q.y, s, table);
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      acc[tm] = mfma16(as_bf16x8(xf[tm][0]), as_bf16x8(w0), acc[tm]);
      acc[tm] = mfma16(as_bf16x8(xf[tm][1]), as_bf16x8(w1), acc[tm]);
    }
  } else {
    const uint4 w0 = codes_dword<kCopies>(q.x, ptl);
    const uint4 w1 = codes_dword<kCopies>(q.y, ptl);
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      f32x4 b = mfma16(as_bf16x8(xf[tm][0]), as_bf16x8(w0), zero);
      b = mfma16(as_bf16x8(xf[tm][1]), as_bf16x8(w1), b);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[tm][e] = __builtin_fmaf(s, b[e], acc[tm][e]);
    }
  }
}

// nvalid: NF4 blocks of this group's K range that lie inside K (others scale 0).
template <class S, int SEG, bool kExact>
__device__ __forceinline__ void compute_segment(f32x4 (&acc)[S::kTM], const float* table, const uint32_t* ptl,
                                                int wave, int lane, int nvalid) {
  const char* wb = lds_region<16 + SEG, S::kWSeg>();
  const char* xb = lds_region<32 + SEG, S::kXSeg>();
  const int n = lane & 15;
  const int gq = lane >> 4;
  const int row = wave * 16 + n;
  const int wrow = row * 128 + ((gq & 1) << 3);
  const int sw = (row >> 1) & 7;
  // All fragment reads of the segment are issued before any decode so the
  // LDS latency is paid once per segment rather than once per block.
  const f32x4 s4 = *reinterpret_cast<const f32x4*>(sc_lds<S>() + sc_pos<S>(row, 4 * SEG));
  uint2 q[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) q[b] = *reinterpret_cast<const uint2*>(wb + wrow + (((2 * b + (gq >> 1)) ^ sw) << 4));
  uint4 xf[4][S::kTM][2];
  const int xr = n & (S::kXRows - 1);
#pragma unroll
  for (int b = 0; b < 4; ++b)
#pragma unroll
    for (int tm = 0; tm < S::kTM; ++tm)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        xf[b][tm][j] = *reinterpret_cast<const uint4*>(xb + ((tm * 16 + xr) % S::kXRows) * 512 +
                                                       (((8 * b + 2 * gq + j) ^ xr) << 4));
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const float s = 4 * SEG + b < nvalid ? s4[b] : 0.f;
    mfma_block<S::kTM, kExact, S::kCopies>(q[b], s, xf[b], acc, table, ptl);
  }
}

struct LoraShared;
template <class S>
__device__ void lora_prologue(const DecodeParams& p, LoraShared* ls, int wave, int lane);

// After segment 0 the LoRA metadata is gathered (its slot copy was issued
// first, so the segment-0 wait covers it); later segments keep arriving.
template <class S, int SEG, bool kDouble, bool kLora, bool kExact>
__device__ __forceinline__ void run_segments(const DecodeParams& p, f32x4 (&acc)[S::kTM], const float* table,
                                             const uint32_t* ptl, int wave, int lane, int row0, int kbase,
                                             float offset, LoraShared* ls) {
  wait_vm_lgkm<(S::kNSeg - 1 - SEG) * S::kDmaSeg>();  // this wave's copies up to segment SEG landed
  barrier_only();                                      // ... and every other wave's
  if constexpr (SEG == 0 && kDouble) {
    rebuild_dq_scales<S>(p, row0, kbase, offset);
    lds_sync();
  }
  compute_segment<S, SEG, kExact>(acc, table, ptl, wave, lane, (p.k >> 6) - (kbase >> 6));
  if constexpr (SEG == 0 && kLora) lora_prologue<S>(p, ls, wave, lane);
  if constexpr (SEG + 1 < S::kNSeg)
    run_segments<S, SEG + 1, kDouble, kLora, kExact>(p, acc, table, ptl, wave, lane, row0, kbase, offset, ls);
}

// ---------------------------------------------------------------------------
// LoRA metadata gathered per group: the batch's distinct slots (in order of
// first use), their rank / offsets / stride / scale, and tokens grouped by
// distinct slot.
// ---------------------------------------------------------------------------
struct LoraShared {
  int tok_d[64];    // token -> distinct index (-1: none)
  int dslot[64];    // distinct index -> slot id
  int drank[64];    // 0: base only (rank 0 or above max_rank)
  int dstride[64];
  float dscale[64];
  int64_t daoff[64];
  int64_t dboff[64];
  int dtok[64];      // tokens grouped by distinct index
  int dptr[65];      // CSR offsets into dtok
  int bounds[4];     // slice boundaries over the output width
  int nd;
  int flag;
};

// Token slot ids, copied to LDS before any other copy of wave 0 (entries past
// M repeat the last token and are ignored).
__device__ __forceinline__ int* slot_lds() { return reinterpret_cast<int*>(lds_region<12, 256>()); }

__device__ __forceinline__ void issue_slots(const DecodeParams& p, int wave, int lane) {
  if (wave == 0)
    __builtin_amdgcn_global_load_lds(p.token_slots + (lane < p.m ? lane : p.m - 1),
                                     (__attribute__((address_space(3))) void*)slot_lds(), 4, 0, 0);
}

template <class S>
__device__ void lora_prologue(const DecodeParams& p, LoraShared* ls, int wave, int lane) {
  if (wave == 0) {
    // Distinct slots in order of first use and their tokens (CSR): one
    // ballot per distinct slot, all in registers.
    const int g = lane < p.m ? slot_lds()[lane] : -1;  // the slot copy is covered by the segment-0 wait
    uint64_t left = __ballot(g >= 0);
    int nd = 0, base = 0, my_d = -1;
    while (left) {
      const int f = __builtin_ctzll(left);
      const int gf = __builtin_amdgcn_readlane(g, f);
      const uint64_t same = __ballot(g == gf) & left;
      if (g == gf) {
        ls->dtok[base + __popcll(same & ((uint64_t(1) << lane) - 1))] = lane;
        my_d = nd;
      }
      if (lane == 0) {
        ls->dslot[nd] = gf;
        ls->dptr[nd] = base;
      }
      base += __popcll(same);
      ++nd;
      left &= ~same;
    }
    ls->tok_d[lane] = my_d;
    if (lane == 0) {
      ls->nd = nd;
      ls->dptr[nd] = base;
    }
  }
  if (wave == 1 % S::kWaves) {  // uniform scalar loads: no vector load may queue behind the copies here
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = i <= p.slices ? sload(p.slice_offsets, i) : 0;
      if (lane == 0) ls->bounds[i] = v;
    }
  }
  lds_sync();
  // Slot metadata through scalar loads, four slots per wave in flight.
  const int nd = ls->nd;
  constexpr int kBatch = 4;
  for (int d0 = wave; d0 < nd; d0 += kBatch * S::kWaves) {
    int r[kBatch], stride[kBatch];
    float scale[kBatch];
    int64_t aoff[kBatch], boff[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int d = min(d0 + i * S::kWaves, nd - 1);
      const int g = __builtin_amdgcn_readfirstlane(ls->dslot[d]);
      r[i] = sload(p.ranks, g);
      stride[i] = sload(p.b_strides, g);
      scale[i] = sload(p.lscales, g);
      aoff[i] = sload(p.a_offsets, g);
      boff[i] = sload(p.b_offsets, g);
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int d = d0 + i * S::kWaves;
      if (lane == 0 && d < nd) {
        ls->drank[d] = (r[i] > 0 && r[i] <= p.max_rank) ? r[i] : 0;  // metadata contract: rank <= max_rank
        ls->dstride[d] = stride[i];
        ls->dscale[d] = scale[i];
        ls->daoff[d] = aoff[i];
        ls->dboff[d] = boff[i];
      }
    }
  }
  lds_sync();
}

// Shrink units owned by this group: unit u = (distinct d = u / kz, k-slice u % kz).
// z partial [tokens of slot g][rows s*r + j of A_g] over the slice on MFMA:
// x rows of the slot's tokens as the A operand, A_g rows as the B operand,
// 16 x 16 tiles; the waves split the slice's 32-k steps (8 steps of loads in
// flight per wave) and their tiles are summed through LDS. A finished unit
// bumps its slot's z-ready counter (the owners of that slot wait for kz).
template <class S>
__device__ void shrink_units(const DecodeParams& p, const LoraShared* ls, int wave, int lane, float* red) {
  const int units = ls->nd * p.kz;
  const int kg = lane >> 4;
  for (int u = blockIdx.x; u < units; u += gridDim.x) {
    const int d = u / p.kz;
    const int ks = u - d * p.kz;
    const int r = ls->drank[d];
    if (r == 0) continue;
    const int rows = p.slices * r;
    const int kb = ks * p.kz_len;
    const int ke = min(p.k, kb + p.kz_len);
    const int nsteps = (ke - kb) >> 5;
    const int t0 = ls->dptr[d], t1 = ls->dptr[d + 1];
    const uint16_t* abase = p.a_store + ls->daoff[d];
    for (int tt0 = t0; tt0 < t1; tt0 += 16) {
      const int ti = tt0 + (lane & 15);
      const int tok = ls->dtok[ti < t1 ? ti : t0];  // padded rows repeat a token; never stored
      const uint16_t* xrow = p.x + int64_t(tok) * p.x_stride + kb + 8 * kg;
      for (int j0 = 0; j0 < rows; j0 += 16) {
        const int jr = j0 + (lane & 15) < rows ? j0 + (lane & 15) : j0;
        const uint16_t* arow = abase + int64_t(jr) * p.k + kb + 8 * kg;
        f32x4 c = {0.f, 0.f, 0.f, 0.f};
        for (int st0 = wave; st0 < nsteps; st0 += 8 * S::kWaves) {
          uint4 xa[8], aa[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int st = st0 + i * S::kWaves;
            const bool ok = st < nsteps;
            xa[i] = ok ? *reinterpret_cast<const uint4*>(xrow + 32 * st) : make_uint4(0, 0, 0, 0);
            aa[i] = ok ? *reinterpret_cast<const uint4*>(arow + 32 * st) : make_uint4(0, 0, 0, 0);
          }
#pragma unroll
          for (int i = 0; i < 8; ++i) c = mfma16(as_bf16x8(xa[i]), as_bf16x8(aa[i]), c);
        }
        *reinterpret_cast<f32x4*>(red + (wave * 64 + lane) * 4) = c;
        __syncthreads();
        if (wave == 0) {
          f32x4 sum = c;
          for (int w = 1; w < S::kWaves; ++w) {
            const f32x4 o = *reinterpret_cast<const f32x4*>(red + (w * 64 + lane) * 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) sum[e] += o[e];
          }
          const int j = j0 + (lane & 15);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int tj = tt0 + 4 * kg + e;
            if (tj < t1 && j < rows)
              shared_store(p.zpart + (int64_t(ks) * p.m + ls->dtok[tj]) * p.zw + j, sum[e]);
          }
        }
        __syncthreads();  // this tile's z partials stored
      }
    }
    if (threadIdx.x == 0) counter_add(p.ctrl + kSlotDone + d, 1);
  }
}

// Bounded wait (thread 0) until the z-ready counter of every owned slot
// (d = split, split + splits, ...) reaches kz. Each poll issues all counter
// loads together, so one device-coherent round trip checks every slot; a
// timeout records a status instead of hanging the launch.
__device__ void wait_owned_slots(const DecodeParams& p, const LoraShared* ls, int split) {
  if (threadIdx.x == 0) {
    int spins = 0;
    for (;;) {
      bool done = true;
      for (int d = split; d < ls->nd; d += p.splits)
        if (ls->drank[d] > 0 && counter_load(p.ctrl + kSlotDone + d) < p.kz) done = false;
      if (done) break;
      __builtin_amdgcn_s_sleep(4);
      if (++spins > kSpinLimit) {
        counter_store(p.ctrl + kStatus, 1);
        break;
      }
    }
  }
  __syncthreads();
}

// B fragment of slot row nn (ranks j0 .. j0+8), zero past the rank.
__device__ __forceinline__ uint4 load_b_frag(const DecodeParams& p, int64_t boff, int stride, int r, int nn, int j0) {
  const uint16_t* bp = p.b_store + boff + int64_t(nn) * stride + j0;
  if (((boff | int64_t(stride)) & 7) == 0 && j0 + 8 <= r) return *reinterpret_cast<const uint4*>(bp);
  uint32_t e[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) e[i] = j0 + i < r ? bp[i] : 0u;
  return make_uint4(e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16));
}

// Expand for the distinct slots owned by this split (d = split mod splits):
// dacc[tm] = per-token fp32 sum_j z[t][s*r + j] * B_g[n][j] for owned tokens.
// B fragments of this split's first 8 owned slots for slice 0, ranks 0..31
// (the whole expand for single-slice adapters of rank <= 32 and <= 8 owned
// slots), requested early like the shrink operands.
struct ExpandPre {
  uint4 bf[8];
};

__device__ __forceinline__ bool slice_hits_tile(const LoraShared* ls, int s, int tile_lo) {
  return !(tile_lo + 15 < ls->bounds[s] || tile_lo >= ls->bounds[s + 1]);
}

__device__ __forceinline__ void expand_frags(const DecodeParams& p, const LoraShared* ls, int d0, int s, int h,
                                             int nn, int kg, uint4 (&bf)[8], int (&dd)[8]) {
  const bool in = nn >= ls->bounds[s] && nn < ls->bounds[s + 1];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int d = d0 + i * p.splits;
    const int r = d < ls->nd ? ls->drank[d] : 0;
    const int j0 = 32 * h + 8 * kg;
    dd[i] = r > 32 * h ? d : -1;
    bf[i] = dd[i] >= 0 && in && j0 < r ? load_b_frag(p, ls->dboff[d], ls->dstride[d], r, nn, j0)
                                       : make_uint4(0, 0, 0, 0);
  }
}

template <class S>
__device__ void lora_expand(const DecodeParams& p, const LoraShared* ls, int split, int row0, int wave, int lane,
                            uint16_t* zl, f32x4 (&dacc)[S::kTM], const ExpandPre& pre, bool have_pre) {
  constexpr int TM = S::kTM;
  const int nd = ls->nd;
  // Stage z = bf16(sum of k-slice partials), [token][slice][64] zero-padded.
  const int total = TM * 16 * p.slices * 64;
  for (int i = threadIdx.x; i < total; i += S::kThreads) {
    const int t = i / (p.slices * 64);
    const int rem = i - t * p.slices * 64;
    const int s = rem >> 6;
    const int j = rem & 63;
    const int d = t < p.m ? ls->tok_d[t] : -1;
    const int r = d >= 0 && d % p.splits == split ? ls->drank[d] : 0;  // owned tokens only
    uint32_t bits = 0;
    if (j < r) {
      const float* zp = p.zpart + int64_t(t) * p.zw + s * r + j;
      const int64_t step = int64_t(p.m) * p.zw;
      float z = 0.f;
      for (int ks0 = 0; ks0 < p.kz; ks0 += 4) {
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = ks0 + q < p.kz ? shared_load(zp + (ks0 + q) * step) : 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) z += v[q];
      }
      bits = f32_to_bf16(z);
    }
    zl[i] = uint16_t(bits);
  }
  __syncthreads();
  const int nn = row0 + wave * 16 + (lane & 15);
  const int kg = lane >> 4;
  const int tile_lo = row0 + wave * 16;
  for (int d0 = split; d0 < nd; d0 += 8 * p.splits) {
    for (int s = 0; s < p.slices; ++s) {
      if (!slice_hits_tile(ls, s, tile_lo)) continue;
      for (int h = 0; h < 2; ++h) {
        uint4 bf[8];
        int dd[8];
        if (have_pre && d0 == split && s == 0 && h == 0) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int d = d0 + i * p.splits;
            dd[i] = d < nd && ls->drank[d] > 0 ? d : -1;
            bf[i] = pre.bf[i];
          }
        } else {
          expand_frags(p, ls, d0, s, h, nn, kg, bf, dd);
        }
        bool any = false;
#pragma unroll
        for (int i = 0; i < 8; ++i) any |= dd[i] >= 0;
        if (!any) break;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if (dd[i] < 0) continue;
#pragma unroll
          for (int tm = 0; tm < TM; ++tm) {
            const int tok = tm * 16 + (lane & 15);
            const bool mine = tok < p.m && ls->tok_d[tok] == dd[i];
            const uint4 av = mine ? *reinterpret_cast<const uint4*>(zl + (tok * p.slices + s) * 64 + 32 * h + 8 * kg)
                                  : make_uint4(0, 0, 0, 0);
            dacc[tm] = mfma16(as_bf16x8(av), as_bf16x8(bf[i]), dacc[tm]);
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// The kernel.
// ---------------------------------------------------------------------------
template <int WAVES, int TM, int NSEG, int XR, bool kDouble, bool kLora, bool kExact>
__global__ __launch_bounds__(WAVES * 64) void nf4_lora_decode_kernel(DecodeParams p) {
  using S = Shape<WAVES, TM, NSEG, XR>;
  __shared__ float table[16];
  __shared__ __attribute__((aligned(16))) uint32_t pt[kExact ? 4 : 256 * S::kCopies];
  __shared__ LoraShared lshared[1];
  __shared__ int flag[1];
  LoraShared* ls = lshared;

  const int grp = blockIdx.x / p.splits;
  const int split = blockIdx.x - grp * p.splits;
  const int row0 = grp * S::kRows;
  const int kbase = split * p.krange;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int n = lane & 15;
  const int gq = lane >> 4;

  // Scalar loads and LDS copies only (see the prologue notes above), slots
  // first, then scales, then every W / x segment.
  const Codebook cb = load_codebook(p.code);
  const float offset = kDouble ? sload(p.src.offset, 0) : 0.f;
  if constexpr (kLora) issue_slots(p, wave, lane);
  if constexpr (kDouble) issue_dq<S>(p, row0, kbase, wave, lane);
  else issue_scales<S>(p, row0, kbase, wave, lane);
  __builtin_amdgcn_sched_barrier(0);
  issue_all<S, 0>(p, row0, kbase, wave, lane);

  stage_tables<kExact, S::kCopies>(cb, table, pt);

  f32x4 acc[TM];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) acc[tm] = (f32x4){0.f, 0.f, 0.f, 0.f};
  const uint32_t* ptl = pt + (lane % S::kCopies);
  run_segments<S, 0, kDouble, kLora, kExact>(p, acc, table, ptl, wave, lane, row0, kbase, offset, ls);
  __syncthreads();  // every copy consumed: LDS buffers may be reused

  f32x4 dacc[TM];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) dacc[tm] = (f32x4){0.f, 0.f, 0.f, 0.f};
  if constexpr (kLora) {
    // The W segment-0 buffer is dead here: it holds the shrink's cross-wave tiles.
    shrink_units<S>(p, ls, wave, lane, reinterpret_cast<float*>(lds_region<16, S::kWSeg>()));
    bool owns = false;
    for (int d = split; d < ls->nd; d += p.splits) owns |= ls->drank[d] > 0;
    if (owns) {
      // B fragments of the first owned batch are requested before the z wait.
      ExpandPre ep;
      const bool have_expand = slice_hits_tile(ls, 0, row0 + wave * 16);
      if (have_expand) {
        int dd[8];
        expand_frags(p, ls, split, 0, 0, row0 + wave * 16 + (lane & 15), lane >> 4, ep.bf, dd);
      }
      wait_owned_slots(p, ls, split);
      // z is staged in a dead segment buffer (x of segment 0, or W of segment 0 when x is small).
      char* zl_bytes;
      if constexpr (S::kXSeg >= S::kZlBytes) zl_bytes = lds_region<32, S::kXSeg>();
      else zl_bytes = lds_region<16, S::kWSeg>();
      static_assert(S::kXSeg >= S::kZlBytes || S::kWSeg >= S::kZlBytes, "z staging space");
      lora_expand<S>(p, ls, split, row0, wave, lane, reinterpret_cast<uint16_t*>(zl_bytes), dacc, ep, have_expand);
    }
  }

  const int col = row0 + wave * 16 + n;
  bool finish = true;
  if (p.splits > 1) {
    float* mine = p.part + int64_t(blockIdx.x) * p.m * S::kRows;
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = tm * 16 + 4 * gq + e;
        if (t < p.m) {
          shared_store(mine + t * S::kRows + wave * 16 + n, acc[tm][e]);
          if constexpr (kLora) {
            const int d = ls->tok_d[t];
            if (d >= 0 && d % p.splits == split) shared_store(p.dpart + int64_t(t) * p.n + col, dacc[tm][e]);
          }
        }
      }
    __syncthreads();  // partial stores complete
    if (threadIdx.x == 0) {
      const int prev = counter_add(p.tile_count + grp, 1);
      const bool last = prev == p.splits - 1;
      if (last) counter_store(p.tile_count + grp, 0);
      flag[0] = last;
    }
    __syncthreads();
    finish = flag[0] != 0;
    if (finish) {
      // Sum the split partials in split order; each batch of 4 splits has all
      // of its loads in flight before the first add.
      const float* parts = p.part + int64_t(grp) * p.splits * p.m * S::kRows + wave * 16 + n;
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) acc[tm] = (f32x4){0.f, 0.f, 0.f, 0.f};
      for (int sp0 = 0; sp0 < p.splits; sp0 += 4) {
        float v[4][TM][4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int t = tm * 16 + 4 * gq + e;
              const int sp = sp0 + i;
              v[i][tm][e] = t < p.m && sp < p.splits
                                ? shared_load(parts + (int64_t(sp) * p.m + t) * S::kRows)
                                : 0.f;
            }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int tm = 0; tm < TM; ++tm)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[tm][e] += v[i][tm][e];
      }
      if constexpr (kLora) {
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int t = tm * 16 + 4 * gq + e;
            if (t < p.m && ls->tok_d[t] >= 0) dacc[tm][e] = shared_load(p.dpart + int64_t(t) * p.n + col);
          }
      }
    }
  }
  if (finish) {
    const float bias = p.bias ? bf16_to_f32(p.bias[col]) : 0.f;
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = tm * 16 + 4 * gq + e;
        if (t < p.m) {
          float v = round_bf16(acc[tm][e]);
          if (p.bias) v = round_bf16(v + bias);
          if constexpr (kLora) {
            const int d = ls->tok_d[t];
            if (d >= 0 && ls->drank[d] > 0) v = round_bf16(v + round_bf16(dacc[tm][e] * ls->dscale[d]));
          }
          p.y[int64_t(t) * p.y_stride + col] = uint16_t(f32_to_bf16(v));
        }
      }
  }
  if constexpr (kLora) {
    if (threadIdx.x == 0) {
      const int done = counter_add(p.ctrl + kDone, 1);
      if (done == int(gridDim.x) - 1) {  // every group is past its z waits: reset for the next call
        for (int d = 0; d < ls->nd; ++d) counter_store(p.ctrl + kSlotDone + d, 0);
        counter_store(p.ctrl + kDone, 0);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
struct Plan {
  int tm;
  int waves;
  int nseg;
  int rows;
  int krange;
  int splits;
  int groups;
  int kz;
  int kz_len;
};

Plan make_plan(int64_t m, int64_t n, int64_t k) {
  Plan pl;
  pl.tm = int((m + 15) / 16);
  if (pl.tm <= 2) {
    pl.waves = 4;
    pl.nseg = 4;
  } else {
    pl.waves = n % 128 == 0 ? 8 : 4;
    pl.nseg = 2;
  }
  pl.rows = 16 * pl.waves;
  pl.krange = kSegK * pl.nseg;
  pl.splits = int((k + pl.krange - 1) / pl.krange);
  pl.groups = int(n / pl.rows) * pl.splits;
  // Shrink units (distinct slots <= m, times k-slices) stay <= min(groups, 256)
  // so every producer is among the first groups dispatched.
  const int64_t cap = std::min<int64_t>(pl.groups, kMaxUnits);
  const int64_t kchunks = (k + kShrinkK - 1) / kShrinkK;
  int64_t kz = std::max<int64_t>(1, std::min<int64_t>(kchunks, cap / std::max<int64_t>(m, 1)));
  pl.kz_len = int((kchunks + kz - 1) / kz) * kShrinkK;
  pl.kz = int((k + pl.kz_len - 1) / pl.kz_len);
  return pl;
}

int64_t align256(int64_t v) { return (v + 255) / 256 * 256; }

struct Layout {
  int64_t tile_count;
  int64_t zpart;
  int64_t dpart;
  int64_t part;
  int64_t total;
};

Layout workspace_layout(int64_t m, int64_t n, int64_t k, int slices, int max_rank) {
  const Plan pl = make_plan(m, n, k);
  Layout l;
  l.tile_count = kCtrlBytes;  // one counter per column group, inside the control header
  l.zpart = kWorkspaceHeader;
  l.dpart = align256(l.zpart + 4 * int64_t(pl.kz) * m * slices * max_rank);
  const int64_t split_bytes = pl.splits > 1 ? 4 * m * n : 0;
  l.part = align256(l.dpart + split_bytes);
  l.total = align256(l.part + split_bytes * pl.splits);
  return l;
}

template <int W, int TM, int NS, int XR, bool D, bool E>
void launch_lora_variant(bool lora, dim3 grid, hipStream_t s, const DecodeParams& p) {
  if (lora) {
    hipLaunchKernelGGL((nf4_lora_decode_kernel<W, TM, NS, XR, D, true, E>), grid, dim3(W * 64), 0, s, p);
  } else {
    hipLaunchKernelGGL((nf4_lora_decode_kernel<W, TM, NS, XR, D, false, E>), grid, dim3(W * 64), 0, s, p);
  }
}

template <int W, int TM, int NS, int XR = 16 * TM>
void launch_variant(bool dq, bool lora, bool exact, dim3 grid, hipStream_t s, const DecodeParams& p) {
  if (exact) {
    if (dq) launch_lora_variant<W, TM, NS, XR, true, true>(lora, grid, s, p);
    else launch_lora_variant<W, TM, NS, XR, false, true>(lora, grid, s, p);
  } else {
    if (dq) launch_lora_variant<W, TM, NS, XR, true, false>(lora, grid, s, p);
    else launch_lora_variant<W, TM, NS, XR, false, false>(lora, grid, s, p);
  }
}

}  // namespace

int64_t decode_workspace_bytes(int64_t m, int64_t n, int64_t k, int slices, int max_rank) {
  return workspace_layout(m, n, k, slices, max_rank).total;
}

int launch_nf4_lora_decode(const uint16_t* x, int64_t m, int64_t x_stride, const lf_nf4_weight* w,
                           const uint16_t* bias, const lf_lora* lora, uint16_t* y, int64_t y_stride,
                           void* workspace, int64_t workspace_bytes, bool exact, void* stream) {
  const int64_t n = w->n, k = w->k;
  const int slices = lora ? lora->num_slices : 1;
  const int max_rank = lora ? lora->max_rank : 1;
  LF_REQUIRE(m >= 1 && m <= 64, "decode path handles 1..64 tokens");
  const Layout lay = workspace_layout(m, n, k, slices, max_rank);
  LF_REQUIRE(workspace && workspace_bytes >= lay.total, "workspace too small: need %lld bytes",
             (long long)lay.total);
  LF_REQUIRE(aligned16(workspace), "workspace must be 16-byte aligned");
  const Plan pl = make_plan(m, n, k);
  LF_REQUIRE(n % pl.rows == 0, "output width must be a multiple of %d", pl.rows);
  LF_REQUIRE(kCtrlBytes + 4 * (n / pl.rows) <= kWorkspaceHeader, "output width too large for the decode path");
  if (!w->scales) {
    // In-kernel double-quant staging covers groups whose second-level scales
    // fit a 256-entry window; other shapes take prepared fp32 scales.
    const int64_t span = ((pl.rows - 1) * (k / 64) + pl.krange / 64) / w->dq_block + 2;
    LF_REQUIRE(k % 256 == 0 && span <= 256,
               "double-quant decode needs K %% 256 == 0 and dq_block >= %lld; pass prepared scales",
               (long long)(((pl.rows - 1) * (k / 64) + pl.krange / 64) / 254 + 1));
  }
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
  p.splits = pl.splits;
  p.krange = pl.krange;
  p.kz = pl.kz;
  p.kz_len = pl.kz_len;
  char* ws = static_cast<char*>(workspace);
  p.ctrl = reinterpret_cast<int*>(ws);
  p.tile_count = reinterpret_cast<int*>(ws + lay.tile_count);
  p.zpart = reinterpret_cast<float*>(ws + lay.zpart);
  p.dpart = reinterpret_cast<float*>(ws + lay.dpart);
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
  }
  const dim3 grid(unsigned(pl.groups));
  auto s = static_cast<hipStream_t>(stream);
  const bool dq = w->scales == nullptr;
  const bool has_lora = lora != nullptr;
  switch (pl.tm * 100 + pl.waves * 10 + pl.nseg) {
    case 144:
      if (m <= 2) launch_variant<4, 1, 4, 2>(dq, has_lora, exact, grid, s, p);
      else launch_variant<4, 1, 4>(dq, has_lora, exact, grid, s, p);
      break;
    case 244: launch_variant<4, 2, 4>(dq, has_lora, exact, grid, s, p); break;
    case 342: launch_variant<4, 3, 2>(dq, has_lora, exact, grid, s, p); break;
    case 382: launch_variant<8, 3, 2>(dq, has_lora, exact, grid, s, p); break;
    case 442: launch_variant<4, 4, 2>(dq, has_lora, exact, grid, s, p); break;
    case 482: launch_variant<8, 4, 2>(dq, has_lora, exact, grid, s, p); break;
    default: return fail(kInvalid, "unsupported decode plan");
  }
  LF_HIP(hipGetLastError());
  return kOk;
}

}  // namespace lf
