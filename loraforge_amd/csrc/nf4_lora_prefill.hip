// Prefill (M > 64 tokens): NF4 GEMM on bf16 MFMA with a multi-LoRA epilogue.
//
// Reference chain (integrations/_sglang_nf4_linear.py:116-129 for the base,
// benchmarks/qwen35_prefill_fused.py:95-171 segmented_ab_kernel for the
// LoRA part):  y = bf16(x @ dequant(W)^T) (+bias);  z = bf16(A_g x);
//              y = bf16(y + bf16(scale_g * B_g z)).
//
// One launch (wide::gemm_kernel) on the caller's stream (a double-quant
// weight first gets its fp32 block scales rebuilt into the workspace):
//  - LoRA launches start with one z producer per 256-token tile: z =
//    bf16(x A_g^T) of the tile's routed tokens, on the GEMM's own LDS
//    pipeline and MFMA fragments, into a slice-padded workspace
//    zpad[m][s*64 + j] (zeros past r), then the tile's flag is set to the
//    call's tag (call_epoch.h).
//  - GEMM tiles of 256 tokens x 192 output features: x streamed by direct
//    global -> LDS copies, W decoded once per tile to the reference's exact
//    weights bf16_rne(code * scale) into LDS, contracted on
//    v_mfma_f32_16x16x32_bf16. LDS rows are 128 B with a 16-byte-unit XOR
//    swizzle (unit ^ row % 8). Epilogue: round, bias; with LoRA, wait for the
//    tile's flag (its producer has a lower block id, so it is already
//    running), stage the tile's z rows per slice in LDS and, for every
//    distinct slot in the tile, a second MFMA pass z x B_g^T over the 16-row
//    blocks holding its tokens gives the delta, applied with the reference's
//    two bf16 roundings to the rows routed to that slot.
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
  uint16_t* zpad;     // [m][slices * 64]
  int y_vec;          // 2: 16-byte aligned y rows, 1: 8-byte aligned, 0: neither
  uint32_t* zflags;   // [mtiles]: the call's tag once the tile's z rows are stored
  CallEpoch ce;
  int* status;  // set to 1 if a wait for z gives up (cannot happen while producers run first)
  int mtiles;
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

// LoRA B row segment [kk, kk + 8) of a row of length br (zeros past br).
__device__ __forceinline__ uint4 load_b8(const uint16_t* brow, int kk, int br) {
  if (kk + 8 <= br) return *reinterpret_cast<const uint4*>(brow + kk);
  uint32_t h[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) h[e] = kk + e < br ? brow[kk + e] : 0u;
  return make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
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

// z producer of M-tile mt (the launch's workgroups below mtiles): z rows
// bf16(x A_g^T) of every token of the tile routed to a live slot, in the
// slice-padded layout zpad[t][s * 64 + j] (zeros for j >= r), then the tile's
// flag is set to the call's tag. The columns of a pass are up to kBN rows of
// the distinct slots' A factors ([slices * r, K] each, concatenated); a pass
// streams the x tile and those rows through the GEMM's LDS layout (direct
// copies, two-step x ring, one-step A slots) and contracts them on the same
// MFMA fragments; each output is kept for the rows routed to its slot.
__device__ __forceinline__ void produce_z(const PrefillParams& p, int mt, uint32_t tag, char* xring, uint4* wdec,
                                          int* tslot, int* list, int* colmap, int* cum) {
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int wm = wave & 1;
  const int wn = wave >> 1;
  const int c = lane & 15;
  const int g = lane >> 4;
  const int m0 = mt * kBM;
  const int count = min(kBM, p.m - m0);
  const int nk = p.k / kBK;
  const int zw = p.slices * kZSlice;
  live_slots(p, m0, count, tslot, list);
  const int nd = list[kMaxList];
  // Column offsets of the distinct slots (cum[d] .. cum[d + 1]).
  if (tid == 0) {
    int acc = 0;
    for (int d = 0; d < nd; ++d) {
      cum[d] = acc;
      acc += p.slices * p.ranks[list[d]];
    }
    cum[nd] = acc;
  }
  // Zero columns r .. 64 of every slice of the live tokens.
  for (int i = tid; i < count * zw; i += kThreads) {
    const int t = i / zw;
    const int col = i - t * zw;
    const int gt = tslot[t];
    if (gt >= 0 && (col % kZSlice) >= p.ranks[gt]) p.zpad[int64_t(m0 + t) * zw + col] = 0;
  }
  __syncthreads();
  const int ncols = cum[nd];
  const uint32_t xa0 = lds_addr(xring) + uint32_t((wm * 128 + c) * 128 + ((g ^ (c & 7)) << 4));
  const uint32_t xa1 = lds_addr(xring) + uint32_t((wm * 128 + c) * 128 + (((4 + g) ^ (c & 7)) << 4));
  const uint32_t wa0 = lds_addr(wdec) + uint32_t((wn * 48 + c) * 128 + ((g ^ (c & 7)) << 4));
  const uint32_t wa1 = lds_addr(wdec) + uint32_t((wn * 48 + c) * 128 + (((4 + g) ^ (c & 7)) << 4));
  for (int c0 = 0; c0 < ncols; c0 += kBN) {
    // colmap[col] = (distinct slot << 16) | (slice << 8) | row within the slice, or -1.
    if (tid < kBN) {
      const int col = c0 + tid;
      int e = -1;
      if (col < ncols) {
        int d = 0;
        while (cum[d + 1] <= col) ++d;
        const int rho = col - cum[d];
        const int r = p.ranks[list[d]];
        e = (d << 16) | ((rho / r) << 8) | (rho % r);
      }
      colmap[tid] = e;
    }
    __syncthreads();
    // This lane's three A-row copies per step: position P = (wave * 3 + q) * 64
    // + lane -> row P / 8, slot P % 8 holding unit (P % 8) ^ (row & 7).
    const uint16_t* asrc[3];
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const int pos = (wave * 3 + q) * 64 + lane;
      const int row = pos >> 3;
      const int u = (pos & 7) ^ (row & 7);
      const int e = colmap[row];
      const int d = e < 0 ? 0 : e >> 16;
      const int rho = e < 0 ? 0 : (((e >> 8) & 0xff) * p.ranks[list[d]] + (e & 0xff));
      asrc[q] = p.a_store + p.a_offsets[list[d]] + int64_t(rho) * p.k + u * 8;
    }
    auto issue_a = [&](int kt, int slot) {
#pragma unroll
      for (int q = 0; q < 3; ++q)
        copy16(asrc[q] + kt * kBK, reinterpret_cast<char*>(wdec) + slot * kWBytes + (wave * 3 + q) * 1024);
    };
    const bool busy = wn * 48 < ncols - c0;  // the wave's columns hold A rows
    f32x4 acc[8][kJ];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < kJ; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
    issue_x(p, xring, m0, 0, wave, lane);
    issue_x(p, xring + kXBytes, m0, min(1, nk - 1), wave, lane);
    issue_a(0, 0);
    wait_vm<0>();
    lds_barrier();
    for (int kt = 0; kt < nk; ++kt) {
      // Requests: A(kt + 1), then x(kt + 2) (past the end: the last step again).
      issue_a(min(kt + 1, nk - 1), (kt + 1) & 1);
      issue_x(p, xring + ((kt + 2) % kXD) * kXBytes, m0, min(kt + 2, nk - 1), wave, lane);
      if (busy) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t ax = (h ? xa1 : xa0) + uint32_t((kt % kXD) * kXBytes);
          const uint32_t bx = (h ? wa1 : wa0) + uint32_t((kt & 1) * kWBytes);
          u32x4 a[8], b[kJ];
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
          wait_lgkm<0>();
#pragma unroll
          for (int i = 0; i < 8; ++i) tie(a[i]);
#pragma unroll
          for (int j = 0; j < kJ; ++j) tie(b[j]);
#pragma unroll
          for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < kJ; ++j) acc[i][j] = mfma16(vec_bf16x8(a[i]), vec_bf16x8(b[j]), acc[i][j]);
        }
      }
      // A(kt + 1) and x(kt + 1) have landed once at most x(kt + 2) is outstanding.
      wait_vm<kXCopies>();
      lds_barrier();
    }
    wait_vm<0>();  // the requests past the end
    // acc[i][j][e] = z[token m0 + wm*128 + 16i + 4g + e][pass column wn*48 + 16j + c]
    if (busy) {
#pragma unroll
      for (int j = 0; j < kJ; ++j) {
        const int e = colmap[wn * 48 + j * 16 + c];
        if (e < 0) continue;
        const int gd = list[e >> 16];
        const int zc = ((e >> 8) & 0xff) * kZSlice + (e & 0xff);
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = wm * 128 + i * 16 + 4 * g + r;
            if (row < count && tslot[row] == gd)
              p.zpad[int64_t(m0 + row) * zw + zc] = uint16_t(f32_to_bf16(acc[i][j][r]));
          }
      }
    }
    __syncthreads();  // colmap and the LDS slots are reused by the next pass
  }
  // Publish: every thread's z stores are performed at device scope before the
  // flag carries the call's tag.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  if (tid == 0) __hip_atomic_store(p.zflags + mt, tag, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}

// Waits until the z rows of M-tile mt carry the call's tag (their producer
// has a lower block id, so it has been dispatched before this workgroup).
// The flag and the z rows are read with device-scope loads (coherent past
// the caches of this CU and XCD), so no acquire fence is needed: an acquire
// at device scope would invalidate the whole L2 of the XCD under the other
// workgroups' feet.
__device__ __forceinline__ void wait_z(const PrefillParams& p, int mt, uint32_t tag) {
  if (threadIdx.x == 0) {
    // Bounded (about a quarter second): a workgroup never waits forever,
    // whatever the launch order; giving up is reported in the status word.
    for (int spins = 0; __hip_atomic_load(p.zflags + mt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != tag; ++spins) {
      if (spins > (1 << 20)) {
        __hip_atomic_store(p.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(8);
    }
  }
  __syncthreads();
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

// Block ids below mtiles (LoRA launches only) produce the tiles' z rows;
// the others are GEMM tiles, M-tile b % mtiles on consecutive ids.
template <bool kLora>
__global__ __launch_bounds__(kThreads) void gemm_kernel(PrefillParams p) {
  __shared__ __attribute__((aligned(16))) char xring[kXD * kXBytes];
  __shared__ __attribute__((aligned(16))) uint4 wdec[2][kBN * 8];
  __shared__ __attribute__((aligned(2048))) float table[512];  // [byte] -> (code[byte >> 4], code[byte & 15])
  __shared__ __attribute__((aligned(16))) int tslot[kLora ? kBM : 1];
  __shared__ int list[kLora ? kMaxList + 1 : 1];
  __shared__ int cum[kLora ? kMaxList + 1 : 1];
  __shared__ int colmap[kLora ? kBN : 1];
  __shared__ int mrank[kLora ? kMaxList : 1];
  __shared__ int mstride[kLora ? kMaxList : 1];
  __shared__ float mscale[kLora ? kMaxList : 1];
  __shared__ int64_t mboff[kLora ? kMaxList : 1];
  const int tid = threadIdx.x;
  int b = blockIdx.x;
  uint32_t tag = 0;
  if constexpr (kLora) {
    tag = __builtin_amdgcn_readfirstlane(epoch_tag(p.ce));
    if (b < p.mtiles) {
      produce_z(p, b, tag, xring, &wdec[0][0], tslot, list, colmap, cum);
      depart(p, tag);
      return;
    }
    b -= p.mtiles;
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
    const int nrow = min(n0 + (tid >> 3) + 64 * i, p.n - 1);
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
  const int wn0 = n0 + wn * 48;
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
    // k-group g of ranks 0..31 (l0) and 32..63 (l1).
    auto load_b = [&](int d, bf16x8 (&l0)[kJ], bf16x8 (&l1)[kJ]) {
      const int br = mstride[d];
      const uint16_t* bg = p.b_store + mboff[d];
      const bool two = mrank[d] > 32;
#pragma unroll
      for (int j = 0; j < kJ; ++j) {
        const int n = wn0 + j * 16 + c;
        uint4 v0 = make_uint4(0, 0, 0, 0), v1 = make_uint4(0, 0, 0, 0);
        if (n < p.n) v0 = load_b8(bg + int64_t(n) * br, g * 8, br);
        if (two && n < p.n) v1 = load_b8(bg + int64_t(n) * br, 32 + g * 8, br);
        l0[j] = as_bf16x8(v0);
        l1[j] = as_bf16x8(v1);
      }
    };
    bf16x8 l0[kJ], l1[kJ];  // B fragments of the slot being applied (slot 0 first)
    wait_z(p, mt, tag);
    load_zs(0);
    if (nd > 0) load_b(0, l0, l1);
    round_bias(p, acc, wn0, g);
    // Routes of this lane's eight tokens.
    int rslot[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) rslot[i] = tslot[wm * 128 + i * 16 + c];
    uint4* zs = reinterpret_cast<uint4*>(xring);  // [token][8 units] with the x swizzle (the ring is idle)
    for (int s = 0; s < p.slices; ++s) {
      const int lo = p.slice_offsets[s];
      const int hi = p.slice_offsets[s + 1];
      if (s > 0) {
        __syncthreads();  // the previous slice's readers of zs are done
        load_zs(s);
      }
      wait_vm<0>();  // the z loads (and anything requested after them)
#pragma unroll
      for (int q = 0; q < kZq; ++q) tie(zr[q]);
#pragma unroll
      for (int q = 0; q < kZq; ++q) {
        const int row = (tid >> 3) + (kThreads / 8) * q;
        zs[swz(row, tid & 7)] = tslot[row] >= 0 ? make_uint4(zr[q].x, zr[q].y, zr[q].z, zr[q].w) : make_uint4(0, 0, 0, 0);
      }
      __syncthreads();
      if (hi <= wn0 || lo >= wn0 + 48) continue;  // this wave's 48 columns miss the slice
      const bool inside = lo <= wn0 && wn0 + 48 <= hi;
      // delta[n][m] = sum_j B_g[n][j] z[m][j] for the wave's 128 tokens x 48
      // features, added with the reference's two roundings to the tokens
      // routed to g and the features of slice s.
      for (int d = 0; d < nd; ++d) {
        const int gd = list[d];
        bool any = false;
#pragma unroll
        for (int i = 0; i < 8; ++i) any |= rslot[i] == gd;
        if (__ballot(any) == 0) continue;  // none of this wave's tokens takes slot d
        if (d > 0 || s > 0) load_b(d, l0, l1);
        const bool two = mrank[d] > 32;
        const float scale = mscale[d];
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
      }
    }
  } else {
    round_bias(p, acc, wn0, g);
  }
  if (p.y_vec == 2) {
    // 16-byte aligned rows: the tile goes through LDS (the idle x ring, rows
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
  } else {
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

// Workspace: the control header (call epoch), one z flag per 256-token tile
// at a fixed place (so a flag word only ever holds tags, whatever the shapes
// of earlier calls on the workspace), the z rows (m x slices x 64 bf16), then
// room for the fp32 block scales of a double-quant weight.
constexpr int64_t kMaxTiles = kFlagRegion / 4;

int64_t prefill_workspace_bytes(int64_t m, int64_t n, int64_t k, int slices, int) {
  return kWorkspaceHeader + kFlagRegion + align256(m * slices * kZSlice * 2) + align256(n * (k / kNf4Block) * 4);
}

int launch_nf4_lora_prefill(const uint16_t* x, int64_t m, int64_t x_stride, const lf_nf4_weight* w,
                            const uint16_t* bias, const lf_lora* lora, uint16_t* y, int64_t y_stride,
                            void* workspace, int64_t workspace_bytes, void* stream) {
  const int slices = lora ? lora->num_slices : 1;
  const bool dq = w->scales == nullptr;
  const int64_t need = prefill_workspace_bytes(m, w->n, w->k, slices, lora ? lora->max_rank : 1);
  LF_REQUIRE(!(lora || dq) || (workspace && workspace_bytes >= need && aligned16(workspace)),
             "workspace too small: need %lld bytes", (long long)need);
  LF_REQUIRE((m - 1) * x_stride * 2 + w->k * 2 < (int64_t(1) << 32), "x spans 4 GiB or more");
  LF_REQUIRE((m + wide::kBM - 1) / wide::kBM <= kMaxTiles, "prefill handles at most %lld tokens per call",
             (long long)(kMaxTiles * wide::kBM));
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
    p.zflags = reinterpret_cast<uint32_t*>(ws + kWorkspaceHeader);  // after the decode header
    p.zpad = reinterpret_cast<uint16_t*>(ws + kWorkspaceHeader + kFlagRegion);
    p.ce = call_epoch_of(ws);
    p.status = reinterpret_cast<int*>(ws + kStatusOffset);
  }
  p.mtiles = int((m + wide::kBM - 1) / wide::kBM);
  // LoRA launches put one z producer per M-tile ahead of the GEMM tiles.
  const dim3 grid(unsigned(p.mtiles * ((w->n + wide::kBN - 1) / wide::kBN) + (lora ? p.mtiles : 0)));
  if (lora) hipLaunchKernelGGL((wide::gemm_kernel<true>), grid, dim3(wide::kThreads), 0, s, p);
  else hipLaunchKernelGGL((wide::gemm_kernel<false>), grid, dim3(wide::kThreads), 0, s, p);
  LF_HIP(hipGetLastError());
  return kOk;
}

}  // namespace lf
