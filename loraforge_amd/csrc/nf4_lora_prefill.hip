// Prefill (M > 64 tokens): NF4 GEMM on bf16 MFMA with a multi-LoRA epilogue.
//
// Reference chain (integrations/_sglang_nf4_linear.py:116-129 for the base,
// benchmarks/qwen35_prefill_fused.py:95-171 segmented_ab_kernel for the
// LoRA part):  y = bf16(x @ dequant(W)^T) (+bias);  z = bf16(A_g x);
//              y = bf16(y + bf16(scale_g * B_g z)).
//
// Two launches on the caller's stream:
//  1. shrink: per 16-token block and distinct slot, z = bf16(x A_g^T) on
//     MFMA into a slice-padded workspace zpad[m][s*64 + j] (zeros past r).
//  2. GEMM: workgroup tile 256 tokens x 128 output features, BK = 64 (one
//     NF4 block per W row per k-step). x tiles go global -> registers -> LDS;
//     W tiles are 16 packed bytes per thread, decoded in registers (codebook
//     in LDS) to exact bf16 and written to LDS; four waves (2 x 2) each own
//     128 x 64 outputs as 8 x 4 fragments of v_mfma_f32_16x16x32_bf16.
//     LDS rows are 128 B with a 16-byte-unit XOR swizzle (unit ^ row % 8).
//     Epilogue: round, bias, then per slice the tile's z rows are staged in
//     LDS once and, for every distinct slot in the tile, a second MFMA pass
//     z x B_g^T over the 16-row blocks holding its tokens gives the LoRA
//     delta, applied with the reference's two bf16 roundings to the rows
//     routed to that slot.
//  Tile order puts M-tile b % mtiles on consecutive block ids, so with 8
//  M-tiles each XCD (block id % 8) keeps one 2 MiB x panel in its L2.
#include "nf4_common.h"
#include "../../include/loraforge_amd.h"

namespace lf {
namespace {

constexpr int kThreads = 256;
constexpr int kBM = 256;
constexpr int kBN = 128;
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
  uint16_t* zpad;  // [m][slices * 64]
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

// ---------------------------------------------------------------------------
// 1. shrink into zpad.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void prefill_shrink_kernel(PrefillParams p) {
  __shared__ int list[kMaxList + 1];
  __shared__ int tslot[kThreads];
  __shared__ int trank[16];
  const int t0 = blockIdx.x * 16;
  const int count = min(16, p.m - t0);
  live_slots(p, t0, count, tslot, list);
  if (threadIdx.x < 16) trank[threadIdx.x] = tslot[threadIdx.x] >= 0 ? p.ranks[tslot[threadIdx.x]] : 0;
  __syncthreads();
  const int nd = list[kMaxList];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int gq = lane >> 4;
  const int zw = p.slices * kZSlice;
  // Zero the padding columns [r, 64) of every live token's slices.
  for (int i = threadIdx.x; i < count * zw; i += kThreads) {
    const int t = i / zw;
    const int col = i - t * zw;
    const int r = trank[t];
    if (r > 0 && (col % kZSlice) >= r) p.zpad[int64_t(t0 + t) * zw + col] = 0;
  }
  for (int d = 0; d < nd; ++d) {
    const int g = list[d];
    const int r = p.ranks[g];
    const int rows = p.slices * r;
    const uint16_t* ag = p.a_store + p.a_offsets[g];
    const int tok = lane & 15;
    const bool mine = tslot[tok] == g;
    for (int ct = wave; ct * 16 < rows; ct += 4) {
      const int j = ct * 16 + (lane & 15);
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      // K is a multiple of 64; 8 steps of 32 k have their loads in flight together.
      const uint16_t* xrow = p.x + int64_t(t0 + (mine ? tok : 0)) * p.x_stride + gq * 8;
      const uint16_t* arow = ag + int64_t(j < rows ? j : 0) * p.k + gq * 8;
      for (int kc = 0; kc < p.k; kc += 8 * 32) {
        uint4 xv[8], av[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int kk = kc + 32 * i;
          const bool ok = kk < p.k;
          xv[i] = ok && mine ? *reinterpret_cast<const uint4*>(xrow + kk) : make_uint4(0, 0, 0, 0);
          av[i] = ok && j < rows ? *reinterpret_cast<const uint4*>(arow + kk) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) acc = mfma16(as_bf16x8(xv[i]), as_bf16x8(av[i]), acc);
      }
      // acc[e] = z[token 4*gq + e][column j]
      if (j < rows) {
        const int s = j / r;
        const int jj = j - s * r;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int t = 4 * gq + e;
          if (t < count && tslot[t] == g) p.zpad[int64_t(t0 + t) * zw + s * kZSlice + jj] = uint16_t(f32_to_bf16(acc[e]));
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 2. GEMM + epilogue.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint4 load_b8(const uint16_t* brow, int kk, int br) {
  if (kk + 8 <= br) return *reinterpret_cast<const uint4*>(brow + kk);
  uint32_t h[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) h[e] = kk + e < br ? brow[kk + e] : 0u;
  return make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
}

template <bool kDouble, bool kLora>
__global__ __launch_bounds__(kThreads, 2) void prefill_gemm_kernel(PrefillParams p) {
  __shared__ uint4 xs[kBM * 8];
  __shared__ uint4 ws[kBN * 8];
  __shared__ float table[16];
  __shared__ float code2[kDouble ? 256 : 1];
  __shared__ __attribute__((aligned(16))) int tslot[kBM];
  __shared__ int list[kMaxList + 1];
  const int tid = threadIdx.x;
  if (tid < 16) table[tid] = p.code[tid];
  if constexpr (kDouble) code2[tid] = p.src.code2[tid];
  const int mt = blockIdx.x % p.mtiles;
  const int nt = blockIdx.x / p.mtiles;
  const int m0 = mt * kBM;
  const int n0 = nt * kBN;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int wm = wave & 1;
  const int wn = wave >> 1;
  const int lr = lane & 15;
  const int gq = lane >> 4;
  __syncthreads();
  const float offset = kDouble ? *p.src.offset : 0.f;

  // Global load assignment.
  const int xrow = tid >> 3;   // + 32 * i
  const int xunit = tid & 7;
  const int wrow = tid >> 1;
  const int whalf = tid & 1;
  const bool wvalid = n0 + wrow < p.n;
  const uint8_t* wsrc = p.q + (int64_t(n0 + wrow) * p.k) / 2 + whalf * 16;
  const int64_t sblock0 = (int64_t(n0 + wrow) * p.k) / kNf4Block;

  uint4 xr[8];
  uint4 wr;
  float wscale;
  auto load_tile = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = m0 + xrow + 32 * i;
      xr[i] = row < p.m ? *reinterpret_cast<const uint4*>(p.x + int64_t(row) * p.x_stride + kt * kBK + xunit * 8)
                        : make_uint4(0, 0, 0, 0);
    }
    if (wvalid) {
      wr = *reinterpret_cast<const uint4*>(wsrc + kt * (kBK / 2));
      wscale = block_scale(p.src, sblock0 + kt, code2, offset);
    } else {
      wr = make_uint4(0, 0, 0, 0);
      wscale = 0.f;
    }
  };

  f32x4 acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  const int nk = p.k / kBK;
  load_tile(0);
  for (int kt = 0; kt < nk; ++kt) {
#pragma unroll
    for (int i = 0; i < 8; ++i) xs[swz(xrow + 32 * i, xunit)] = xr[i];
    ws[swz(wrow, whalf * 4 + 0)] = decode_dword(wr.x, wscale, table);
    ws[swz(wrow, whalf * 4 + 1)] = decode_dword(wr.y, wscale, table);
    ws[swz(wrow, whalf * 4 + 2)] = decode_dword(wr.z, wscale, table);
    ws[swz(wrow, whalf * 4 + 3)] = decode_dword(wr.w, wscale, table);
    __syncthreads();
    if (kt + 1 < nk) load_tile(kt + 1);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      bf16x8 af[8], bf[4];
#pragma unroll
      for (int i = 0; i < 8; ++i) af[i] = as_bf16x8(xs[swz(wm * 128 + i * 16 + lr, ks * 4 + gq)]);
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[j] = as_bf16x8(ws[swz(wn * 64 + j * 16 + lr, ks * 4 + gq)]);
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma16(af[i], bf[j], acc[i][j]);
    }
    __syncthreads();
  }

  // ---- epilogue ----------------------------------------------------------
  // acc[i][j][e] = C[token m0 + wm*128 + 16i + 4gq + e][feature n0 + wn*64 + 16j + lr]
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = n0 + wn * 64 + j * 16 + lr;
    const float bias = (p.bias && n < p.n) ? bf16_to_f32(p.bias[n]) : 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = round_bf16(acc[i][j][e]);
        if (p.bias) v = round_bf16(v + bias);
        acc[i][j][e] = v;
      }
  }
  if constexpr (kLora) {
    live_slots(p, m0, min(kBM, p.m - m0), tslot, list);
    const int nd = list[kMaxList];
    const int zw = p.slices * kZSlice;
    const int wn0 = n0 + wn * 64;
    // Per distinct slot metadata in the (idle) W buffer.
    int* mrank = reinterpret_cast<int*>(ws);
    int* mstride = mrank + kMaxList;
    float* mscale = reinterpret_cast<float*>(mstride + kMaxList);
    int64_t* mboff = reinterpret_cast<int64_t*>(mscale + kMaxList);
    static_assert(sizeof(ws) >= kMaxList * (3 * 4 + 8), "slot metadata fits the W buffer");
    for (int d = tid; d < nd; d += kThreads) {
      const int g = list[d];
      mrank[d] = p.ranks[g];
      mstride[d] = p.b_strides[g];
      mscale[d] = p.lscales[g];
      mboff[d] = p.b_offsets[g];
    }
    for (int s = 0; s < p.slices; ++s) {
      const int lo = p.slice_offsets[s];
      const int hi = p.slice_offsets[s + 1];
      // Every token's z row of this slice (zeros past its rank; zeros for
      // base-only tokens) is staged once in the x buffer, [token][64] bf16
      // with the x swizzle; each slot's pass reads the rows it needs.
      __syncthreads();  // previous users of xs (and the metadata stores) are done
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int row = (tid >> 3) + 32 * q;
        const int unit = tid & 7;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (tslot[row] >= 0) v = *reinterpret_cast<const uint4*>(p.zpad + int64_t(m0 + row) * zw + s * kZSlice + unit * 8);
        xs[swz(row, unit)] = v;
      }
      __syncthreads();
      if (hi <= wn0 || lo >= wn0 + 64) continue;  // this wave's 64 columns miss the slice
      for (int d = 0; d < nd; ++d) {
        const int g = list[d];
        // Bit 4i + e: the lane's row wm*128 + 16i + 4gq + e is routed to g.
        uint32_t mine = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int4 ts = *reinterpret_cast<const int4*>(tslot + wm * 128 + i * 16 + 4 * gq);
          mine |= (uint32_t(ts.x == g) | uint32_t(ts.y == g) << 1 | uint32_t(ts.z == g) << 2 | uint32_t(ts.w == g) << 3)
                  << (4 * i);
        }
        if (__ballot(mine != 0) == 0) continue;  // none of this wave's 128 rows takes g
        // B fragments of slot d: 4 column blocks, up to 2 k-steps (r <= 64).
        const int r = mrank[d];
        const int br = mstride[d];
        const uint16_t* bg = p.b_store + mboff[d];
        bf16x8 b0[4], b1[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int n = wn0 + j * 16 + lr;
          uint4 v0 = make_uint4(0, 0, 0, 0), v1 = make_uint4(0, 0, 0, 0);
          if (n < p.n) v0 = load_b8(bg + int64_t(n) * br, gq * 8, br);
          if (r > 32 && n < p.n) v1 = load_b8(bg + int64_t(n) * br, 32 + gq * 8, br);
          b0[j] = as_bf16x8(v0);
          b1[j] = as_bf16x8(v1);
        }
        const bool two = r > 32;
        const float scale = mscale[d];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if (__ballot((mine >> (4 * i)) & 15u) == 0) continue;  // no row of this 16-row block takes g
          const int arow = wm * 128 + i * 16 + lr;
          const bf16x8 z0 = as_bf16x8(xs[swz(arow, gq)]);
          const bf16x8 z1 = as_bf16x8(xs[swz(arow, 4 + gq)]);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            f32x4 dacc = {0.f, 0.f, 0.f, 0.f};
            dacc = mfma16(z0, b0[j], dacc);
            if (two) dacc = mfma16(z1, b1[j], dacc);
            const int n = wn0 + j * 16 + lr;
            const bool col = n >= lo && n < hi;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if (col && ((mine >> (4 * i + e)) & 1u)) acc[i][j][e] = round_bf16(acc[i][j][e] + round_bf16(dacc[e] * scale));
            }
          }
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = m0 + wm * 128 + i * 16 + 4 * gq + e;
      if (m >= p.m) continue;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = n0 + wn * 64 + j * 16 + lr;
        if (n < p.n) p.y[int64_t(m) * p.y_stride + n] = uint16_t(f32_to_bf16(acc[i][j][e]));
      }
    }
}

}  // namespace

int64_t prefill_workspace_bytes(int64_t m, int64_t, int64_t, int slices, int) {
  return kWorkspaceHeader + (m * slices * kZSlice * 2 + 255) / 256 * 256 + 256;
}

int launch_nf4_lora_prefill(const uint16_t* x, int64_t m, int64_t x_stride, const lf_nf4_weight* w,
                            const uint16_t* bias, const lf_lora* lora, uint16_t* y, int64_t y_stride,
                            void* workspace, int64_t workspace_bytes, void* stream) {
  const int slices = lora ? lora->num_slices : 1;
  const int64_t need = prefill_workspace_bytes(m, w->n, w->k, slices, lora ? lora->max_rank : 1);
  LF_REQUIRE(!lora || (workspace && workspace_bytes >= need && aligned16(workspace)),
             "workspace too small: need %lld bytes", (long long)need);
  PrefillParams p{};
  p.x = x;
  p.x_stride = x_stride;
  p.m = int(m);
  p.q = w->qweight;
  p.src = ScaleSource{w->scales, w->absmax_q, w->absmax2, w->code2, w->offset, int(w->dq_block)};
  p.code = w->code;
  p.n = int(w->n);
  p.k = int(w->k);
  p.bias = bias;
  p.y = y;
  p.y_stride = y_stride;
  p.slices = slices;
  p.mtiles = int((m + kBM - 1) / kBM);
  const int ntiles = int((w->n + kBN - 1) / kBN);
  auto s = static_cast<hipStream_t>(stream);
  const bool dq = w->scales == nullptr;
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
    p.zpad = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) + kWorkspaceHeader);  // after the decode header
    hipLaunchKernelGGL(prefill_shrink_kernel, dim3(unsigned((m + 15) / 16)), dim3(kThreads), 0, s, p);
    LF_HIP(hipGetLastError());
  }
  const dim3 grid(unsigned(p.mtiles * ntiles));
  if (dq) {
    if (lora) hipLaunchKernelGGL((prefill_gemm_kernel<true, true>), grid, dim3(kThreads), 0, s, p);
    else hipLaunchKernelGGL((prefill_gemm_kernel<true, false>), grid, dim3(kThreads), 0, s, p);
  } else {
    if (lora) hipLaunchKernelGGL((prefill_gemm_kernel<false, true>), grid, dim3(kThreads), 0, s, p);
    else hipLaunchKernelGGL((prefill_gemm_kernel<false, false>), grid, dim3(kThreads), 0, s, p);
  }
  LF_HIP(hipGetLastError());
  return kOk;
}

}  // namespace lf
