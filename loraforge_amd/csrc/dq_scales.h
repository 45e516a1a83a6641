// Double-quantised block scales inside a decode wave's LDS scale area.
//
// A decode base wave keeps the fp32 block scales of its rows over its blocks
// kb0 .. kb0 + nb - 1 in an LDS area, row r (local; global row lo + r for
// r < R / 2, hi + r - R / 2 otherwise) at r * stride floats. Given a nested
// (double-quant) state instead of fp32 scales, the wave copies into the
// area's tail, where the fp32 copies would have been issued:
//   - a 256-byte slot of absmax2 entries: lanes 0..31 the entries from the
//     first row half's first block on, lanes 32..63 from the second half's;
//   - each row's uint8 absmax codes from block kb0 & ~3 on, cw dwords a row;
// and once they have landed converts them in place with the closed form of
// lf_nf4_dequant_dq (the same two fp32 operations, no contraction):
//   scale = code2[code] * absmax2[block >> dq_shift] + offset.
// That reads 1 byte per 64 weights from HBM instead of the 4 of prepared
// scales (reference: ops/nf4.py:109-148, the nested branch of prepare_scales,
// and _nf4_kernels.py:29-61 for its use).
//
// The host takes this path only where the area holds the staging
// (dq_stage_bytes), the absmax2 entries of a row half number at most 32,
// K % 256 == 0 (codes rows start on dwords), the code pointer is 4-byte
// aligned, dq_block is a power of two of at least 64 blocks and a lane
// converts at most kDqEntries (16) columns; elsewhere it rebuilds fp32 scales
// into the workspace first.
#pragma once

#include "lds_pipeline.h"

namespace lf {

constexpr int kDqEntries = 16;  // columns of a row one lane converts, at most

// Columns per lane for an area of `rows` rows of `stride` entries.
__host__ __device__ inline int dq_cols_per_lane(int rows, int stride) {
  const int parts = 64 / rows;
  return (stride + parts - 1) / parts;
}

// Code dwords per row for nb blocks starting anywhere in a dword.
__host__ __device__ inline int dq_code_dwords(int nb) { return (nb + 6) >> 2; }
// Bytes of the staging at the area's tail: the absmax2 slot and the codes.
__host__ __device__ inline int dq_stage_bytes(int rows, int nb) {
  return 256 + (rows * dq_code_dwords(nb) + 63) / 64 * 256;
}

struct DqStage {
  int cw;     // code dwords per row
  int slot;   // byte offset of the absmax2 slot in the area
  int codes;  // byte offset of the codes
  int a0;     // absmax2 entry of the first row half's first block
  int a1;     // the same for the second half
};

template <class P>
__device__ __forceinline__ DqStage dq_stage(const P& p, int area_bytes, int rows, int lo, int hi, int kb0, int nb) {
  DqStage st;
  const int nblk = p.k >> 6;
  st.cw = dq_code_dwords(nb);
  st.slot = area_bytes - dq_stage_bytes(rows, nb);
  st.codes = st.slot + 256;
  st.a0 = int((int64_t(lo) * nblk + kb0) >> p.dq_shift);
  st.a1 = int((int64_t(hi) * nblk + kb0) >> p.dq_shift);
  return st;
}

// The staging copies (dword direct copies, in issue order with the wave's
// other copies). Every source address is inside its array.
template <class P>
__device__ __forceinline__ void dq_issue(const P& p, char* area, const DqStage& st, int rows, int lo, int hi, int kb0,
                                         int lane) {
  const int nblk = p.k >> 6;
  const int half = rows >> 1;
  copy4(p.absmax2 + min((lane < 32 ? st.a0 : st.a1) + (lane & 31), p.a2_len - 1), area + st.slot);
  const int total = rows * st.cw;
  const int64_t last = int64_t(p.n) * nblk - 4;  // the last whole dword of codes (nblk % 4 == 0)
  for (int i = 0; i * 64 < total; ++i) {
    const int e = min(i * 64 + lane, total - 1);
    const int r = e / st.cw;
    const int d = e - r * st.cw;
    const int row = r < half ? lo + r : hi + (r - half);
    const int64_t b = min(int64_t(row) * nblk + (kb0 & ~3) + 4 * d, last);
    copy4(p.absmax_q + b, area + st.codes + i * 256);
  }
}

// code2 into the workgroup's 1 KiB table (four dword direct copies; one wave
// issues them ahead of its staging and raises a flag once they have landed).
template <class P>
__device__ __forceinline__ void dq_issue_code2(const P& p, float* table, int lane) {
#pragma unroll
  for (int c = 0; c < 4; ++c) copy4(p.code2 + c * 64 + lane, reinterpret_cast<char*>(table + c * 64));
}

// The conversion, once the staging copies have landed (LDS accesses the
// compiler does not track: direct copies of later stages may still be in
// flight). Lane l takes row l % rows and a run of cpp = ceil(stride / parts)
// consecutive columns, parts = 64 / rows: its codes are a few dwords of the
// row's staging and its absmax2 entries at most two (dq_block >= 64 blocks,
// cpp <= kCols <= 16), so per entry only a table lookup, a multiply and an
// add are left. Padding columns (nb .. stride - 1) repeat column 0, as the fp32
// copies do. Every lane reads its staging before any lane of the wave stores
// (the staging may share the area's tail with the entries).
template <int kCols, class P>
__device__ __forceinline__ void dq_convert(const P& p, char* area, const DqStage& st, int rows, int lo, int hi,
                                           int kb0, int nb, const float* table, float offset, int lane) {
  static_assert(kCols % 4 == 0 && kCols <= kDqEntries, "columns per lane");
  const int nblk = p.k >> 6;
  const int half = rows >> 1;
  const int parts = 64 / rows;
  const int stride = p.sc_stride;
  const int cpp = (stride + parts - 1) / parts;  // <= kCols (host-checked)
  const int r = lane % rows;
  const int c_lo = (lane / rows) * cpp;
  const bool first = r < half;
  const int row = first ? lo + r : hi + (r - half);
  const int64_t g0 = int64_t(row) * nblk + kb0;  // global block of column 0
  const int a_base = first ? st.a0 : st.a1;
  const uint32_t base = lds_addr(area);
  // Codes of columns c_lo .. c_lo + cpp - 1 (byte (kb0 & 3) + c of the row's
  // staging; padding columns read column 0's byte): the dwords from the
  // run's first byte on, clamped into the row's cw dwords.
  const int b0 = (kb0 & 3) + c_lo;
  const uint32_t row_codes = base + uint32_t(st.codes + r * st.cw * 4);
  const int d0 = b0 >> 2;
  uint32_t words[kCols / 4 + 2];
#pragma unroll
  for (int i = 0; i < kCols / 4 + 2; ++i) words[i] = lds_read32(row_codes + uint32_t(min(d0 + i, st.cw - 1) * 4));
  const uint32_t col0 = lds_read32(row_codes + uint32_t(((kb0 & 3) >> 2) * 4));  // the dword of column 0's byte
  // absmax2 entries: the run's first column's and the next.
  const int a_first = int((g0 + min(c_lo, nb > 0 ? nb - 1 : 0)) >> p.dq_shift) - a_base;
  const uint32_t slot = base + uint32_t(st.slot + ((first ? 0 : 32) + a_first) * 4);
  float a2_lo = lds_read32f(slot);
  float a2_hi = lds_read32f(slot + 4u);
  const float a2_col0 = lds_read32f(base + uint32_t(st.slot + ((first ? 0 : 32) + int((g0 >> p.dq_shift) - a_base)) * 4));
  lds_wait();
#pragma unroll
  for (int i = 0; i < kCols / 4 + 2; ++i) tie(words[i]);
  uint32_t c0w = col0;
  tie(c0w);
  tie(a2_lo);
  tie(a2_hi);
  float a2c0 = a2_col0;
  tie(a2c0);
  // The run's codes from byte b0 & 3 of the first word on, realigned so that
  // column c_lo + j is byte j % 4 of dword j / 4 (compile-time indices only:
  // a register array indexed at run time would go through scratch).
  uint32_t run[kCols / 4];
#pragma unroll
  for (int i = 0; i < kCols / 4; ++i) run[i] = __builtin_amdgcn_alignbyte(words[i + 1], words[i], uint32_t(b0 & 3));
  const uint32_t tbase = lds_addr(table);
  float code2[kCols];
  float a2[kCols];
#pragma unroll
  for (int j = 0; j < kCols; ++j) {
    const int c = c_lo + j;
    const bool pad = c >= nb;
    const uint32_t code = pad ? ((c0w >> (8 * (kb0 & 3))) & 0xffu) : ((run[j >> 2] >> (8 * (j & 3))) & 0xffu);
    code2[j] = lds_read32f(tbase + (code << 2));
    const bool second = int((g0 + c) >> p.dq_shift) - a_base > a_first;
    a2[j] = pad ? a2c0 : (second ? a2_hi : a2_lo);
  }
  lds_wait();
#pragma unroll
  for (int j = 0; j < kCols; ++j) {
    tie(code2[j]);
    const int c = c_lo + j;
    const float level = code2[j] * a2[j];
    const float v = level + offset;
    if (j < cpp && c < stride)
      asm volatile("ds_write_b32 %0, %1" ::"v"(base + uint32_t((r * stride + c) * 4)), "v"(v) : "memory");
  }
}

}  // namespace lf
