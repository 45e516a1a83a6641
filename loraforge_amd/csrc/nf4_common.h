// NF4 decode helpers shared by the dequantisation, decode and prefill kernels.
//
// Packed layout (bitsandbytes / reference, ops/nf4.py:47-49): element e of a
// row-major [N, K] weight is nibble (e & 1 ? low : high) of byte e / 2.
// Block scale: scale[e / 64]; value = bf16_rne(code[nibble] * scale) with a
// single fp32 multiply (ops/_nf4_kernels.py:33-35,55-59).
#pragma once

#include "common.h"

namespace lf {

constexpr int kNf4Block = 64;

// Every fused-linear workspace starts with this control header, owned by the
// decode kernel: its launch word, status word and tagged shrink partials
// (entries are valid only for the call whose tag they carry, so nothing is
// reset between calls). No other kernel writes it, so decode and prefill
// calls can share one workspace.
constexpr int64_t kWorkspaceHeader = 262144;
// The prefill's z flags follow the header at a fixed place: 4096 flags, one
// per 256-token tile.
constexpr int64_t kFlagRegion = 16384;

// Codebook lookup by a byte offset (nibble * 4) into a 16-entry fp32 table in
// LDS. All lanes read at most 16 distinct words, so the read is bank-conflict
// free; broadcast covers repeated nibbles.
__device__ __forceinline__ float code_at(const float* table, uint32_t byte_offset) {
  return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(table) + byte_offset);
}

// One packed dword (8 consecutive elements, high nibble first in each byte)
// -> 4 packed bf16 pairs in element order, each = bf16_rne(code * scale).
__device__ __forceinline__ uint4 decode_dword(uint32_t d, float scale, const float* table) {
  const uint32_t even = (d >> 2) & 0x3c3c3c3cu;  // byte b: 4 * high nibble of byte b
  const uint32_t odd = (d << 2) & 0x3c3c3c3cu;   // byte b: 4 * low nibble of byte b
  uint4 r;
  r.x = pack_bf16x2(code_at(table, even & 0xffu) * scale, code_at(table, odd & 0xffu) * scale);
  r.y = pack_bf16x2(code_at(table, (even >> 8) & 0xffu) * scale, code_at(table, (odd >> 8) & 0xffu) * scale);
  r.z = pack_bf16x2(code_at(table, (even >> 16) & 0xffu) * scale, code_at(table, (odd >> 16) & 0xffu) * scale);
  r.w = pack_bf16x2(code_at(table, even >> 24) * scale, code_at(table, odd >> 24) * scale);
  return r;
}

// Block-scale source: either an fp32 vector or the double-quantised triple
// (uint8 absmax codes, fp32 second-level scales per dq_block, 256-entry
// fp32 code2 and a scalar offset) reconstructed as
// fl32(fl32(code2[q] * absmax2[j / dq_block]) + offset)  (ops/nf4.py:144-147).
struct ScaleSource {
  const float* scales;    // fp32 [nblocks] or nullptr when double-quantised
  const uint8_t* absmax_q;  // uint8 [nblocks]
  const float* absmax2;   // fp32 [ceil(nblocks / dq_block)]
  const float* code2;     // fp32 [256]
  const float* offset;    // fp32 [1]
  int dq_block;
};

// code2 must already be staged into LDS (code2_lds) when double-quantised.
__device__ __forceinline__ float block_scale(const ScaleSource& s, int64_t block, const float* code2_lds,
                                             float offset) {
  if (s.scales) return s.scales[block];
  const float level = code2_lds[s.absmax_q[block]] * s.absmax2[block / s.dq_block];
  return level + offset;
}

}  // namespace lf
