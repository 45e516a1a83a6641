/*
 * loraforge_amd -- C ABI of the MI355X (gfx950) NF4 + multi-LoRA serving path.
 *
 * Every entry point takes raw device pointers, element counts/strides and a
 * HIP stream (passed as void*, NULL = the null stream), launches
 * asynchronously on that stream, allocates nothing and returns an int status:
 *   LF_OK (0), LF_EINVAL (1, argument/layout contract -> ValueError),
 *   LF_EHIP (2, HIP runtime error -> RuntimeError).
 * lf_last_error() returns the calling thread's message for the last failure.
 * bf16 tensors are passed as uint16_t bit patterns. Device metadata values are
 * trusted (never read back to the host), so calls are graph-capturable.
 *
 * Reference citations are relative to the reference tree
 * (lishenghui/loraforge, src/loraforge/...).
 */
#ifndef LORAFORGE_AMD_H
#define LORAFORGE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 2: lf_row_shrink gained num_adapters, workspace, workspace_bytes and flags,
 * lf_row_expand gained segments (arguments inserted mid-list).
 * 3: lf_lora gained num_slots (appended).
 * 4: lf_row_expand_tiled added. */
#define LF_ABI_VERSION 4
#define LF_OK 0
#define LF_EINVAL 1
#define LF_EHIP 2

const char* lf_last_error(void);
int lf_abi_version(void);
/* gcnArchName of a device (e.g. "gfx950:sramecc+:xnack-"). */
int lf_device_arch(int device, char* name, int capacity);

/* --------------------------------------------------------------------------
 * NF4 dequantisation.
 * Replaces the Triton launch of ops/nf4.py:7-38 (_dequantize, byte-pair
 * kernel ops/_nf4_kernels.py:44-61) behind dequantize_nf4 (ops/nf4.py:44).
 * out[e] = bf16_rne(code[nibble(e)] * scales[e / 64]); nibble(e) is the high
 * nibble of byte e/2 for even e, the low nibble for odd e.
 * numel = N*K, a positive multiple of 4096. Any byte address for qweight and
 * any 2-byte address for out (the reference accepts every contiguous tensor);
 * qweight 4-byte aligned with out 16-byte aligned takes the vector path.
 * ------------------------------------------------------------------------ */
int lf_nf4_dequant(const uint8_t* qweight, const float* scales, const float* code, uint16_t* out,
                   int64_t numel, void* stream);

/* Same, with double-quantised block scales reconstructed in-kernel as
 * fl32(fl32(code2[absmax_q[j]] * absmax2[j / dq_block]) + *offset)
 * (ops/nf4.py:144-147, prepare_scales nested branch). offset is a device
 * pointer to one fp32; code2 holds 256 fp32. */
int lf_nf4_dequant_dq(const uint8_t* qweight, const uint8_t* absmax_q, const float* absmax2,
                      const float* code2, const float* offset, int64_t dq_block, const float* code,
                      uint16_t* out, int64_t numel, void* stream);

/* prepare_scales (ops/nf4.py:109-148) nested branch: writes the nblocks fp32
 * scales that bitsandbytes dequantize_blockwise(absmax, state2) + offset
 * produces, without bitsandbytes. */
int lf_nf4_prepare_scales_dq(const uint8_t* absmax_q, const float* absmax2, const float* code2,
                             const float* offset, int64_t dq_block, float* scales, int64_t nblocks,
                             void* stream);

/* --------------------------------------------------------------------------
 * Retained-rank row operators.
 * lf_row_shrink replaces the pybind `shrink` of ops/csrc/lora_rows.cu:172-186
 * (row_shrink, ops/lora_rows.py:54-109): x [tokens, width] with row stride
 * x_stride; a [G, num_slices*capacity, width] contiguous; z [tokens,
 * num_slices*capacity] contiguous; slots int32 [tokens]; ranks int32 [G];
 * num_adapters = G (the pybind binding reads it from a's shape).
 * num_slices 1..4 (the row_shrink API allows 3, the Fleet direct_shrink of
 * ops/rowexpand.py:34-39 / rowexpand.cu:87-97 allows 4).
 * ------------------------------------------------------------------------ */
int lf_row_shrink(const uint16_t* x, const uint16_t* a, uint16_t* z, const int32_t* slots,
                  const int32_t* ranks, int64_t tokens, int64_t width, int64_t x_stride,
                  int64_t num_adapters, int32_t num_slices, int64_t capacity, int32_t max_rank,
                  void* workspace, int64_t workspace_bytes, int32_t flags, void* stream);

/* Bytes of workspace lf_row_shrink needs (0: none). Small token counts split
 * K across workgroups and sum the fp32 partials in the workspace; it must be
 * zero before its first use and is never reset between calls (entries carry
 * the tag of the call that wrote them, as in lf_nf4_lora_workspace_size).
 * Calls that share a workspace must not overlap; lf_nf4_lora_status reads
 * its status word (1: a partial had to be recomputed by the summing
 * workgroup after a bounded wait; the result is still exact). */
int64_t lf_row_shrink_workspace_size(int64_t tokens, int64_t width, int64_t num_adapters,
                                     int32_t num_slices, int32_t max_rank);

/* Test hook (lf_row_shrink and lf_nf4_lora_linear): the producers publish
 * nothing (row shrink: K chunks past the first store no partials; fused
 * linear: decode shrink producers store no tagged partials, prefill z
 * producers store no z and set no flag), so every consumer gives up its
 * (shortened) bounded wait, recomputes what it waited for from x and A and
 * sets the status word; the output must not change beyond rounding. */
#define LF_TEST_WITHHOLD_PARTIALS 0x100

/* lf_row_expand replaces the pybind `expand` of ops/csrc/lora_rows.cu:188-209
 * (row_expand, ops/lora_rows.py:115-239); arguments keep that binding's
 * order and meaning. b_strides is the reference's "buckets". segments is the
 * length of segment_slots (segment_indptr holds segments + 1 entries; the
 * binding reads it from the tensor): the kernel reads a segment's bounds and
 * slot together with the live count instead of after it. */
int lf_row_expand(const uint16_t* z, const uint16_t* b, const int64_t* b_offsets,
                  const int32_t* b_strides, uint16_t* y, const int32_t* segment_indptr,
                  const int32_t* segment_slots, const int32_t* token_indices, const int32_t* ranks,
                  const float* scales, const int32_t* slice_offsets, const int32_t* segment_count,
                  int64_t segments, int64_t tokens, int64_t out_width, int64_t y_stride,
                  int32_t num_slices, int64_t capacity, int32_t blocks, int32_t threads, void* stream);

/* lf_row_expand_tiled replaces the pybind `expand` of ops/csrc/rowexpand.cu:98-127
 * (the Fleet row_expand, ops/rowexpand.py:42-92): lf_row_expand's arguments
 * plus row_tile (2, 4, 8 or 16; anything else is LF_EINVAL, as there). The
 * reference splits a segment's B work into items of row_tile tokens; here an
 * item is a segment times a run of output columns, and row_tile bounds that
 * run: 16 lets the library pick it from the work count (as lf_row_expand
 * does), 8 caps it at 32 columns per wave, 4 and 2 at 16. Outputs are
 * bitwise identical for every row_tile. */
int lf_row_expand_tiled(const uint16_t* z, const uint16_t* b, const int64_t* b_offsets,
                        const int32_t* b_strides, uint16_t* y, const int32_t* segment_indptr,
                        const int32_t* segment_slots, const int32_t* token_indices, const int32_t* ranks,
                        const float* scales, const int32_t* slice_offsets, const int32_t* segment_count,
                        int64_t segments, int64_t tokens, int64_t out_width, int64_t y_stride,
                        int32_t num_slices, int64_t capacity, int32_t blocks, int32_t threads, int32_t row_tile,
                        void* stream);

/* --------------------------------------------------------------------------
 * Fused NF4 base linear + per-token multi-LoRA (one launch for decode).
 * Replaces the three-call sequence of the reference serving path:
 *   integrations/_sglang_nf4_linear.py:116-129 (dequant -> F.linear -> +bias),
 *   ops/rowexpand.py:34-39 / ops/lora_rows.py:54 (shrink),
 *   ops/rowexpand.py:42-92 / ops/lora_rows.py:115 (expand).
 * y[m, n] = bf16(x[m] . W[n]) (+bias, bf16) then, for token m with slot
 * g = token_slots[m] >= 0 and r = ranks[g] > 0, column n in slice s:
 *   z = bf16(A_g[s*r + j] . x[m]),
 *   y[m, n] = bf16(y[m, n] + bf16(scales[g] * sum_j z[s*r + j] * B_g[n, j])).
 * A_g: num_slices*r rows of width K at element a_offsets[g] of a_store.
 * B_g: [N, b_strides[g]] at element b_offsets[g] of b_store (zero padded).
 * ------------------------------------------------------------------------ */
typedef struct lf_nf4_weight {
  const uint8_t* qweight; /* [N*K/2] */
  const float* scales;    /* fp32 [N*K/64], or NULL when double-quantised:
                             then the decode kernels stage the uint8 codes
                             and absmax2 entries of their rows into LDS and
                             convert them there (K % 256 == 0, dq_block a
                             power of two >= 64, absmax_q 4-byte and code2
                             16-byte aligned; other shapes, and the prefill
                             GEMM, rebuild fp32 scales into the workspace
                             first, as lf_nf4_prepare_scales_dq does) */
  const uint8_t* absmax_q;/* uint8 [N*K/64] (double quant) */
  const float* absmax2;   /* fp32 [ceil(N*K/64/dq_block)] */
  const float* code2;     /* fp32 [256] */
  const float* offset;    /* fp32 [1] */
  int64_t dq_block;
  const float* code;      /* fp32 [16] */
  int64_t n;              /* output features, multiple of 64 */
  int64_t k;              /* input features, multiple of 64 */
} lf_nf4_weight;

typedef struct lf_lora {
  const uint16_t* a_store;
  const int64_t* a_offsets;   /* [G] element offsets, multiples of 8 */
  const uint16_t* b_store;
  const int64_t* b_offsets;   /* [G] element offsets, multiples of 8 */
  const int32_t* b_strides;   /* [G] power of two in 1..64, >= rank */
  const int32_t* ranks;       /* [G] 0..max_rank */
  const float* scales;        /* [G] */
  const int32_t* token_slots; /* [M] slot or -1 */
  const int32_t* slice_offsets; /* [num_slices+1] */
  int32_t num_slices;         /* 1..3 */
  int32_t max_rank;           /* 1..64 */
  int32_t num_slots;          /* G, the entries of the per-slot arrays, or 0
                                 when not given. When given, token slots >= G
                                 run base only, and with G <= 256 the wide
                                 decode kernel (9..64 tokens; 3..64 at
                                 N >= 8192) requests the per-slot arrays
                                 whole at its start, before it has read the
                                 tokens' slots. */
} lf_lora;

/* Bytes of device workspace lf_nf4_lora_linear needs for this problem. The
 * first 256 KiB are the decode kernel's control header (a launch word, a
 * status word and the shrink partials, each tagged with the call that wrote
 * it); it must be zero before the first call and is never reset between
 * calls. A prefill call uses the rest for its z rows and, for a double-quant
 * weight, the rebuilt fp32 block scales; a decode call of a double-quant
 * weight whose kernel does not read the nested state itself rebuilds them
 * after the prefill's flag region (a decode call with fp32 scales, or whose
 * kernel reads the nested state, needs only the header). Decode and prefill
 * calls may share one workspace; calls that share one workspace must not
 * overlap in time. */
int64_t lf_nf4_lora_workspace_size(int64_t m, int64_t n, int64_t k, int32_t num_slices, int32_t max_rank);

/* x [m, K] bf16 with row stride x_stride (multiple of 8, 16-byte aligned);
 * y [m, N] bf16 with row stride y_stride; bias bf16 [N] or NULL;
 * lora NULL for the base linear alone. M <= 64 runs the decode kernel
 * (fp32 block scales required). M > 64 runs either the prefill GEMM, which
 * multiplies the reference's dequantised weights bf16_rne(code * scale) bit
 * for bit and takes fp32 block scales or a double-quant state (rebuilt into
 * the workspace first; the workspace is then required even without LoRA),
 * or, when its 256 x 192 tiles would leave most CUs idle (few tokens, narrow
 * N) and fp32 block scales are given, the decode kernel over 64-token chunks
 * (one launch per chunk, in token order). A cost model of the two, from
 * measured times, picks the plan; LF_PLAN_DECODE_CHUNKS or LF_PLAN_PREFILL
 * forces one (a forced chunked plan needs fp32 block scales).
 * flags: LF_EXACT_WEIGHTS makes the decode kernel multiply the same exact
 * weights; by default it contracts bf16(code) and applies each fp32 block
 * scale to the block's MFMA sum. The prefill GEMM ignores the flag.
 * LF_SWIGLU_OUTPUT (any M; the prefill GEMM also needs y 16-byte aligned
 * with y_stride % 8 == 0): the weight is a merged gate/up projection (gate
 * rows 0 .. N/2, up rows N/2 .. N; with LoRA its two slices are
 * [0, N/2, N]) and y receives h[m][f] = bf16(bf16(silu(gate[m][f])) *
 * up[m][f]), [M, N/2] with row stride y_stride >= N/2, where gate and up are
 * the bf16 outputs including their LoRA adds (benchmarks/qwen35_decode_silu.py:60-61
 * and the prefill expand_act_kernel, benchmarks/qwen35_prefill_fused.py:14-93,
 * fused into the epilogue instead of a second launch). */
#define LF_EXACT_WEIGHTS 1
#define LF_SWIGLU_OUTPUT 2
#define LF_PLAN_DECODE_CHUNKS 4
#define LF_PLAN_PREFILL 8
int lf_nf4_lora_linear(const uint16_t* x, int64_t m, int64_t x_stride, const lf_nf4_weight* weight,
                       const uint16_t* bias, const lf_lora* lora, uint16_t* y, int64_t y_stride,
                       void* workspace, int64_t workspace_bytes, int32_t flags, void* stream);

/* LoRA-only update of existing bf16 outputs, in one launch per 64 tokens:
 * for every token t routed to slot g = token_slots[t] >= 0 with rank
 * r = ranks[g] > 0, and every output column n of slice s,
 *   z[t, s*r + j] = bf16(sum_w x[t, w] * A_g[s*r + j, w]),
 *   y[t, n] = bf16(bf16(y[t, n]) + bf16(scales[g] * sum_j z[t, s*r + j] * B_g[n, j])).
 * It replaces lf_row_shrink followed by lf_row_expand (the reference chain
 * ops/lora_rows.py:51-239, ops/csrc/lora_rows.cu:35-162; its one-launch
 * precedent is benchmarks/qwen35_tiny_fused.cu:34-53) when z is not needed
 * by the caller: routing is per token (no segment lists) and z never leaves
 * the chip. Tokens without an adapter keep their y bit for bit. x [m, K]
 * bf16 (16-byte aligned rows, stride % 8 == 0), y [m, N] bf16 updated in
 * place (row stride >= N); N and K multiples of 64; the workspace is that of
 * lf_nf4_lora_linear for m <= 64 (lf_nf4_lora_workspace_size(min(m, 64), ...))
 * and calls sharing it must not overlap. flags: LF_TEST_WITHHOLD_PARTIALS only. */
int lf_lora_apply(const uint16_t* x, int64_t m, int64_t x_stride, int64_t n, int64_t k, const lf_lora* lora,
                  uint16_t* y, int64_t y_stride, void* workspace, int64_t workspace_bytes, int32_t flags, void* stream);

/* Allocation-free variant of lf_nf4_lora_linear. It has no counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Arguments and results are those of lf_nf4_lora_linear; the
 * workspace is a library-owned device array of LF_NOALLOC_SCRATCH_BYTES per
 * device (held until the process ends), and problems whose
 * lf_nf4_lora_workspace_size exceeds it are rejected with LF_EINVAL. The
 * first call on a device clears the array on its stream and must not be
 * captured; it finishes the clear (synchronising its stream once) before
 * returning, so later calls on any stream find the array cleared; later
 * calls may be captured. It calls no allocator. Every call on a device
 * shares that device's array: calls that overlap in time on one GPU race,
 * so calls on different streams must be ordered by the caller (events). */
#define LF_NOALLOC_SCRATCH_BYTES (8 * 1024 * 1024)
int lf_nf4_lora_linear_noalloc(const uint16_t* x, int64_t m, int64_t x_stride, const lf_nf4_weight* weight,
                               const uint16_t* bias, const lf_lora* lora, uint16_t* y, int64_t y_stride,
                               int32_t flags, void* stream);

/* Reads the workspace status word written by the last call (0 = ok); for
 * tests and diagnostics only (synchronises the stream). */
int lf_nf4_lora_status(const void* workspace, void* stream, int32_t* status);

/* --------------------------------------------------------------------------
 * SwiGLU between an MLP's gate/up and down projections (the c3 chain):
 * out[t, c] = bf16(bf16(silu(g)) * u), g = gate_up[t, c], u = gate_up[t, n + c],
 * silu(g) = g / (1 + exp(-g)) in fp32. Replaces the activation step of
 * benchmarks/qwen35_decode_silu.py:60-61 (row_act_kernel) and
 * benchmarks/qwen35_prefill_fused.py:14-93 (expand_act_kernel), which apply
 * it after the gate/up LoRA adds; here it reads the merged two-slice output
 * of lf_nf4_lora_linear. in_stride >= 2n, out_stride >= n (elements).
 * ------------------------------------------------------------------------ */
int lf_swiglu(const uint16_t* gate_up, int64_t rows, int64_t n, int64_t in_stride, uint16_t* out,
              int64_t out_stride, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* LORAFORGE_AMD_H */
