// C-ABI entry of the fused NF4 + multi-LoRA linear: argument validation and
// dispatch between the decode kernel (M <= 64 tokens, or 64-token chunks of a
// larger batch that the prefill tiles would not spread over the chip) and the
// prefill GEMM.
#include <algorithm>

#include "nf4_common.h"
#include "../../include/loraforge_amd.h"

namespace lf {
int64_t gemv_workspace_bytes(int64_t m, int64_t n, int64_t k, int slices, int max_rank);
int launch_nf4_gemv(const uint16_t* x, int64_t m, int64_t x_stride, const lf_nf4_weight* w, const uint16_t* bias,
                    const lf_lora* lora, uint16_t* y, int64_t y_stride, void* workspace, int64_t workspace_bytes,
                    bool exact, bool swiglu, bool withhold, void* stream, bool residual = false);
int64_t prefill_workspace_bytes(int64_t m, int64_t n, int64_t k, int slices, int max_rank);
int launch_nf4_lora_prefill(const uint16_t* x, int64_t m, int64_t x_stride, const lf_nf4_weight* w,
                            const uint16_t* bias, const lf_lora* lora, uint16_t* y, int64_t y_stride,
                            void* workspace, int64_t workspace_bytes, bool swiglu, bool withhold, void* stream);
int device_cus();
bool decode_wide_fits(int64_t m, int64_t n, int64_t k, const lf_lora* lora);
bool wide_takes_dq(const lf_nf4_weight* w);
bool gemv_takes_dq(int64_t m, const lf_nf4_weight* w, const lf_lora* lora, bool exact);
int rebuild_decode_scales(const lf_nf4_weight* w, void* workspace, int64_t workspace_bytes, void* stream,
                          const float** scales);
bool lora_apply_wide_fits(int64_t m, int64_t n, int64_t k, const lf_lora* lora);
int launch_lora_apply_wide(const uint16_t* x, int64_t m, int64_t x_stride, int64_t n, int64_t k, const lf_lora* lora,
                           uint16_t* y, int64_t y_stride, void* workspace, int64_t workspace_bytes, bool withhold,
                           void* stream);
int launch_decode_wide(const uint16_t* x, int64_t m, int64_t x_stride, const lf_nf4_weight* w, const uint16_t* bias,
                       const lf_lora* lora, uint16_t* y, int64_t y_stride, void* workspace, int64_t workspace_bytes,
                       bool exact, bool swiglu, bool withhold, void* stream);
constexpr int64_t kDecodeMaxTokens = 64;

// Whether the wide decode kernel (32 rows x 32 tokens per workgroup over the
// whole K) serves M > 64 tokens faster than the prefill GEMM. Costs in us from
// measured times on MI355X: a round of 256 wide workgroups takes about 4 us
// per 4096 of K (its per-CU x and weight reads); a prefill round of 256 x 192
// tiles about 85 us per 4096 of K.
bool wide_cheaper(int64_t m, int64_t n, int64_t k) {
  const int64_t cus = device_cus();
  const int64_t wide_groups = ((n / 32 + 7) / 8) * 8 * ((m + 31) / 32);
  const double wide_us = double((wide_groups + cus - 1) / cus) * 4.0 * double(k) / 4096.0;
  const int64_t tiles = ((m + 255) / 256) * ((n + 191) / 192);
  const double prefill_us = double((tiles + cus - 1) / cus) * 85.0 * double(k) / 4096.0;
  return wide_us < prefill_us;
}

// Whether M > 64 tokens are served faster by the decode kernel over 64-token
// chunks than by one prefill launch. The prefill GEMM runs 256 x 192 tiles,
// one workgroup per CU, so a call with fewer tiles than CUs leaves the rest
// of the chip idle (c4: 256 tokens x 4096 features are 22 tiles on 256 CUs);
// each decode chunk streams W again but uses every CU. Costs in us, from
// measured times on MI355X: a decode launch of 64 tokens streams its weight
// bytes (packed + fp32 scales) at about 0.8 TB/s, plus about 6 us with LoRA
// (4096 x 4096: 11.9 us base only, 18.0 us with 32 rank-16 adapters); a
// prefill round of tiles takes about 85 us per 4096 of K (c5: 1.81 rounds in
// 189 us; c4: one round of 22 tiles in 77 us), plus about 20 us with LoRA.
bool decode_chunks_cheaper(int64_t m, int64_t n, int64_t k, bool lora) {
  const double weight_bytes = double(n) * double(k) * (0.5 + 4.0 / 64.0);
  const double chunk_us = (lora ? 6.0 : 0.0) + weight_bytes / 0.8e6;
  const int64_t chunks = (m + kDecodeMaxTokens - 1) / kDecodeMaxTokens;
  const int64_t tiles = ((m + 255) / 256) * ((n + 191) / 192);
  const int64_t cus = device_cus();
  const int64_t rounds = (tiles + cus - 1) / cus;
  const double prefill_us = double(rounds) * 85.0 * double(k) / 4096.0 + (lora ? 20.0 : 0.0);
  return double(chunks) * chunk_us < prefill_us;
}
// One decode launch of up to 64 tokens: the wide kernel for the batches and
// shapes it takes (above 8 tokens, above 2 at N >= 8192, above 16 at
// K > 8192), else the narrow one (the kernel a direct call of these rows
// would use, so each chunk of the chunked plan equals that call).
int launch_decode(const uint16_t* x, int64_t m, int64_t x_stride, const lf_nf4_weight* w, const uint16_t* bias,
                  const lf_lora* lora, uint16_t* y, int64_t y_stride, void* workspace, int64_t workspace_bytes,
                  bool exact, bool swiglu, bool withhold, void* stream) {
  if (decode_wide_fits(m, w->n, w->k, lora))
    return launch_decode_wide(x, m, x_stride, w, bias, lora, y, y_stride, workspace, workspace_bytes, exact, swiglu,
                              withhold, stream);
  return launch_nf4_gemv(x, m, x_stride, w, bias, lora, y, y_stride, workspace, workspace_bytes, exact, swiglu,
                         withhold, stream);
}
}  // namespace lf

extern "C" int64_t lf_nf4_lora_workspace_size(int64_t m, int64_t n, int64_t k, int32_t num_slices,
                                              int32_t max_rank) {
  if (m < 0 || n <= 0 || k <= 0 || num_slices < 1 || max_rank < 1) return -1;
  if (m <= lf::kDecodeMaxTokens) return lf::gemv_workspace_bytes(m, n, k, num_slices, max_rank);
  return lf::prefill_workspace_bytes(m, n, k, num_slices, max_rank);
}

extern "C" int lf_nf4_lora_linear(const uint16_t* x, int64_t m, int64_t x_stride, const lf_nf4_weight* w,
                                  const uint16_t* bias, const lf_lora* lora, uint16_t* y, int64_t y_stride,
                                  void* workspace, int64_t workspace_bytes, int32_t flags, void* stream) {
  LF_REQUIRE(w != nullptr, "weight descriptor required");
  LF_REQUIRE((flags & ~(LF_EXACT_WEIGHTS | LF_SWIGLU_OUTPUT | LF_PLAN_DECODE_CHUNKS | LF_PLAN_PREFILL |
                        LF_TEST_WITHHOLD_PARTIALS)) == 0,
             "unknown flags");
  LF_REQUIRE((flags & (LF_PLAN_DECODE_CHUNKS | LF_PLAN_PREFILL)) != (LF_PLAN_DECODE_CHUNKS | LF_PLAN_PREFILL),
             "LF_PLAN_DECODE_CHUNKS and LF_PLAN_PREFILL exclude each other");
  const bool withhold = (flags & LF_TEST_WITHHOLD_PARTIALS) != 0;
  const bool swiglu = (flags & LF_SWIGLU_OUTPUT) != 0;
  LF_REQUIRE(m >= 0 && m < (int64_t(1) << 31), "token count out of range");
  const int64_t n = w->n, k = w->k;
  LF_REQUIRE(n > 0 && k > 0 && n % 64 == 0 && k % 64 == 0, "weight shape must contain two positive multiples of 64");
  LF_REQUIRE(n < (int64_t(1) << 28) && k < (int64_t(1) << 28), "weight shape too large");
  if (m == 0) return lf::kOk;
  LF_REQUIRE(x && y && w->qweight && w->code, "null pointer argument");
  LF_REQUIRE(w->scales || (w->absmax_q && w->absmax2 && w->code2 && w->offset && w->dq_block > 0),
             "scales or a complete double-quant state required");
  LF_REQUIRE(lf::aligned16(x) && x_stride >= k && x_stride % 8 == 0, "x must be 16-byte aligned with row stride %% 8 == 0");
  LF_REQUIRE(lf::aligned16(w->qweight), "packed weight must be 16-byte aligned");
  LF_REQUIRE(y_stride >= (swiglu ? n / 2 : n), "output row stride must cover the output width");
  LF_REQUIRE(!swiglu || n % 64 == 0, "SwiGLU output needs N a multiple of 64");
  LF_REQUIRE(!swiglu || !lora || lora->num_slices == 2, "SwiGLU output with LoRA needs the two gate/up slices");
  if (lora) {
    LF_REQUIRE(lora->num_slices >= 1 && lora->num_slices <= 3, "num_slices must be in 1..3");
    LF_REQUIRE(lora->max_rank >= 1 && lora->max_rank <= 64, "max_rank must be in 1..64");
    LF_REQUIRE(lora->a_store && lora->a_offsets && lora->b_store && lora->b_offsets && lora->b_strides &&
                   lora->ranks && lora->scales && lora->token_slots && lora->slice_offsets,
               "incomplete LoRA descriptor");
    LF_REQUIRE(lf::aligned16(lora->a_store) && lf::aligned16(lora->b_store), "A/B stores must be 16-byte aligned");
  }
  const bool exact = (flags & LF_EXACT_WEIGHTS) != 0;
  // Above 8 tokens (2 at N >= 8192, 16 at K > 8192): the wide decode kernel
  // (one launch, base linear with or without LoRA and the SwiGLU output),
  // unless the prefill GEMM is forced or cheaper, or the shape is outside the
  // kernel's range.
  if (lf::decode_wide_fits(m, n, k, lora) && !(flags & LF_PLAN_PREFILL) &&
      (m <= lf::kDecodeMaxTokens || (flags & LF_PLAN_DECODE_CHUNKS) || lf::wide_cheaper(m, n, k)))
    return lf::launch_decode_wide(x, m, x_stride, w, bias, lora, y, y_stride, workspace, workspace_bytes, exact,
                                  swiglu, withhold, stream);
  if (m <= lf::kDecodeMaxTokens)
    return lf::launch_decode(x, m, x_stride, w, bias, lora, y, y_stride, workspace, workspace_bytes, exact, swiglu,
                             withhold, stream);
  bool chunked = false;
  if (flags & LF_PLAN_DECODE_CHUNKS) chunked = true;
  else if (!(flags & LF_PLAN_PREFILL)) chunked = lf::decode_chunks_cheaper(m, n, k, lora != nullptr);
  if (!chunked)
    return lf::launch_nf4_lora_prefill(x, m, x_stride, w, bias, lora, y, y_stride, workspace, workspace_bytes,
                                       swiglu, withhold, stream);
  // 64-token chunks in token order on the caller's stream; each is one decode
  // launch over its rows of x, y and the token routes. A nested state that a
  // chunk's kernel does not read itself is rebuilt to fp32 scales once, ahead
  // of the chunks.
  lf_nf4_weight wc = *w;
  if (!w->scales) {
    const int64_t last = m - (m - 1) / lf::kDecodeMaxTokens * lf::kDecodeMaxTokens;
    auto reads = [&](int64_t mc) {
      return lf::decode_wide_fits(mc, n, k, lora) ? lf::wide_takes_dq(w) : lf::gemv_takes_dq(mc, w, lora, exact);
    };
    if (!reads(lf::kDecodeMaxTokens) || !reads(last)) {
      const int rc = lf::rebuild_decode_scales(w, workspace, workspace_bytes, stream, &wc.scales);
      if (rc != lf::kOk) return rc;
    }
  }
  w = &wc;
  for (int64_t t0 = 0; t0 < m; t0 += lf::kDecodeMaxTokens) {
    const int64_t mc = std::min<int64_t>(lf::kDecodeMaxTokens, m - t0);
    lf_lora part{};
    if (lora) {
      part = *lora;
      part.token_slots = lora->token_slots + t0;
    }
    const int rc = lf::launch_decode(x + t0 * x_stride, mc, x_stride, w, bias, lora ? &part : nullptr,
                                     y + t0 * y_stride, y_stride, workspace, workspace_bytes, exact, swiglu, withhold,
                                     stream);
    if (rc != lf::kOk) return rc;
  }
  return lf::kOk;
}

extern "C" int lf_nf4_lora_status(const void* workspace, void* stream, int32_t* status) {
  LF_REQUIRE(workspace && status, "null pointer argument");
  auto s = static_cast<hipStream_t>(stream);
  LF_HIP(hipMemcpyAsync(status, static_cast<const char*>(workspace) + 8, 4, hipMemcpyDeviceToHost, s));
  LF_HIP(hipStreamSynchronize(s));
  return lf::kOk;
}

extern "C" int lf_lora_apply(const uint16_t* x, int64_t m, int64_t x_stride, int64_t n, int64_t k, const lf_lora* lora,
                             uint16_t* y, int64_t y_stride, void* workspace, int64_t workspace_bytes, int32_t flags,
                             void* stream) {
  LF_REQUIRE((flags & ~LF_TEST_WITHHOLD_PARTIALS) == 0, "unknown flags");
  LF_REQUIRE(m >= 0 && m < (int64_t(1) << 31), "token count out of range");
  LF_REQUIRE(n > 0 && k > 0 && n % 64 == 0 && k % 64 == 0, "N and K must be positive multiples of 64");
  LF_REQUIRE(n < (int64_t(1) << 28) && k < (int64_t(1) << 28), "shape too large");
  if (m == 0) return lf::kOk;
  LF_REQUIRE(x && y && lora, "null pointer argument");
  LF_REQUIRE(lf::aligned16(x) && x_stride >= k && x_stride % 8 == 0, "x must be 16-byte aligned with row stride %% 8 == 0");
  LF_REQUIRE(y_stride >= n, "output row stride must cover the output width");
  LF_REQUIRE(lora->num_slices >= 1 && lora->num_slices <= 3, "num_slices must be in 1..3");
  LF_REQUIRE(lora->max_rank >= 1 && lora->max_rank <= 64, "max_rank must be in 1..64");
  LF_REQUIRE(lora->a_store && lora->a_offsets && lora->b_store && lora->b_offsets && lora->b_strides && lora->ranks &&
                 lora->scales && lora->token_slots && lora->slice_offsets,
             "incomplete LoRA descriptor");
  LF_REQUIRE(lf::aligned16(lora->a_store) && lf::aligned16(lora->b_store), "A/B stores must be 16-byte aligned");
  lf_nf4_weight shape{};
  shape.n = n;
  shape.k = k;
  const bool withhold = (flags & LF_TEST_WITHHOLD_PARTIALS) != 0;
  // One launch per 64 tokens, in token order.
  for (int64_t t0 = 0; t0 < m; t0 += lf::kDecodeMaxTokens) {
    const int64_t mc = std::min<int64_t>(lf::kDecodeMaxTokens, m - t0);
    lf_lora part = *lora;
    part.token_slots = lora->token_slots + t0;
    // 33..64 tokens: the wide kernel's residual form where it fits.
    const int rc = lf::lora_apply_wide_fits(mc, n, k, &part)
                       ? lf::launch_lora_apply_wide(x + t0 * x_stride, mc, x_stride, n, k, &part, y + t0 * y_stride,
                                                    y_stride, workspace, workspace_bytes, withhold, stream)
                       : lf::launch_nf4_gemv(x + t0 * x_stride, mc, x_stride, &shape, nullptr, &part, y + t0 * y_stride,
                                             y_stride, workspace, workspace_bytes, false, false, withhold, stream, true);
    if (rc != lf::kOk) return rc;
  }
  return lf::kOk;
}
