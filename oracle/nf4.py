"""NF4 restatement in numpy. TEST INFRASTRUCTURE ONLY (see ``oracle/__init__``).

Reference behaviour restated here:

* Element ``e`` of a row-major ``[N, K]`` weight lives in byte ``e // 2`` of the
  packed vector; even elements take the high nibble, odd elements the low one
  (``src/loraforge/ops/_nf4_kernels.py:31-32,52-60``, ``ops/nf4.py:47-49``).
* ``W[e] = bf16_RNE(fp32(code[nibble]) * fp32(scale[e // 64]))`` -- one fp32
  multiply, no FMA contraction (``_nf4_kernels.py:33-35,55-59``,
  ``ops/nf4.py:27`` ``enable_fp_fusion=False``).
* The canonical codebook is the 16 fp32 literals of ``ops/nf4.py:120-141``.
* Double quantisation (``ops/nf4.py:144-147``): ``scale[j] =
  fl32(fl32(code2[absmax_q[j]] * absmax2[j // 256]) + offset)``, the
  bitsandbytes ``dequantize_blockwise`` + ``offset`` order of operations.

Pinning (tests/test_oracle_nf4.py): the codebook literals against the
reference text; closed-form special cases (zero block, code 7 = 0, codes 0/15
= -/+ absmax, the nibble order of hand-built bytes, a round-to-nearest-even
tie); exhaustive enumeration of all 256 byte values against an independent
torch-CPU evaluation; and quantise -> dequantise round trips.
``dynamic_map`` is "parity unpinned" against bitsandbytes (absent offline).
"""

from __future__ import annotations

import numpy as np

# ops/nf4.py:120-141 (the canonical NF4 table checked by prepare_scales).
NF4_CODE = np.array(
    [
        -1.0,
        -0.6961928009986877,
        -0.5250730514526367,
        -0.39491748809814453,
        -0.28444138169288635,
        -0.18477343022823334,
        -0.09105003625154495,
        0.0,
        0.07958029955625534,
        0.16093020117282867,
        0.24611230194568634,
        0.33791524171829224,
        0.44070982933044434,
        0.5626170039176941,
        0.7229568362236023,
        1.0,
    ],
    dtype=np.float32,
)

BLOCK = 64
DQ_BLOCK = 256


def bf16_bits(values, *, nan: str = "quiet") -> np.ndarray:
    """fp32 -> bf16 bit patterns with round-to-nearest-even.

    ``nan="quiet"`` maps NaN to a quiet NaN (Triton's ``.to(tl.bfloat16)``);
    ``nan="truncate"`` keeps the high half unrounded for Inf/NaN exactly as
    ``round_bf16`` does (``ops/csrc/lora_rows.cu:27-33``).
    """
    arr = np.asarray(values, dtype=np.float32)
    u = np.ascontiguousarray(arr).reshape(-1).view(np.uint32)
    special = (u & 0x7F800000) == 0x7F800000
    rounded = (u + (0x7FFF + ((u >> 16) & 1))) & 0xFFFFFFFF
    out = np.where(special, u, rounded) >> 16
    if nan == "quiet":
        is_nan = special & ((u & 0x007FFFFF) != 0)
        out = np.where(is_nan, (u >> 16) | 0x0040, out)
    return out.astype(np.uint16).reshape(arr.shape)


def bf16_to_f32(bits) -> np.ndarray:
    """bf16 bit patterns -> fp32 (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_f32(values) -> np.ndarray:
    """Round fp32 to the nearest bf16 and return it as fp32."""
    return bf16_to_f32(bf16_bits(values))


def f64_to_bf16_bits(values) -> np.ndarray:
    """float64 -> fp32 -> bf16, the double rounding of torch's ``.bfloat16()``."""
    return bf16_bits(np.asarray(values, dtype=np.float64).astype(np.float32))


def unpack_nibbles(qweight) -> np.ndarray:
    """Packed bytes -> nibble per element, high nibble first (``_nf4_kernels.py:32``)."""
    q = np.asarray(qweight, dtype=np.uint8).reshape(-1)
    out = np.empty(q.size * 2, dtype=np.uint8)
    out[0::2] = q >> 4
    out[1::2] = q & 0x0F
    return out


def pack_nibbles(nibbles) -> np.ndarray:
    n = np.asarray(nibbles, dtype=np.uint8).reshape(-1)
    if n.size % 2:
        raise ValueError("element count must be even")
    return ((n[0::2] << 4) | (n[1::2] & 0x0F)).astype(np.uint8)


def dq_scales(absmax_q, absmax2, code2, offset, *, dq_block: int = DQ_BLOCK) -> np.ndarray:
    """Double-quantised absmax -> fp32 block scales (``ops/nf4.py:144-147``)."""
    q = np.asarray(absmax_q, dtype=np.uint8).reshape(-1)
    a2 = np.asarray(absmax2, dtype=np.float32).reshape(-1)
    c2 = np.asarray(code2, dtype=np.float32).reshape(-1)
    if c2.size != 256:
        raise ValueError("code2 must hold 256 entries")
    if a2.size != -(-q.size // dq_block):
        raise ValueError("absmax2 must hold one scale per dq block")
    blockwise = (c2[q] * a2[np.arange(q.size) // dq_block]).astype(np.float32)
    return (blockwise + np.float32(offset)).astype(np.float32)


def dequantize(qweight, scales, shape, code=NF4_CODE) -> np.ndarray:
    """Packed NF4 + fp32 block scales -> bf16 bits ``[N, K]`` (``_nf4_kernels.py:44-61``)."""
    n, k = shape
    if n <= 0 or k <= 0 or n % BLOCK or k % BLOCK:
        raise ValueError("shape must contain two positive multiples of 64")
    nib = unpack_nibbles(qweight)
    s = np.asarray(scales, dtype=np.float32).reshape(-1)
    if nib.size != n * k or s.size != n * k // BLOCK:
        raise ValueError("packed/scales sizes disagree with shape")
    values = np.asarray(code, dtype=np.float32)[nib] * np.repeat(s, BLOCK)
    return bf16_bits(values.astype(np.float32)).reshape(n, k)


def linspace_f32(start: float, end: float, steps: int) -> np.ndarray:
    """fp32 linspace with the two-sided evaluation torch's CPU kernel uses.

    ``start + step * i`` below the midpoint and ``end - step * (steps - 1 - i)``
    above it, each rounded once (fused multiply-add; the float64 product of
    two fp32 values is exact).
    """
    start32, end32 = np.float32(start), np.float32(end)
    step = np.float32((end32 - start32) / np.float32(steps - 1))
    idx = np.arange(steps)
    half = steps // 2
    lo = (np.float64(start32) + np.float64(step) * idx).astype(np.float32)
    hi = (np.float64(end32) - np.float64(step) * (steps - idx - 1)).astype(np.float32)
    return np.where(idx < half, lo, hi).astype(np.float32)


def dynamic_map() -> np.ndarray:
    """Signed 8-bit dynamic code table (bitsandbytes ``create_dynamic_map``).

    Parity unpinned: bitsandbytes 0.50.2 (the reference's pinned dependency,
    ``integrations/sglang_experimental.py:54-55``) is not installed, so the
    exact fp32 entries it produces cannot be compared here. The kernels take
    ``code2`` as an input, so only synthetic inputs depend on this table.
    Properties pinned by tests: 256 sorted entries, contains 0 and 1, and
    seven decades of +/- means.
    """
    data: list[float] = []
    for i in range(7):
        bounds = linspace_f32(0.1, 1.0, 2**i + 1)
        means = ((bounds[:-1] + bounds[1:]) / np.float32(2)).astype(np.float32)
        decade = np.float32(10.0 ** (i - 6))
        data += (decade * means).astype(np.float32).tolist()
        data += (-decade * means).astype(np.float32).tolist()
    data += [0.0, 1.0]
    return np.sort(np.array(data, dtype=np.float32))


def nf4_nearest(normalised) -> np.ndarray:
    """Nearest NF4 code index of values in [-1, 1] (ties go to the upper code)."""
    mids = ((NF4_CODE[:-1].astype(np.float64) + NF4_CODE[1:]) / 2).astype(np.float32)
    return np.searchsorted(mids, np.asarray(normalised, dtype=np.float32), side="right").astype(np.uint8)


def quantize(weight, *, blocksize: int = BLOCK, double_quant: bool = False, dq_block: int = DQ_BLOCK) -> dict:
    """Input generator: bf16-valued fp32 weight ``[N, K]`` -> NF4 state dict.

    Mirrors the bitsandbytes ``quantize_4bit(blocksize=64, quant_type="nf4",
    compress_statistics=...)`` recipe used by the reference fixtures
    (``benchmarks/prepare_qwen35_nf4.py:40-42``). Nearest-code choice affects
    only which inputs are generated, never dequantisation exactness.
    """
    w = np.asarray(weight, dtype=np.float32)
    n, k = w.shape
    if blocksize != BLOCK:
        raise ValueError("only blocksize 64 is supported")
    blocks = w.reshape(-1, blocksize)
    absmax = np.abs(blocks).max(axis=1).astype(np.float32)
    safe = np.where(absmax > 0, absmax, np.float32(1))
    normalised = (blocks * (np.float32(1) / safe)[:, None]).astype(np.float32)
    codes = np.where(absmax[:, None] > 0, nf4_nearest(normalised), np.uint8(7))
    state = {
        "qweight": pack_nibbles(codes.reshape(-1)),
        "shape": (n, k),
        "blocksize": blocksize,
        "code": NF4_CODE.copy(),
    }
    if not double_quant:
        state["absmax"] = absmax
        state["scales"] = absmax
        return state
    offset = np.float32(absmax.mean(dtype=np.float64))
    centred = (absmax - offset).astype(np.float32)
    nb2 = -(-centred.size // dq_block)
    padded = np.zeros(nb2 * dq_block, dtype=np.float32)
    padded[: centred.size] = centred
    absmax2 = np.abs(padded.reshape(nb2, dq_block)).max(axis=1).astype(np.float32)
    safe2 = np.where(absmax2 > 0, absmax2, np.float32(1))
    code2 = dynamic_map()
    norm2 = (centred / np.repeat(safe2, dq_block)[: centred.size]).astype(np.float32)
    idx = np.searchsorted(code2, norm2).clip(1, 255)
    lower = code2[idx - 1]
    upper = code2[idx]
    absmax_q = np.where(np.abs(norm2 - lower) <= np.abs(upper - norm2), idx - 1, idx).astype(np.uint8)
    state.update(
        absmax_q=absmax_q,
        absmax2=absmax2,
        code2=code2,
        offset=offset,
        dq_block=dq_block,
        scales=dq_scales(absmax_q, absmax2, code2, offset, dq_block=dq_block),
    )
    return state
