"""Fused NF4 base linear + per-token multi-LoRA (decode and prefill) on gfx950.

This is the one-call replacement for the reference's three-step serving path
of a quantised projection with LoRA:

* ``integrations/_sglang_nf4_linear.py:116-129``: ``dequantize`` -> ``F.linear``
  -> ``+ bias`` (bf16 result, fp32 accumulation);
* ``ops/rowexpand.py:34-39`` / ``ops/lora_rows.py:54``: shrink ``z = bf16(A_g x)``;
* ``ops/rowexpand.py:42-92`` / ``ops/lora_rows.py:115``: expand
  ``y = bf16(y + bf16(scale_g * B_g z))``.

The adapters are described by a ``LoraBatch`` in the same compact layout the
reference's row operators use (per-slot A rows packed at ``s * r``, compact B
regions of ``[N, b_strides[g]]`` at ``b_offsets[g]``), with a per-token slot
map instead of segments (segments expand to it, see ``segments_to_slots``).
Decode batches (<= 64 tokens) run as one kernel launch; prefill runs an MFMA
GEMM with the LoRA delta applied in its epilogue.
"""

from __future__ import annotations

import threading
from dataclasses import dataclass

from .. import _lib
from ..annotations import ExperimentalAPI
from ._checks import distinct_output, require_arch, tensor, vector

_WS_LOCK = threading.Lock()
_WORKSPACES: dict = {}
_RETIRED: list = []  # replaced workspaces a captured graph may still address


@dataclass
class LoraBatch:
    """Device-resident adapter table plus the per-token routing of one call.

    a_store/b_store: flat bf16 stores (16-byte aligned); a_offsets/b_offsets:
    int64 element offsets per slot (multiples of 8); b_strides: int32 power of
    two in 1..64 (>= rank); ranks: int32; scales: fp32 (alpha/r or
    alpha/sqrt(r)); token_slots: int32 per token (-1 = base only);
    slice_offsets: int32 partition of the output columns (1..3 slices).
    Slot g's A has ``num_slices * ranks[g]`` rows of width K.
    """

    a_store: object
    a_offsets: object
    b_store: object
    b_offsets: object
    b_strides: object
    ranks: object
    scales: object
    token_slots: object
    slice_offsets: object
    max_rank: int = 64

    @property
    def num_slices(self) -> int:
        return self.slice_offsets.numel() - 1

    @classmethod
    def from_padded(cls, a, b, *, b_offsets, b_strides, ranks, scales, token_slots, slice_offsets, max_rank=64):
        """Wrap the row-operator layout: ``a`` is ``[G, slices * capacity, K]``."""
        import torch

        slots, rows, width = a.shape
        a_offsets = torch.arange(slots, dtype=torch.int64, device=a.device) * (rows * width)
        return cls(a.reshape(-1), a_offsets, b, b_offsets, b_strides, ranks, scales, token_slots, slice_offsets, max_rank)

    def with_tokens(self, token_slots) -> "LoraBatch":
        return LoraBatch(
            self.a_store,
            self.a_offsets,
            self.b_store,
            self.b_offsets,
            self.b_strides,
            self.ranks,
            self.scales,
            token_slots,
            self.slice_offsets,
            self.max_rank,
        )


def segments_to_slots(segment_lengths, segment_slots, device=None):
    """Contiguous prefill segments -> int32 per-token slot map."""
    import torch

    lengths = torch.as_tensor(segment_lengths, dtype=torch.int64)
    slots = torch.as_tensor(segment_slots, dtype=torch.int32)
    return torch.repeat_interleave(slots, lengths).to(device=device)


def workspace_bytes(m: int, n: int, k: int, *, num_slices: int = 1, max_rank: int = 64) -> int:
    size = _lib.library().lf_nf4_lora_workspace_size(m, n, k, num_slices, max_rank)
    if size < 0:
        raise ValueError("invalid problem size")
    return int(size)


def _workspace(device, stream: int, size: int, kind: str = "fused"):
    """The cached workspace of (device, stream), grown to ``size`` bytes.

    ``kind`` keeps the fused linear's and the row shrink's buffers apart.

    A HIP graph captured earlier keeps the raw address of the buffer it was
    captured with and writes its z rows, flags and call epoch there on every
    replay, so a replaced buffer is never released: it moves to ``_RETIRED``
    and stays allocated until the process ends.
    """
    import torch

    key = (device.index, stream) if kind == "fused" else (kind, device.index, stream)
    with _WS_LOCK:
        ws = _WORKSPACES.get(key)
        if ws is None or ws.numel() < size:
            if torch.cuda.is_current_stream_capturing() and kind == "fused":
                raise RuntimeError("warm nf4_lora_linear on this stream before graph capture")
            # (A row-shrink workspace may be made under capture: it comes from the
            # graph's pool and its zero fill is a kernel of the graph, so every
            # replay starts from a zeroed workspace, which the tags allow.)
            if ws is not None:
                _RETIRED.append(ws)
            ws = torch.zeros(max(size, 1 << 20), dtype=torch.uint8, device=device)
            _WORKSPACES[key] = ws
        return ws


def _kernel_takes_nested(m: int, exact: bool, plan: str | None = None) -> bool:
    """Whether a call for ``m`` tokens with ``scales=None`` passes a nested state to the library.

    Decode calls (and the chunked decode plan) take the prepared scales,
    rebuilt once per weight and cached on the state: the decode kernels can
    read the nested state themselves (``scales="nested"``), but converting it
    costs each workgroup about 1.3 us before its weight loop, more than the
    3 bytes per 64 weights it saves. The prefill launch rebuilds fp32 scales
    into its workspace on every call; by default calls above 64 tokens also
    take the cached scales (no per-call rebuild), and ``exact=True`` passes
    the nested state, which keeps them on the prefill GEMM's exact weights.
    """
    return m > 64 and exact and plan != "decode"


def _version(tensor):
    try:
        return tensor._version
    except RuntimeError:  # tensors made under inference_mode carry no version counter
        return None


def scale_key(qweight, state):
    """Version key of a state's prepared scales.

    Mirrors ``integrations/_sglang_nf4_linear.py:44-57``: the state's identity
    plus the address and version counter of the packed weight, the absmax,
    the codebook and, for a nested state, the second-level absmax/code and
    the offset. Contents changed outside PyTorch's versioned updates are not
    seen (as in the reference).
    """
    tensors = [qweight, state.absmax, state.code]
    if state.nested:
        tensors += [state.state2.absmax, state.state2.code, state.offset]
    return (id(state), tuple((t.data_ptr(), _version(t)) for t in tensors))


def _prepared_scales(qweight, state):
    """fp32 scales of a nested state, rebuilt whenever its version key changes."""
    from loraforge_amd.ops.nf4 import prepare_scales

    key = scale_key(qweight, state)
    cached = getattr(state, "_lf_prepared_scales", None)
    if cached is None or cached[0] != key:
        import torch

        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("warm nf4_lora_linear with this weight before graph capture")
        cached = (key, prepare_scales(state))
        state._lf_prepared_scales = cached
    return cached[1]


def _weight_struct(qweight, state, scales, n, k, device, m=0, exact=False, plan=None):
    import torch

    code = state.code
    if code.device != device or code.dtype != torch.float32 or code.numel() != 16 or not code.is_contiguous():
        raise ValueError("code must be a contiguous 16-entry FP32 codebook on the input device")
    w = _lib.NF4Weight()
    w.qweight = qweight.data_ptr()
    w.code = code.data_ptr()
    w.n = n
    w.k = k
    keep = [qweight, code]
    if scales is None and not state.nested:
        scales = state.absmax
    if isinstance(scales, str):
        if scales != "nested" or not state.nested:
            raise ValueError('scales="nested" needs a double-quant (nested) state')
        scales = None
    elif scales is None and not _kernel_takes_nested(m, exact, plan):
        scales = _prepared_scales(qweight, state)
    if scales is not None:
        vector(scales.reshape(-1), "scales", torch.float32, device, n * k // 64)
        w.scales = scales.data_ptr()
        keep.append(scales)
        return w, keep
    absmax = state.absmax
    s2 = state.state2
    if (
        absmax.dtype != torch.uint8
        or absmax.numel() != n * k // 64
        or not absmax.is_contiguous()
        or s2.absmax.dtype != torch.float32
        or not s2.absmax.is_contiguous()
        or s2.absmax.numel() != -(-absmax.numel() // s2.blocksize)
        or s2.code.dtype != torch.float32
        or s2.code.numel() != 256
        or state.offset.dtype != torch.float32
        or any(t.device != device for t in (absmax, s2.absmax, s2.code, state.offset))
    ):
        raise ValueError("double-quant state must be uint8 absmax + fp32 absmax2/code2/offset on the input device")
    w.absmax_q = absmax.data_ptr()
    w.absmax2 = s2.absmax.data_ptr()
    w.code2 = s2.code.data_ptr()
    w.offset = state.offset.data_ptr()
    w.dq_block = int(s2.blocksize)
    keep += [absmax, s2.absmax, s2.code, state.offset]
    return w, keep


def _lora_struct(lora: LoraBatch, m: int, k: int, n: int, device):
    import torch

    if type(lora.max_rank) is not int or not 1 <= lora.max_rank <= 64:
        raise ValueError("max_rank must be in 1..64")
    tensor(lora.a_store, "a_store", 1, torch.bfloat16, device)
    tensor(lora.b_store, "b_store", 1, torch.bfloat16, device)
    vector(lora.ranks, "ranks", torch.int32, device)
    g = lora.ranks.numel()
    vector(lora.a_offsets, "a_offsets", torch.int64, device, g)
    vector(lora.b_offsets, "b_offsets", torch.int64, device, g)
    vector(lora.b_strides, "b_strides", torch.int32, device, g)
    vector(lora.scales, "scales", torch.float32, device, g)
    vector(lora.token_slots, "token_slots", torch.int32, device, m)
    vector(lora.slice_offsets, "slice_offsets", torch.int32, device)
    if not 1 <= lora.num_slices <= 3:
        raise ValueError("num_slices must be in 1..3")
    if not lora.a_store.is_contiguous() or not lora.b_store.is_contiguous():
        raise ValueError("A/B stores must be contiguous")
    if lora.a_store.data_ptr() % 16 or lora.b_store.data_ptr() % 16:
        raise ValueError("A/B stores must be 16-byte aligned")
    s = _lib.Lora()
    s.a_store = lora.a_store.data_ptr()
    s.a_offsets = lora.a_offsets.data_ptr()
    s.b_store = lora.b_store.data_ptr()
    s.b_offsets = lora.b_offsets.data_ptr()
    s.b_strides = lora.b_strides.data_ptr()
    s.ranks = lora.ranks.data_ptr()
    s.scales = lora.scales.data_ptr()
    s.token_slots = lora.token_slots.data_ptr()
    s.slice_offsets = lora.slice_offsets.data_ptr()
    s.num_slices = lora.num_slices
    s.max_rank = lora.max_rank
    s.num_slots = g
    return s


@ExperimentalAPI(reason="gfx950 fused NF4 + multi-LoRA linear; caller-owned device metadata.")
def nf4_lora_linear(
    x,
    qweight,
    state,
    *,
    scales=None,
    bias=None,
    lora: LoraBatch | None = None,
    out=None,
    workspace=None,
    exact=False,
    swiglu=False,
    plan=None,
):
    """``y = bf16(x @ dequant(W)^T) (+bias)``, then the per-token LoRA delta.

    x: bf16 ``[..., K]`` with unit column stride. qweight: packed uint8
    ``N*K/2`` (high nibble first). state: NF4 state (``NF4State`` or a
    bitsandbytes ``QuantState``); ``scales`` (fp32 ``N*K/64``, e.g. from
    ``prepare_scales``) overrides its absmax. For a nested (double-quant)
    state, ``scales=None`` uses fp32 scales prepared once per weight and
    cached on the state (the faster decode), and ``scales="nested"`` hands
    the library the nested state itself: the decode kernels stage the uint8
    codes into LDS and convert them there (no fp32 scales resident, 1 byte
    per 64 weights read instead of 4, about 1.3 us more per workgroup), and
    the prefill GEMM rebuilds fp32 scales into its workspace per call. Returns bf16 ``[..., N]`` (``out`` if given).
    Launches on the current stream; the workspace (cached per device and
    stream unless passed) must not be shared by overlapping calls.

    The prefill GEMM (more than 64 tokens) always multiplies the reference's
    dequantised weights ``bf16_rne(code * scale)``. By default the decode
    kernel (<= 64 tokens) contracts ``bf16(code[nibble])`` on MFMA and applies
    each fp32 block scale to the block's partial sum; ``exact=True`` makes it
    multiply the exact weights too (bit-identical W, slower).

    ``swiglu=True``: the weight is a merged gate/up projection (gate rows
    ``0 .. N/2``, up rows ``N/2 .. N``; with LoRA, slices ``[0, N/2, N]``) and
    the result is ``h = bf16(bf16(silu(gate)) * up)``, ``[..., N/2]``, of the
    LoRA-updated bf16 gate and up outputs, computed in the epilogue of the
    decode kernels and of the prefill GEMM (no gate/up round trip, no second
    launch); above 64 tokens into an ``out`` whose rows are not 16-byte
    aligned, the linear and then ``silu_mul``.

    Above 64 tokens the library picks the prefill GEMM or the decode kernel
    over 64-token chunks (when the prefill tiles would leave most of the chip
    idle, e.g. 256 tokens x 4096 features); ``plan="prefill"`` or
    ``plan="decode"`` forces one (``None``: the library's cost model).
    """
    import torch

    if plan not in (None, "prefill", "decode"):
        raise ValueError("plan must be None, 'prefill' or 'decode'")
    if not isinstance(x, torch.Tensor) or not isinstance(qweight, torch.Tensor):
        raise TypeError("x and qweight must be tensors")
    if state.quant_type != "nf4" or state.blocksize != 64:
        raise ValueError("requires NF4 block64 weights")
    n, k = (int(v) for v in state.shape)
    if n <= 0 or k <= 0 or n % 64 or k % 64:
        raise ValueError("weight shape must contain two positive multiples of 64")
    device = x.device
    if x.dtype != torch.bfloat16 or x.shape[-1] != k or x.stride(-1) != 1:
        raise ValueError("x must be bf16 [..., K] with unit column stride")
    if x.requires_grad:
        raise ValueError("nf4_lora_linear is inference-only")
    if device.type != "cuda" or qweight.device != device:
        raise ValueError("all tensors must be on the same CUDA/ROCm GPU")
    if qweight.dtype != torch.uint8 or qweight.numel() != n * k // 2 or not qweight.is_contiguous():
        raise ValueError("qweight must be contiguous uint8 holding N*K/2 bytes")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, k)
    m = x2.shape[0]
    if x2.stride(0) < k or x2.stride(0) % 8 or x2.data_ptr() % 16 or qweight.data_ptr() % 16:
        raise ValueError("x rows must be 16-byte aligned with a stride multiple of 8; qweight 16-byte aligned")
    if bias is not None:
        vector(bias, "bias", torch.bfloat16, device, n)
    width = n
    if swiglu:
        if n % 32:
            raise ValueError("SwiGLU output needs N a multiple of 32")
        if lora is not None and lora.num_slices != 2:
            raise ValueError("SwiGLU output with LoRA needs the two gate/up slices")
        width = n // 2
        # The prefill GEMM stores the activation in 16-byte chunks: a caller's
        # output whose rows are not 16-byte aligned takes the linear and then
        # the activation above 64 tokens.
        unaligned = out is not None and (out.data_ptr() % 16 or (out.dim() > 1 and out.stride(-2) % 8))
        if m > 64 and unaligned:
            from .activation import silu_mul

            if out is not None:
                if out.dtype != torch.bfloat16 or out.shape != (*lead, width) or out.device != device or out.stride(-1) != 1:
                    raise ValueError("out must be bf16 [..., N/2] on the input device")
                distinct_output(out, (x, qweight, bias))
            gate_up = nf4_lora_linear(
                x2, qweight, state, scales=scales, bias=bias, lora=lora, workspace=workspace, exact=exact, plan=plan
            )
            h = silu_mul(gate_up, out=None if out is None else out.reshape(-1, width))
            return h.reshape(*lead, width) if out is None else out
    if out is None:
        out = torch.empty((*lead, width), dtype=torch.bfloat16, device=device)
    elif out.dtype != torch.bfloat16 or out.shape != (*lead, width) or out.device != device or out.stride(-1) != 1:
        raise ValueError(f"out must be bf16 [..., {'N/2' if swiglu else 'N'}] on the input device")
    y2 = out.reshape(-1, width)
    if y2.data_ptr() != out.data_ptr():
        raise ValueError("out must be viewable as [M, N]")
    distinct_output(out, (x, qweight, bias))
    if m == 0:
        return out
    require_arch(device)
    w, keep = _weight_struct(qweight, state, scales, n, k, device, m, exact, plan)
    lib = _lib.library()
    slices = lora.num_slices if lora is not None else 1
    max_rank = lora.max_rank if lora is not None else 1
    lstruct = _lora_struct(lora, m, k, n, device) if lora is not None else None
    if lora is not None and lora.slice_offsets.numel() - 1 != slices:
        raise ValueError("slice_offsets length disagrees with num_slices")
    with torch.cuda.device(device):
        stream = _lib.stream_of(device)
        need = workspace_bytes(m, n, k, num_slices=slices, max_rank=max_rank)
        if workspace is None:
            workspace = _workspace(device, stream, need)
        elif workspace.dtype != torch.uint8 or workspace.device != device or workspace.numel() < need:
            raise ValueError(f"workspace must be uint8 on the input device with at least {need} bytes")
        _lib.check(
            lib.lf_nf4_lora_linear(
                x2.data_ptr(),
                m,
                x2.stride(0),
                w,
                _lib.ptr(bias),
                lstruct,
                y2.data_ptr(),
                y2.stride(0),
                workspace.data_ptr(),
                workspace.numel(),
                (_lib.LF_EXACT_WEIGHTS if exact else 0)
                | (_lib.LF_SWIGLU_OUTPUT if swiglu else 0)
                | {None: 0, "decode": _lib.LF_PLAN_DECODE_CHUNKS, "prefill": _lib.LF_PLAN_PREFILL}[plan],
                stream,
            )
        )
    del keep
    return out


@ExperimentalAPI(reason="gfx950 one-launch row_shrink + row_expand; caller-owned device metadata.")
def lora_apply(x, y, lora: LoraBatch, *, workspace=None):
    """``y += LoRA(x)`` in place for every routed token, one launch per 64 tokens.

    The reference chain ``row_shrink`` then ``row_expand``
    (``ops/lora_rows.py:51-239``) without materialising z or building
    segments: token ``t`` routed to slot ``g`` gets
    ``y[t] = bf16(bf16(y[t]) + bf16(scale_g * bf16(x[t] A_g^T) B_g^T))`` per
    slice, tokens without an adapter keep their bits. x: bf16 ``[M, K]``;
    y: bf16 ``[M, N]`` (unit column stride); N and K multiples of 64. Runs on
    the current stream with the cached per-stream workspace unless one is
    passed. Returns ``y``.
    """
    import torch

    if not isinstance(x, torch.Tensor) or not isinstance(y, torch.Tensor):
        raise TypeError("x and y must be tensors")
    if not isinstance(lora, LoraBatch):
        raise TypeError("lora must be a LoraBatch")
    device = x.device
    if device.type != "cuda" or y.device != device:
        raise ValueError("all tensors must be on the same CUDA/ROCm GPU")
    if x.dtype != torch.bfloat16 or y.dtype != torch.bfloat16 or x.ndim != 2 or y.ndim != 2:
        raise ValueError("x and y must be bf16 matrices")
    if x.requires_grad or y.requires_grad:
        raise ValueError("lora_apply is inference-only")
    m, k = x.shape
    n = y.shape[1]
    if y.shape[0] != m:
        raise ValueError("x and y must have the same number of rows (tokens)")
    if n <= 0 or k <= 0 or n % 64 or k % 64:
        raise ValueError("N and K must be positive multiples of 64")
    if x.stride(1) != 1 or y.stride(1) != 1 or x.stride(0) % 8 or x.data_ptr() % 16:
        raise ValueError("x rows must be 16-byte aligned with a stride multiple of 8; unit column strides")
    distinct_output(y, (x,))
    if lora.slice_offsets.numel() - 1 != lora.num_slices:
        raise ValueError("slice_offsets length disagrees with num_slices")
    if m == 0:
        return y
    require_arch(device)
    lstruct = _lora_struct(lora, m, k, n, device)
    lib = _lib.library()
    with torch.cuda.device(device):
        stream = _lib.stream_of(device)
        need = workspace_bytes(min(m, 64), n, k, num_slices=lora.num_slices, max_rank=lora.max_rank)
        if workspace is None:
            workspace = _workspace(device, stream, need)
        elif workspace.dtype != torch.uint8 or workspace.device != device or workspace.numel() < need:
            raise ValueError(f"workspace must be uint8 on the input device with at least {need} bytes")
        _lib.check(
            lib.lf_lora_apply(
                x.data_ptr(), m, x.stride(0), n, k, lstruct, y.data_ptr(), y.stride(0),
                workspace.data_ptr(), workspace.numel(), 0, stream,
            )
        )
    return y


def decode_status(workspace=None, device=None) -> int:
    """Status word of the fused calls on a workspace (0 = ok; 1 = a wait for z gave up); synchronises."""
    import ctypes

    import torch

    device = torch.device(device or "cuda")
    if workspace is None:
        stream = _lib.stream_of(device)
        workspace = _WORKSPACES.get((device.index if device.index is not None else torch.cuda.current_device(), stream))
        if workspace is None:
            return 0
    value = ctypes.c_int32(0)
    _lib.check(_lib.library().lf_nf4_lora_status(workspace.data_ptr(), _lib.stream_of(workspace.device), ctypes.byref(value)))
    return int(value.value)
