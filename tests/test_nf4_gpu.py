"""NF4 dequantisation on gfx950 is bit-exact against the oracle (reference recipe:
``tests/test_nf4_gpu.py:10-48`` -- seed 731, ``randn * 0.1``, shapes
(64,64)/(1024,2048)/(8192,1024), graph replay, a side stream, alias rejection).
"""

import numpy as np
import pytest
import torch

from loraforge_amd.ops import dequantize_nf4, dequantize_nf4_nested, prepare_scales, quantize_nf4
from loraforge_amd.ops.nf4 import NF4State, NestedState
from oracle import nf4 as onf4
from tests import _cases

pytestmark = pytest.mark.gpu


def _state_tensors(state, device):
    code = torch.from_numpy(state["code"]).to(device)
    q = torch.from_numpy(state["qweight"]).to(device)
    if "absmax_q" not in state:
        st = NF4State(torch.from_numpy(state["absmax"]).to(device), torch.Size(state["shape"]), code, torch.bfloat16)
        return q, st
    nested = NestedState(torch.from_numpy(state["absmax2"]).to(device), torch.from_numpy(state["code2"]).to(device), 256)
    st = NF4State(
        torch.from_numpy(state["absmax_q"]).to(device),
        torch.Size(state["shape"]),
        code,
        torch.bfloat16,
        offset=torch.tensor(state["offset"], dtype=torch.float32, device=device),
        state2=nested,
    )
    return q, st


def _bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("shape", [(64, 64), (1024, 2048), (8192, 1024)])
def test_exact_reconstruction_graph_and_stream(shape, device):
    rng = np.random.default_rng(731)
    w = onf4.bf16_to_f32(_cases.bf16(rng.standard_normal(shape) * 0.1))
    state = onf4.quantize(w)
    expect = onf4.dequantize(state["qweight"], state["scales"], shape)
    q, st = _state_tensors(state, device)
    scales = prepare_scales(st)
    out = torch.empty(shape, dtype=torch.bfloat16, device=device)
    assert dequantize_nf4(q, scales, st.code, shape, out=out) is out
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out), expect)
    address = out.data_ptr()
    out.zero_()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        dequantize_nf4(q, scales, st.code, shape, out=out)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert out.data_ptr() == address and np.array_equal(_bits(out), expect)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        value = dequantize_nf4(q, scales, st.code, shape)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(value), expect)


@pytest.mark.parametrize("shape", [(64, 64), (1024, 2048)])
def test_double_quant_scales_and_in_kernel_reconstruction(shape, device):
    rng = np.random.default_rng(731)
    w = onf4.bf16_to_f32(_cases.bf16(rng.standard_normal(shape) * 0.1))
    state = onf4.quantize(w, double_quant=True)
    q, st = _state_tensors(state, device)
    scales = prepare_scales(st)
    torch.cuda.synchronize()
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), state["scales"].view(np.uint32))
    expect = onf4.dequantize(state["qweight"], state["scales"], shape)
    assert np.array_equal(_bits(dequantize_nf4(q, scales, st.code, shape)), expect)
    assert np.array_equal(_bits(dequantize_nf4_nested(q, st)), expect)


def test_every_byte_and_special_scales(device):
    shape = (256, 64)
    q = np.resize(np.arange(256, dtype=np.uint8), shape[0] * shape[1] // 2)
    scales = np.resize(np.array([0.0, 1.00390625, 1.01171875, 3e-5, 7.5, 0.02, 1e-38, 65504.0], np.float32), 256)
    expect = onf4.dequantize(q, scales, shape)
    code = torch.from_numpy(onf4.NF4_CODE).to(device)
    out = dequantize_nf4(torch.from_numpy(q).to(device), torch.from_numpy(scales).to(device), code, shape)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out), expect)


def test_product_quantiser_on_device(device):
    g = torch.Generator(device="cpu").manual_seed(731)
    w = (torch.randn(512, 1024, generator=g) * 0.1).bfloat16().to(device)
    q, st = quantize_nf4(w, compress_statistics=True)
    out = dequantize_nf4_nested(q, st)
    ref = onf4.dequantize(
        q.cpu().numpy(),
        onf4.dq_scales(st.absmax.cpu().numpy(), st.state2.absmax.cpu().numpy(), st.state2.code.cpu().numpy(), st.offset.item()),
        (512, 1024),
    )
    assert np.array_equal(_bits(out), ref)


def test_output_cannot_alias_packed_input_storage(device):
    out = torch.empty((64, 64), device=device, dtype=torch.bfloat16)
    packed = out.view(torch.uint8).view(-1)[:2048]
    scales = torch.ones(64, device=device, dtype=torch.float32)
    code = torch.zeros(16, device=device, dtype=torch.float32)
    with pytest.raises(ValueError, match="alias"):
        dequantize_nf4(packed, scales, code, (64, 64), out=out)


@pytest.mark.parametrize("q_offset,out_offset", [(1, 4), (3, 1), (4, 4), (0, 3)])
def test_views_at_unaligned_offsets(q_offset, out_offset, device):
    """Contiguous views at any offset are accepted, as the reference accepts them
    (``ops/nf4.py:76-104`` checks dtype, size and contiguity only): qweight at a byte
    offset, out at an element offset (2-byte steps), both bit-exact, for fp32 and nested
    scales."""
    shape = (128, 192)
    rng = np.random.default_rng(733)
    w = onf4.bf16_to_f32(_cases.bf16(rng.standard_normal(shape) * 0.1))
    state = onf4.quantize(w, double_quant=True)
    expect = onf4.dequantize(state["qweight"], state["scales"], shape)
    q, st = _state_tensors(state, device)
    scales = prepare_scales(st)
    packed = torch.zeros(q.numel() + 16, dtype=torch.uint8, device=device)
    qv = packed[q_offset : q_offset + q.numel()]
    qv.copy_(q)
    backing = torch.zeros(shape[0] * shape[1] + 16, dtype=torch.bfloat16, device=device)
    out = backing[out_offset : out_offset + shape[0] * shape[1]].view(shape)
    print(f"[nf4] unaligned views q+{q_offset} out+{out_offset}", flush=True)
    assert dequantize_nf4(qv, scales, st.code, shape, out=out) is out
    torch.cuda.synchronize()
    assert np.array_equal(_bits(out), expect)
    assert not backing[:out_offset].any() and not backing[out_offset + shape[0] * shape[1] :].any()
    assert np.array_equal(_bits(dequantize_nf4_nested(qv, st, out=torch.empty(shape, dtype=torch.bfloat16, device=device))), expect)
    nested_out = backing[out_offset : out_offset + shape[0] * shape[1]].view(shape)
    nested_out.zero_()
    dequantize_nf4_nested(qv, st, out=nested_out)
    torch.cuda.synchronize()
    assert np.array_equal(_bits(nested_out), expect)
