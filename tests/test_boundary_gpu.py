"""Semantic boundary on the GPU: strided sides and logical orders gathered to
packed natural order, transformed, scattered (reference src/c_api.cpp:
5064-5085; gather / scatter src/general_kernels.cu:30-54). Each case checks
the whole output buffer: transformed elements against the oracle applied to
the gathered rows, and every element outside the output layout unchanged.
"""
import json

import numpy as np
import pytest

import cubutterfly_amd as cb
import oracle
from cubutterfly_amd import workloads
from gpu_util import to_device, to_host

pytestmark = pytest.mark.gpu

Q30 = workloads.C2_MODULUS


def bitrev(j, log_n):
    r = np.zeros_like(j)
    for b in range(log_n):
        r |= ((j >> b) & 1) << (log_n - 1 - b)
    return r


def positions(n, batch, stride, batch_stride, reversed_):
    log_n = n.bit_length() - 1
    j = np.arange(n, dtype=np.int64)
    r = bitrev(j, log_n) if reversed_ else j
    return np.arange(batch, dtype=np.int64)[:, None] * batch_stride_of(n, stride, batch_stride) + r[None, :] * stride


def batch_stride_of(n, stride, batch_stride):
    """Zero means the axis span; a negative value -p means pitched rows, the
    span plus p padding elements."""
    span_ = (n - 1) * stride + 1
    return span_ - batch_stride if batch_stride < 0 else batch_stride or span_


def span(n, batch, stride, batch_stride):
    return (n - 1) * stride + (batch - 1) * batch_stride_of(n, stride, batch_stride) + 1


def run(torch, lib, stream, t, x_flat, out_len, sentinel, in_place=False):
    x = to_device(torch, x_flat)
    if in_place:
        y = x
    else:
        y = to_device(torch, np.full(out_len, sentinel, dtype=x_flat.dtype))
    with cb.Plan(lib, t, stream=stream) as plan:
        assert plan.input_size() == x.numel() * x.element_size()
        assert plan.output_size() == y.numel() * y.element_size()
        name = plan.algorithm_name()
        assert name.startswith("semantic-boundary[") or name.endswith("-pitched") or "-bitrev-" in name, name
        ws = plan.workspace_size()
        buf = torch.empty(ws, dtype=torch.uint8, device="cuda")
        plan.set_workspace(buf, ws)
        plan.execute(x, y)
        torch.cuda.synchronize()
    return to_host(torch, y, x_flat.dtype)


def case(n, batch, dtype, seed, in_layout, out_layout, sentinel):
    """Strided host input, gathered rows, and the untouched output image."""
    (s_in, bs_in, rev_in), (s_out, bs_out, rev_out) = in_layout, out_layout
    rng = np.random.default_rng(seed)
    n_in = span(n, batch, s_in, bs_in)
    if np.dtype(dtype).kind == "c":
        x_flat = (rng.standard_normal(n_in) + 1j * rng.standard_normal(n_in)).astype(dtype)
    elif np.dtype(dtype).kind == "u":
        x_flat = rng.integers(0, Q30, n_in).astype(dtype)
    else:
        x_flat = rng.standard_normal(n_in).astype(dtype)
    rows = x_flat[positions(n, batch, s_in, bs_in, rev_in)]
    out_pos = positions(n, batch, s_out, bs_out, rev_out)
    return x_flat, rows, out_pos, span(n, batch, s_out, bs_out)


def transform(op, n, batch, in_layout, out_layout, storage, **kw):
    (s_in, bs_in, rev_in), (s_out, bs_out, rev_out) = in_layout, out_layout
    order = lambda rev: [cb.LogicalOrder.BIT_REVERSED if rev else cb.LogicalOrder.NATURAL]
    bs_in, bs_out = (b if b >= 0 else batch_stride_of(n, s, b) for s, b in ((s_in, bs_in), (s_out, bs_out)))
    return cb.describe(op, storage, [n], batch=batch, input_strides=[s_in], input_batch_stride=bs_in, output_strides=[s_out], output_batch_stride=bs_out, input_orders=order(rev_in), output_orders=order(rev_out), **kw)


LAYOUTS = [
    ((5, 1, False), (1, 0, False)),      # interleaved input rows, packed output
    ((1, 0, True), (2, 0, False)),       # bit-reversed packed input, strided output with gaps
    ((3, 0, False), (1, 0, True)),       # strided input, bit-reversed packed output
    ((1, 0, False), (1, 0, True)),       # packed, logical order only
    ((1, -8, False), (1, -4, False)),    # pitched rows on both sides
    ((1, -8, False), (1, -3, False)),    # pitched input, odd output pitch
    ((1, -40, True), (1, -24, True)),    # pitched rows, bit-reversed on both sides
]


@pytest.mark.parametrize("n", [64, 2048])
@pytest.mark.parametrize("in_layout,out_layout", LAYOUTS)
def test_fwht_fp32(torch_gpu, lib, stream, n, in_layout, out_layout):
    # 2048: bit-reversed unit-stride rows move through the tiled reversal.
    batch = 5
    x_flat, rows, out_pos, out_len = case(n, batch, np.float32, 1, in_layout, out_layout, 0)
    t = transform(cb.Operator.FWHT, n, batch, in_layout, out_layout, storage=cb.DataType.FP32,
                  compute=cb.ComputeType.FP32)
    got = run(torch_gpu, lib, stream, t, x_flat, out_len, np.float32(-7.0))
    expected = np.full(out_len, -7.0, np.float32)
    expected[out_pos] = oracle.fwht_f32(rows)
    np.testing.assert_array_equal(got, expected)


@pytest.mark.parametrize("n", [128, 1024])
@pytest.mark.parametrize("in_layout,out_layout", LAYOUTS)
def test_fwht_fp16_final(torch_gpu, lib, stream, n, in_layout, out_layout):
    batch, scale = 3, n ** -0.5
    x_flat, rows, out_pos, out_len = case(n, batch, np.float16, 2, in_layout, out_layout, 0)
    t = transform(cb.Operator.FWHT, n, batch, in_layout, out_layout, storage=cb.DataType.FP16,
                  compute=cb.ComputeType.FP32, output_scale=scale, output_rounding=cb.OutputRounding.FINAL_STORAGE)
    got = run(torch_gpu, lib, stream, t, x_flat, out_len, np.float16(3.0))
    expected = np.full(out_len, 3.0, np.float16)
    expected[out_pos] = oracle.fwht_f16_final(rows, scale)
    np.testing.assert_array_equal(got.view(np.uint16), expected.view(np.uint16))


@pytest.mark.parametrize("log_n", [10, 15])
@pytest.mark.parametrize("in_layout,out_layout", LAYOUTS)
def test_fft(torch_gpu, lib, stream, log_n, in_layout, out_layout):
    n, batch = 1 << log_n, 3
    x_flat, rows, out_pos, out_len = case(n, batch, np.complex64, 3, in_layout, out_layout, 0)
    t = transform(cb.Operator.FFT, n, batch, in_layout, out_layout, storage=cb.DataType.COMPLEX_FP32,
                  compute=cb.ComputeType.FP32)
    got = run(torch_gpu, lib, stream, t, x_flat, out_len, np.complex64(5 + 5j))
    ref = oracle.fft_c64(rows).astype(np.complex128)
    mask = np.ones(out_len, bool)
    mask[out_pos] = False
    assert np.all(got[mask] == np.complex64(5 + 5j))
    err = np.linalg.norm(got[out_pos].astype(np.complex128) - ref) / np.linalg.norm(ref)
    assert err <= 1e-5, err


@pytest.mark.parametrize("log_n", [9, 14])
@pytest.mark.parametrize("in_layout,out_layout", LAYOUTS)
def test_ntt_negacyclic(torch_gpu, lib, stream, log_n, in_layout, out_layout):
    n, batch = 1 << log_n, 2
    x_flat, rows, out_pos, out_len = case(n, batch, np.uint32, 4, in_layout, out_layout, 0)
    t = transform(cb.Operator.NTT, n, batch, in_layout, out_layout, storage=cb.DataType.UINT32,
                  compute=cb.ComputeType.UINT32, modulus=Q30, word_bits=32, ntt_ring=cb.NttRing.NEGACYCLIC)
    if in_layout[:2] in ((1, 0),) and out_layout[:2] in ((1, 0),):
        pytest.skip("packed NTT orders are native (not a boundary plan); covered by test_ntt_gpu")
    got = run(torch_gpu, lib, stream, t, x_flat, out_len, np.uint32(0xDEADBEEF))
    expected = np.full(out_len, 0xDEADBEEF, np.uint32)
    expected[out_pos] = oracle.ntt_negacyclic(rows.astype(np.uint64), Q30).astype(np.uint32)
    np.testing.assert_array_equal(got, expected)


def test_in_place_interleaved(torch_gpu, lib, stream):
    # Same interleaved layout on both sides, executed in place.
    n, batch = 256, 4
    layout = (4, 1, False)
    x_flat, rows, out_pos, out_len = case(n, batch, np.float32, 5, layout, layout, 0)
    t = transform(cb.Operator.FWHT, n, batch, layout, layout, storage=cb.DataType.FP32,
                  compute=cb.ComputeType.FP32, placement=cb.Placement.IN_PLACE)
    got = run(torch_gpu, lib, stream, t, x_flat, out_len, 0, in_place=True)
    expected = x_flat.copy()
    expected[out_pos] = oracle.fwht_f32(rows)
    np.testing.assert_array_equal(got, expected)


def test_fft_logical_order_plan(torch_gpu, lib):
    # One-pass lengths take bit-reversed orders natively; longer ones write a
    # bit-reversed output natively (final row pass) and gather a bit-reversed
    # input through the boundary.
    t = cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [64], compute=cb.ComputeType.FP32, batch=2, output_orders=[cb.LogicalOrder.BIT_REVERSED], input_orders=[cb.LogicalOrder.NATURAL])
    with cb.Plan(lib, t) as plan:
        assert plan.algorithm_name() == "fft-c64-resident-r16-bitrev-out"
    t["shape"] = [1 << 15]
    with cb.Plan(lib, t) as plan:
        assert plan.algorithm_name() == "fft-c64-two-pass-r16-bitrev-out"
    t["output_orders"], t["input_orders"] = [int(cb.LogicalOrder.NATURAL)], [int(cb.LogicalOrder.BIT_REVERSED)]
    with cb.Plan(lib, t) as plan:
        assert plan.algorithm_name().startswith("semantic-boundary[fft-c64")
        assert plan.mapping()["input_bit_reversed"] is True


def test_packed_ntt_orders_stay_native(torch_gpu, lib):
    t = cb.describe(cb.Operator.NTT, cb.DataType.UINT32, [64], compute=cb.ComputeType.UINT32, batch=2, modulus=998244353, word_bits=32, ntt_output_layout=cb.NttLayout.BIT_REVERSED)
    with cb.Plan(lib, t) as plan:
        assert not plan.algorithm_name().startswith("semantic-boundary")


def test_strided_two_pass_ntt_workspace(torch_gpu, lib):
    t = cb.describe(cb.Operator.NTT, cb.DataType.UINT64, [1 << 14], compute=cb.ComputeType.UINT64, batch=2, modulus=576460756061519873, word_bits=64, input_strides=[2], input_batch_stride=1)
    with cb.Plan(lib, t) as plan:
        assert plan.algorithm_name().startswith("semantic-boundary[ntt")
        m = plan.mapping()
        packed = (1 << 15) * 8
        assert plan.workspace_size() == m["workspace_bytes"] >= 2 * packed
