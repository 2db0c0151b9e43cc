"""FFT and NTT on pitched rows (n >= 2^12): one transform per tile, read and
written at a caller's row pitch without a boundary plan. Each case checks
the whole output buffer against the oracle, padding untouched; shorter rows
keep the gather / scatter boundary (reference layout semantics,
semantic_contract.cpp:55-123)."""
import numpy as np
import pytest

import cubutterfly_amd as cb
import oracle
from gpu_util import to_device, to_host

pytestmark = pytest.mark.gpu

Q30 = 1073479681
Q60 = 576460756061519873


def execute(torch, lib, stream, t, x, span_out, sentinel, in_place):
    xd = to_device(torch, x)
    yd = xd if in_place else to_device(torch, np.full(span_out, sentinel, x.dtype))
    with cb.Plan(lib, t, stream=stream) as plan:
        name = plan.algorithm_name()
        ws_bytes = plan.workspace_size()
        if ws_bytes:
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
            plan.set_workspace(ws, ws_bytes)
        plan.execute(xd, yd)
        torch.cuda.synchronize()
    return name, to_host(torch, yd, x.dtype)


def rows_of(x, batch, pitch, n):
    return np.stack([x[b * pitch: b * pitch + n] for b in range(batch)])


def place(base, rows, pitch):
    out = base.copy()
    for b, row in enumerate(rows):
        out[b * pitch: b * pitch + row.size] = row
    return out


@pytest.mark.parametrize("log_n", [12, 14, 16, 20])
@pytest.mark.parametrize("inverse", [False, True])
def test_fft(torch_gpu, lib, stream, log_n, inverse):
    n, batch = 1 << log_n, 3
    in_pitch, out_pitch = n + 3, n + 40
    rng = np.random.default_rng(log_n)
    span_in, span_out = (batch - 1) * in_pitch + n, (batch - 1) * out_pitch + n
    x = (rng.standard_normal(span_in) + 1j * rng.standard_normal(span_in)).astype(np.complex64)
    t = cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [n], compute=cb.ComputeType.FP32, batch=batch, inverse=inverse, input_strides=[1], input_batch_stride=in_pitch, output_strides=[1], output_batch_stride=out_pitch)
    sentinel = np.complex64(7 - 7j)
    name, got = execute(torch_gpu, lib, stream, t, x, span_out, sentinel, False)
    assert name.endswith("-pitched"), name
    ref = oracle.fft_c64(rows_of(x, batch, in_pitch, n), inverse=inverse, normalize=inverse,
                         threads=oracle.default_threads())
    mask = np.ones(span_out, bool)
    for b in range(batch):
        mask[b * out_pitch: b * out_pitch + n] = False
    assert np.all(got[mask] == sentinel)
    got_rows = rows_of(got, batch, out_pitch, n).astype(np.complex128)
    err = np.linalg.norm(got_rows - ref) / np.linalg.norm(ref)
    assert err <= 1e-5, err


@pytest.mark.parametrize("log_n", [12, 13, 16])
def test_fft_in_place(torch_gpu, lib, stream, log_n):
    n, batch, pitch = 1 << log_n, 4, (1 << log_n) + 16
    rng = np.random.default_rng(5)
    span = (batch - 1) * pitch + n
    x = (rng.standard_normal(span) + 1j * rng.standard_normal(span)).astype(np.complex64)
    t = cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [n], compute=cb.ComputeType.FP32, batch=batch, placement=cb.Placement.IN_PLACE, input_strides=[1], input_batch_stride=pitch, output_strides=[1], output_batch_stride=pitch)
    name, got = execute(torch_gpu, lib, stream, t, x, span, 0, True)
    assert name.endswith("-pitched")
    ref = oracle.fft_c64(rows_of(x, batch, pitch, n), threads=oracle.default_threads())
    gaps = np.ones(span, bool)
    for b in range(batch):
        gaps[b * pitch: b * pitch + n] = False
    assert np.array_equal(got[gaps], x[gaps])
    err = np.linalg.norm(rows_of(got, batch, pitch, n) - ref) / np.linalg.norm(ref)
    assert err <= 1e-5


@pytest.mark.parametrize("word_bits,q", [(32, Q30), (64, Q60)])
@pytest.mark.parametrize("log_n", [12, 13, 16])
@pytest.mark.parametrize("inverse", [False, True])
def test_ntt_negacyclic(torch_gpu, lib, stream, word_bits, q, log_n, inverse):
    n, batch = 1 << log_n, 5
    in_pitch, out_pitch = n + 1, n + 17
    dtype = np.uint32 if word_bits == 32 else np.uint64
    rng = np.random.default_rng(log_n + word_bits)
    span_in, span_out = (batch - 1) * in_pitch + n, (batch - 1) * out_pitch + n
    x = rng.integers(0, q, span_in).astype(dtype)
    storage = cb.DataType.UINT32 if word_bits == 32 else cb.DataType.UINT64
    compute = cb.ComputeType.UINT32 if word_bits == 32 else cb.ComputeType.UINT64
    t = cb.describe(cb.Operator.NTT, storage, [n], compute=compute, batch=batch, modulus=q, word_bits=word_bits, ntt_ring=cb.NttRing.NEGACYCLIC, inverse=inverse, input_strides=[1], input_batch_stride=in_pitch, output_strides=[1], output_batch_stride=out_pitch)
    sentinel = dtype(0xDEADBEEF)
    name, got = execute(torch_gpu, lib, stream, t, x, span_out, sentinel, False)
    assert name.endswith("-pitched"), name
    result = oracle.ntt_negacyclic(rows_of(x, batch, in_pitch, n).astype(np.uint64), q, inverse=inverse)
    expected = place(np.full(span_out, sentinel, dtype), result.astype(dtype), out_pitch)
    np.testing.assert_array_equal(got, expected)


def test_ntt_bit_reversed_output_and_in_place(torch_gpu, lib, stream):
    n, batch, pitch = 1 << 14, 3, (1 << 14) + 5
    rng = np.random.default_rng(9)
    span = (batch - 1) * pitch + n
    x = rng.integers(0, Q30, span).astype(np.uint32)
    t = cb.describe(cb.Operator.NTT, cb.DataType.UINT32, [n], compute=cb.ComputeType.UINT32, batch=batch, modulus=Q30, word_bits=32, ntt_ring=cb.NttRing.NEGACYCLIC, ntt_output_layout=cb.NttLayout.BIT_REVERSED, placement=cb.Placement.IN_PLACE, input_strides=[1], input_batch_stride=pitch, output_strides=[1], output_batch_stride=pitch)
    name, got = execute(torch_gpu, lib, stream, t, x, span, 0, True)
    assert name.endswith("-pitched")
    natural = oracle.ntt_negacyclic(rows_of(x, batch, pitch, n).astype(np.uint64), Q30)
    rev = np.array([int(format(i, "014b")[::-1], 2) for i in range(n)])
    expected = place(x, natural[:, rev].astype(np.uint32), pitch)
    np.testing.assert_array_equal(got, expected)


def test_short_rows_keep_the_boundary(torch_gpu, lib, stream):
    n, batch, pitch = 1 << 10, 3, (1 << 10) + 4
    x = np.arange((batch - 1) * pitch + n, dtype=np.uint32) % Q30
    t = cb.describe(cb.Operator.NTT, cb.DataType.UINT32, [n], compute=cb.ComputeType.UINT32, batch=batch, modulus=Q30, word_bits=32, input_strides=[1], input_batch_stride=pitch)
    name, got = execute(torch_gpu, lib, stream, t, x, batch * n, 0, False)
    assert name.startswith("semantic-boundary[")
    expected = oracle.ntt_cyclic(rows_of(x, batch, pitch, n).astype(np.uint64), Q30).astype(np.uint32).ravel()
    np.testing.assert_array_equal(got, expected)
