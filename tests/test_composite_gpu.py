"""Rank-2 and higher transforms on the GPU against the per-axis oracle
composition, innermost axis first (reference rank-two lowering,
src/c_api.cpp:5231-5327; axis schedule src/c_api.cpp:4578-4600). The
composition itself is pinned in test_composite.py (brute-force 2-D DFT mod q,
numpy fftn, the flat FWHT)."""
import json

import numpy as np
import pytest

import cubutterfly_amd as cb
import oracle
from gpu_util import run_plan, to_device, to_host
from test_composite import along, compose

pytestmark = pytest.mark.gpu

Q30 = 998244353
Q60 = 576460756061519873


def data(shape, dtype, seed, q=None):
    rng = np.random.default_rng(seed)
    if np.dtype(dtype).kind == "c":
        return (rng.standard_normal(shape) + 1j * rng.standard_normal(shape)).astype(dtype)
    if np.dtype(dtype).kind == "u":
        return rng.integers(0, q, shape).astype(dtype)
    return rng.standard_normal(shape).astype(dtype)


def fwht_t(extents, batch, **kw):
    return cb.describe(cb.Operator.FWHT, cb.DataType.FP32, list(extents), compute=cb.ComputeType.FP32, batch=batch, **kw)


def fft_t(extents, batch, **kw):
    return cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, list(extents), compute=cb.ComputeType.FP32, batch=batch, **kw)


def ntt_t(extents, batch, word_bits, q, **kw):
    storage = cb.DataType.UINT32 if word_bits == 32 else cb.DataType.UINT64
    compute = cb.ComputeType.UINT32 if word_bits == 32 else cb.ComputeType.UINT64
    return cb.describe(cb.Operator.NTT, storage, list(extents), compute=compute, batch=batch, modulus=q, word_bits=word_bits, **kw)


@pytest.mark.parametrize("extents,inverse,prefix", [
    ((16, 64), False, "rank2-kronecker"),
    ((32, 64), True, "rank2-fwht-columns"),    # normalised inverse composes per axis
    ((64, 32), True, "rank2-transpose"),       # rows under 64 points: transposes
    ((128, 512), False, "rank2-fwht-columns"), # 2^16 points: above one resident plan
    ((128, 256), False, "rank2-kronecker"),    # 2^15 points: one 2^15-point row plan
    ((4096, 64), True, "rank2-fwht-columns"),  # axis 0 as two column passes
    ((4, 8, 16), True, "rankN-composite"),
    ((8, 4, 64), True, "rankN-fwht-columns"),
    ((2, 4, 8, 16), False, "rankN-kronecker"),
])
def test_fwht_fp32(torch_gpu, lib, stream, extents, inverse, prefix):
    batch = 3
    x = data((batch,) + extents, np.float32, 1)
    t = fwht_t(extents, batch, inverse=inverse)
    with cb.Plan(lib, t) as plan:
        assert plan.algorithm_name().startswith(prefix)
    got = run_plan(torch_gpu, lib, t, x, stream)
    expected = compose(x, lambda rows: oracle.fwht_f32(rows, inverse=inverse, normalize=inverse))
    np.testing.assert_array_equal(got.view(np.uint32), expected.view(np.uint32))


@pytest.mark.parametrize("extents", [(64, 128), (1 << 12, 16), (8, 16, 32)])
@pytest.mark.parametrize("inverse", [False, True])
def test_fft_c64(torch_gpu, lib, stream, extents, inverse):
    batch = 2
    x = data((batch,) + extents, np.complex64, 2)
    t = fft_t(extents, batch, inverse=inverse)
    got = run_plan(torch_gpu, lib, t, x, stream).astype(np.complex128)
    axes = tuple(range(1, len(extents) + 1))
    ref = (np.fft.ifftn if inverse else np.fft.fftn)(x.astype(np.complex128), axes=axes)
    err = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert err <= 1e-5, err


@pytest.mark.parametrize("word_bits,q", [(32, Q30), (64, Q60)])
@pytest.mark.parametrize("extents", [(16, 64), (64, 1 << 13), (4, 8, 32)])
@pytest.mark.parametrize("inverse", [False, True])
def test_ntt_cyclic(torch_gpu, lib, stream, word_bits, q, extents, inverse):
    batch = 2
    dtype = np.uint32 if word_bits == 32 else np.uint64
    x = data((batch,) + extents, dtype, 3, q)
    t = ntt_t(extents, batch, word_bits, q, inverse=inverse)
    got = run_plan(torch_gpu, lib, t, x, stream)
    expected = compose(x.astype(np.uint64), lambda rows: oracle.ntt_cyclic(rows, q, inverse=inverse))
    np.testing.assert_array_equal(got.astype(np.uint64), expected)


def test_ntt_rank2_brute_force(torch_gpu, lib, stream):
    q, n0, n1 = Q30, 4, 8
    x = data((1, n0, n1), np.uint32, 4, q)
    got = run_plan(torch_gpu, lib, ntt_t((n0, n1), 1, 32, q), x, stream)
    w0, w1 = oracle.find_primitive_root(2, q), oracle.find_primitive_root(3, q)
    for k0 in range(n0):
        for k1 in range(n1):
            acc = sum(int(x[0, j0, j1]) * pow(w0, j0 * k0, q) * pow(w1, j1 * k1, q)
                      for j0 in range(n0) for j1 in range(n1))
            assert int(got[0, k0, k1]) == acc % q


def test_in_place(torch_gpu, lib, stream):
    extents, batch = (64, 32), 2
    x = data((batch,) + extents, np.complex64, 5)
    t = fft_t(extents, batch, placement=cb.Placement.IN_PLACE)
    got = run_plan(torch_gpu, lib, t, x, stream, in_place=True).astype(np.complex128)
    ref = np.fft.fftn(x.astype(np.complex128), axes=(1, 2))
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 1e-5


def test_strided_sides_and_orders(torch_gpu, lib, stream):
    # Input rows with a pitch and interleaved columns; output bit-reversed
    # along axis 0 into a pitched buffer. Untouched output elements keep
    # their sentinel.
    n0, n1, batch = 16, 32, 2
    s_in = (2 * n1 + 8, 2)          # row pitch, column stride
    bs_in = n0 * s_in[0] + 4
    s_out = (n1 + 4, 1)
    bs_out = n0 * s_out[0]
    rng = np.random.default_rng(6)
    span_in = (batch - 1) * bs_in + (n0 - 1) * s_in[0] + (n1 - 1) * s_in[1] + 1
    span_out = (batch - 1) * bs_out + (n0 - 1) * s_out[0] + (n1 - 1) * s_out[1] + 1
    x_flat = rng.integers(0, Q30, span_in).astype(np.uint32)
    b, i0, i1 = np.meshgrid(np.arange(batch), np.arange(n0), np.arange(n1), indexing="ij")
    logical = x_flat[b * bs_in + i0 * s_in[0] + i1 * s_in[1]]
    result = compose(logical.astype(np.uint64), lambda rows: oracle.ntt_cyclic(rows, Q30))
    rev0 = np.array([int(format(i, "04b")[::-1], 2) for i in range(n0)])
    expected = np.full(span_out, 0xDEADBEEF, np.uint32)
    expected[b * bs_out + rev0[i0] * s_out[0] + i1 * s_out[1]] = result.astype(np.uint32)
    t = ntt_t((n0, n1), batch, 32, Q30, input_strides=list(s_in), input_batch_stride=bs_in,
              output_strides=list(s_out), output_batch_stride=bs_out,
              output_orders=[cb.LogicalOrder.BIT_REVERSED, cb.LogicalOrder.NATURAL])
    xd = to_device(torch_gpu, x_flat)
    yd = to_device(torch_gpu, np.full(span_out, 0xDEADBEEF, np.uint32))
    with cb.Plan(lib, t, stream=stream) as plan:
        name = plan.algorithm_name()
        assert name.startswith("rank2-transpose[") and "+direct" not in name
        assert plan.input_size() == span_in * 4 and plan.output_size() == span_out * 4
        ws = torch_gpu.empty(plan.workspace_size(), dtype=torch_gpu.uint8, device="cuda")
        plan.set_workspace(ws, plan.workspace_size())
        plan.execute(xd, yd)
        torch_gpu.cuda.synchronize()
    np.testing.assert_array_equal(to_host(torch_gpu, yd, np.uint32), expected)


def test_transpose_edges(torch_gpu, lib, stream):
    # Axes shorter than the 64-element transpose tile, and a long thin shape.
    for extents in [(2, 4), (4, 2), (2, 1 << 12), (1 << 12, 2)]:
        x = data((2,) + extents, np.complex64, 7)
        got = run_plan(torch_gpu, lib, fft_t(extents, 2), x, stream).astype(np.complex128)
        ref = np.fft.fftn(x.astype(np.complex128), axes=(1, 2))
        assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 1e-5, extents


def test_mapping_reports_children(torch_gpu, lib):
    with cb.Plan(lib, ntt_t((64, 1 << 13), 2, 64, Q60)) as plan:
        m = plan.mapping()
        assert m["kind"] == "composition" and m["rank"] == 2
        axes = [s for s in m["schedule"] if s["step"] == "axis"]
        assert [s["axis"] for s in axes] == [1, 0]
        assert plan.workspace_size() == m["workspace_bytes"] >= 2 * 2 * 64 * (1 << 13) * 8


@pytest.mark.parametrize("extents", [(256, 256), (1024, 512), (4096, 16), (512, 1024)])
@pytest.mark.parametrize("inverse", [False, True])
def test_fft_transposing_rows(torch_gpu, lib, stream, extents, inverse):
    # Two row passes with transposing stores, no transpose kernels.
    batch = 3
    x = data((batch,) + extents, np.complex64, 8)
    t = fft_t(extents, batch, inverse=inverse)
    with cb.Plan(lib, t) as plan:
        assert plan.algorithm_name().startswith("rank2-transposing[fft-c64-rows-transposed-r16,")
        m = plan.mapping()
        assert [s["step"] for s in m["schedule"]] == ["axis", "axis"]
        assert plan.workspace_size() == batch * extents[0] * extents[1] * 8  # one intermediate
    got = run_plan(torch_gpu, lib, t, x, stream).astype(np.complex128)
    ref = (np.fft.ifftn if inverse else np.fft.fftn)(x.astype(np.complex128), axes=(1, 2))
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 1e-5


# Axes of 2^11 points or more: axis 0 as one column pass (2^4 .. 2^8 points)
# or two (the split of 2^9 .. 2^16), then the rows stored in natural order.
@pytest.mark.parametrize("extents,batch,inverse", [
    ((4096, 4096), 1, False),
    ((4096, 4096), 1, True),
    ((2048, 4096), 1, False),
    ((4096, 2048), 1, True),
    ((16, 4096), 3, False),     # one 4-bit column pass
    ((256, 2048), 2, True),     # one 8-bit column pass
    ((512, 4096), 2, False),    # 5 + 4 bits
    ((8192, 1024), 1, True),    # 7 + 6 bits
    ((65536, 256), 1, False),   # 8 + 8 bits, 256-point rows
])
def test_fft_rank2_columns(torch_gpu, lib, stream, extents, batch, inverse):
    x = data((batch,) + extents, np.complex64, 10)
    t = fft_t(extents, batch, inverse=inverse)
    with cb.Plan(lib, t) as plan:
        assert plan.algorithm_name() == "rank2-columns[fft-c64-rank2-columns-r16]+direct-input+direct-output"
        m = plan.mapping()
        assert m["lowering"] == "columns-then-rows"
        assert [s["step"] for s in m["schedule"]] == ["axes"]
        child = m["schedule"][0]["child"]
        assert child["axis0_bits"] == int(np.log2(extents[0]))
        assert child["column_passes"] == (1 if extents[0] <= 256 else 2)
        assert plan.workspace_size() == batch * extents[0] * extents[1] * 8  # one intermediate
    got = run_plan(torch_gpu, lib, t, x, stream).astype(np.complex128)
    ref = (np.fft.ifftn if inverse else np.fft.fftn)(x.astype(np.complex128), axes=(1, 2))
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 1e-5


ROWS_NAME = "rank2-transposing[fft-c64-rows-transposed-r16,fft-c64-rows-transposed-r16]+direct-input+direct-output"
COLUMNS_NAME = "rank2-columns[fft-c64-rank2-columns-r16]+direct-input+direct-output"


@pytest.mark.parametrize("extents,batch,name", [
    ((2048, 4096), 1, ROWS_NAME),     # the default there is column passes
    ((1024, 512), 2, COLUMNS_NAME),   # the default there is transposing rows
])
def test_fft_rank2_lowering_by_name(torch_gpu, lib, stream, extents, batch, name):
    x = data((batch,) + extents, np.complex64, 13)
    t = fft_t(extents, batch)
    with cb.Plan(lib, t) as plan:
        assert plan.algorithm_name() != name
    with cb.Plan(lib, t, algorithm=name) as plan:
        assert plan.algorithm_name() == name
        assert plan.selection_source() == cb.SelectionSource.EXPLICIT
    got = run_plan(torch_gpu, lib, t, x, stream, algorithm=name).astype(np.complex128)
    ref = np.fft.fftn(x.astype(np.complex128), axes=(1, 2))
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 1e-5


def test_fft_rank2_measure_times_both_lowerings_and_the_cache_replays(torch_gpu, lib, stream, tmp_path):
    extents, batch = (512, 2048), 2
    t = fft_t(extents, batch)
    cache = tmp_path / "sel.tsv"
    with cb.Plan(lib, t, policy=cb.AlgorithmPolicy.MEASURE, stream=stream, cache_path=cache) as plan:
        reason = plan.selection_reason()
        chosen = plan.algorithm_name()
        assert plan.selection_source() == cb.SelectionSource.RUNTIME_MEASURED
    assert "rank2-columns[" in reason and "rank2-transposing[" in reason, reason
    assert chosen in (ROWS_NAME, COLUMNS_NAME)
    records = [line.split("\t") for line in cache.read_text().splitlines()]
    assert records[-1][0].endswith("|rank2-fft|512x2048") and records[-1][1] == chosen
    with cb.Plan(lib, t, stream=stream, cache_path=cache) as plan:
        assert plan.algorithm_name() == chosen
        assert plan.selection_source() == cb.SelectionSource.USER_CACHE
    x = data((batch,) + extents, np.complex64, 14)
    got = run_plan(torch_gpu, lib, t, x, stream, cache_path=cache).astype(np.complex128)
    ref = np.fft.fftn(x.astype(np.complex128), axes=(1, 2))
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 1e-5


def test_fft_rank2_measure_refuses_stream_capture(torch_gpu, lib):
    # Refused before either lowering allocates its tables: the capture stays
    # valid.
    s = torch_gpu.cuda.Stream()
    graph = torch_gpu.cuda.CUDAGraph()
    with torch_gpu.cuda.graph(graph, stream=s):
        with pytest.raises(cb.AbiError) as e:
            cb.Plan(lib, fft_t((512, 2048), 2), policy=cb.AlgorithmPolicy.MEASURE, stream=s.cuda_stream)
        assert e.value.status == cb.Status.NOT_SUPPORTED and "capture" in e.value.detail


def test_fft_rank2_columns_by_name_where_no_kernel_covers_it(lib):
    # 16-point rows: no natural-order row tiles of that length.
    with pytest.raises(cb.AbiError) as e:
        cb.Plan(lib, fft_t((4096, 16), 1), algorithm=COLUMNS_NAME)
    assert e.value.status == cb.Status.NOT_SUPPORTED


def test_fft_rank2_columns_in_place_unnormalised(torch_gpu, lib, stream):
    extents, batch = (2048, 4096), 1
    x = data((batch,) + extents, np.complex64, 11)
    t = fft_t(extents, batch, inverse=True, normalize_inverse=False, placement=cb.Placement.IN_PLACE)
    with cb.Plan(lib, t) as plan:
        assert plan.algorithm_name().startswith("rank2-columns[")
    got = run_plan(torch_gpu, lib, t, x, stream, in_place=True).astype(np.complex128)
    ref = np.fft.ifftn(x.astype(np.complex128), axes=(1, 2)) * (extents[0] * extents[1])
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 1e-5


def test_fft_rank2_columns_strided_sides(torch_gpu, lib, stream):
    # Pitched rows on both sides: gather into packed order, the column plan,
    # scatter; the gaps between rows stay untouched.
    n0, n1, batch, pitch = 2048, 2048, 1, 2048 + 16
    span = (batch * n0 - 1) * pitch + n1
    rng = np.random.default_rng(12)
    flat = (rng.standard_normal(span) + 1j * rng.standard_normal(span)).astype(np.complex64)
    t = fft_t((n0, n1), batch, input_strides=[pitch, 1], input_batch_stride=n0 * pitch,
              output_strides=[pitch, 1], output_batch_stride=n0 * pitch)
    with cb.Plan(lib, t) as plan:
        name = plan.algorithm_name()
        assert name.startswith("rank2-columns[") and "+direct" not in name
    x = to_device(torch_gpu, flat)
    y = to_device(torch_gpu, np.full(span, 7 + 7j, np.complex64))
    with cb.Plan(lib, t, stream=stream) as plan:
        ws_bytes = plan.workspace_size()
        ws = torch_gpu.empty(ws_bytes, dtype=torch_gpu.uint8, device="cuda")
        plan.set_workspace(ws, ws_bytes)
        plan.execute(x, y)
        torch_gpu.cuda.synchronize()
    got = to_host(torch_gpu, y, np.complex64)
    rows = np.stack([flat[k * pitch: k * pitch + n1] for k in range(n0)])
    ref = np.fft.fftn(rows.astype(np.complex128))
    got_rows = np.stack([got[k * pitch: k * pitch + n1] for k in range(n0)]).astype(np.complex128)
    assert np.linalg.norm(got_rows - ref) / np.linalg.norm(ref) <= 1e-5
    gaps = np.ones(span, bool)
    for k in range(n0):
        gaps[k * pitch: k * pitch + n1] = False
    assert np.all(got[gaps] == np.complex64(7 + 7j))


def test_fft_transposing_rows_strided_in_place(torch_gpu, lib, stream):
    # In place on pitched rows: gather, the two row passes, scatter.
    n0, n1, batch, pitch = 256, 256, 2, 256 + 8
    span = (batch * n0 - 1) * pitch + n1
    rng = np.random.default_rng(9)
    flat = (rng.standard_normal(span) + 1j * rng.standard_normal(span)).astype(np.complex64)
    t = fft_t((n0, n1), batch, placement=cb.Placement.IN_PLACE, input_strides=[pitch, 1], input_batch_stride=n0 * pitch,
              output_strides=[pitch, 1], output_batch_stride=n0 * pitch)
    got = run_plan(torch_gpu, lib, t, flat, stream, in_place=True)
    rows = np.stack([flat[k * pitch: k * pitch + n1] for k in range(batch * n0)]).reshape(batch, n0, n1)
    ref = np.fft.fftn(rows.astype(np.complex128), axes=(1, 2)).reshape(batch * n0, n1)
    got_rows = np.stack([got[k * pitch: k * pitch + n1] for k in range(batch * n0)]).astype(np.complex128)
    assert np.linalg.norm(got_rows - ref) / np.linalg.norm(ref) <= 1e-5
    gaps = np.ones(span, bool)
    for k in range(batch * n0):
        gaps[k * pitch: k * pitch + n1] = False
    assert np.array_equal(got[gaps], flat[gaps])
