"""FWHT beyond one resident row (n > 2^15): factored into a resident row of
2^12 to 2^15 points and axes of at most 2^7 points (in-place column passes),
lowest index bits first, which is the reference's stage order
(src/butterfly_reference.cpp:349-369), so results are bit-identical to the
oracle; the inverse divides by n once, after the last stage. FP16 final-storage rows run as the reference's FP32 promotion
(src/butterfly.cu:1452-1470: widen, the FP32 transform, one narrowing of
y * scale), bit-identical to the oracle's FP16 contract
(tests/test_fwht_final_storage.py:28-40); bit-reversed orders gather through
the boundary (src/c_api.cpp:5064-5085)."""
import numpy as np
import pytest

import cubutterfly_amd as cb
import oracle
from gpu_util import run_plan, to_device, to_host

pytestmark = pytest.mark.gpu


def fwht(n, batch, **kw):
    return cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [n], compute=cb.ComputeType.FP32, batch=batch, **kw)


@pytest.mark.parametrize("log_n,batch", [(14, 8), (16, 4), (20, 2), (24, 1)])
def test_forward_bit_exact(torch_gpu, lib, stream, log_n, batch):
    x = np.random.default_rng(log_n).standard_normal((batch, 1 << log_n)).astype(np.float32)
    got = run_plan(torch_gpu, lib, fwht(1 << log_n, batch), x, stream)
    expected = oracle.fwht_f32(x, threads=oracle.default_threads())
    np.testing.assert_array_equal(got.view(np.uint32), expected.view(np.uint32))


def test_inverse_normalised_and_in_place(torch_gpu, lib, stream):
    x = np.random.default_rng(3).standard_normal((3, 1 << 16)).astype(np.float32)
    got = run_plan(torch_gpu, lib, fwht(1 << 16, 3, inverse=True, placement=cb.Placement.IN_PLACE), x, stream, in_place=True)
    expected = oracle.fwht_f32(x, inverse=True, normalize=True, threads=oracle.default_threads())
    np.testing.assert_array_equal(got.view(np.uint32), expected.view(np.uint32))


def test_pitched_rows(torch_gpu, lib, stream):
    n, batch, pitch = 1 << 15, 3, (1 << 15) + 32
    rng = np.random.default_rng(4)
    flat = rng.standard_normal((batch - 1) * pitch + n).astype(np.float32)
    t = fwht(n, batch, input_strides=[1], input_batch_stride=pitch)
    got = run_plan(torch_gpu, lib, t, flat, stream).reshape(batch, n)
    rows = np.stack([flat[b * pitch: b * pitch + n] for b in range(batch)])
    np.testing.assert_array_equal(got.view(np.uint32), oracle.fwht_f32(rows).view(np.uint32))


def fwht16(n, batch, scale, **kw):
    return cb.describe(cb.Operator.FWHT, cb.DataType.FP16, [n], compute=cb.ComputeType.FP32, batch=batch,
                       output_scale=scale, output_rounding=cb.OutputRounding.FINAL_STORAGE, **kw)


def f16_rows(batch, n, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((batch, n))
    x[:, rng.integers(0, n, 7)] *= 50.0  # outlier channels, as in the C5 workload
    return x.astype(np.float16)


# Scales that are not powers of two make the two roundings of y * scale (to
# FP32, then to FP16) observable: a fused single rounding fails these.
@pytest.mark.parametrize("log_n,batch,scale", [(16, 2, None), (16, 3, 0.37), (18, 2, 2.0 ** -7.5), (20, 2, None),
                                               (17, 2, -0.75)])
def test_fp16_promoted_bit_exact(torch_gpu, lib, stream, log_n, batch, scale):
    n = 1 << log_n
    scale = float(np.float32(n ** -0.5 if scale is None else scale))
    x = f16_rows(batch, n, log_n)
    print(f"case fp16 promoted fwht n=2^{log_n} batch={batch} scale={scale}", flush=True)
    with cb.Plan(lib, fwht16(n, batch, scale)) as plan:
        assert plan.algorithm_name().startswith("fwht-fp16-promoted[")
    got = run_plan(torch_gpu, lib, fwht16(n, batch, scale), x, stream)
    expected = oracle.fwht_f16_final(x, scale, threads=oracle.default_threads())
    np.testing.assert_array_equal(got.view(np.uint16), expected.view(np.uint16))


def test_fp16_promoted_inverse_normalised_in_place(torch_gpu, lib, stream):
    n, batch = 1 << 16, 3
    x = f16_rows(batch, n, 9)
    t = fwht16(n, batch, 1.0, inverse=True, normalize_inverse=True, placement=cb.Placement.IN_PLACE)
    got = run_plan(torch_gpu, lib, t, x, stream, in_place=True)
    expected = oracle.fwht_f16_final(x, 1.0, inverse=True, normalize=True)
    np.testing.assert_array_equal(got.view(np.uint16), expected.view(np.uint16))


def test_fp16_promoted_unaligned_buffers(torch_gpu, lib, stream):
    # Buffers off a 16-byte boundary take the element-wise widening and narrowing.
    n, batch, scale = 1 << 16, 2, float(np.float32(0.3))
    x = f16_rows(batch, n, 11)
    xd = to_device(torch_gpu, np.concatenate([np.zeros(1, np.float16), x.ravel()]))
    yd = to_device(torch_gpu, np.zeros(batch * n + 1, np.float16))
    import ctypes
    t = fwht16(n, batch, scale)
    with cb.Plan(lib, t, stream=stream) as plan:
        ws = plan.workspace_size()
        buf = torch_gpu.empty(ws, dtype=torch_gpu.uint8, device="cuda")
        plan.set_workspace(buf, ws)
        plan.execute(ctypes.c_void_p(xd.data_ptr() + 2), ctypes.c_void_p(yd.data_ptr() + 2))
        torch_gpu.cuda.synchronize()
    got = to_host(torch_gpu, yd, np.float16)[1:].reshape(batch, n)
    np.testing.assert_array_equal(got.view(np.uint16), oracle.fwht_f16_final(x, scale).view(np.uint16))


def bitrev_perm(log_n):
    j = np.arange(1 << log_n)
    r = np.zeros_like(j)
    for b in range(log_n):
        r |= ((j >> b) & 1) << (log_n - 1 - b)
    return r


@pytest.mark.parametrize("fp16", [False, True])
@pytest.mark.parametrize("log_n", [14, 18])
@pytest.mark.parametrize("rev_in,rev_out", [(True, False), (False, True), (True, True)])
def test_bit_reversed_orders(torch_gpu, lib, stream, fp16, log_n, rev_in, rev_out):
    # Logical coordinate i of a BIT_REVERSED side lives at reverse_bits(i)
    # (cubutterfly.h:23-30).
    n, batch = 1 << log_n, 2
    order = lambda rev: [cb.LogicalOrder.BIT_REVERSED if rev else cb.LogicalOrder.NATURAL]
    perm = bitrev_perm(log_n)
    if fp16:
        logical = f16_rows(batch, n, log_n + 1)
        scale = float(np.float32(0.37))
        t = fwht16(n, batch, scale, input_orders=order(rev_in), output_orders=order(rev_out))
        expected = oracle.fwht_f16_final(logical, scale)
    else:
        logical = np.random.default_rng(log_n).standard_normal((batch, n)).astype(np.float32)
        t = fwht(n, batch, input_orders=order(rev_in), output_orders=order(rev_out))
        expected = oracle.fwht_f32(logical)
    stored = logical[:, perm] if rev_in else logical
    got = run_plan(torch_gpu, lib, t, np.ascontiguousarray(stored), stream)
    want = expected[:, perm] if rev_out else expected
    bits = np.uint16 if fp16 else np.uint32
    np.testing.assert_array_equal(got.view(bits), want.view(bits))


def test_fp16_strided_sides(torch_gpu, lib, stream):
    # Element stride 2 on the input, pitched output rows: gathered, promoted,
    # scattered; the output's padding keeps its sentinel.
    n, batch, scale = 1 << 16, 3, float(np.float32((1 << 16) ** -0.5))
    rows = f16_rows(batch, n, 21)
    in_bs, out_bs = 2 * n + 6, n + 24
    flat = np.zeros((batch - 1) * in_bs + 2 * (n - 1) + 1, np.float16)
    for b in range(batch):
        flat[b * in_bs: b * in_bs + 2 * n: 2] = rows[b]
    t = fwht16(n, batch, scale, input_strides=[2], input_batch_stride=in_bs, output_strides=[1],
               output_batch_stride=out_bs)
    sentinel = np.float16(-5.0)
    xd = to_device(torch_gpu, flat)
    yd = to_device(torch_gpu, np.full((batch - 1) * out_bs + n, sentinel, np.float16))
    with cb.Plan(lib, t, stream=stream) as plan:
        assert plan.algorithm_name().startswith("semantic-boundary[fwht-fp16-promoted[")
        ws = plan.workspace_size()
        buf = torch_gpu.empty(ws, dtype=torch_gpu.uint8, device="cuda")
        plan.set_workspace(buf, ws)
        plan.execute(xd, yd)
        torch_gpu.cuda.synchronize()
    got = to_host(torch_gpu, yd, np.float16)
    want = np.full_like(got, sentinel)
    result = oracle.fwht_f16_final(rows, scale)
    for b in range(batch):
        want[b * out_bs: b * out_bs + n] = result[b]
    np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("inverse", [False, True])
def test_rank2_with_a_long_axis(torch_gpu, lib, stream, inverse):
    # H(4) (x) H(2^14): the 2^14-point axis is itself factored; innermost
    # first, the composition is the flat transform's stage order, bit for bit.
    batch, n0, n1 = 2, 4, 1 << 14
    x = np.random.default_rng(31).standard_normal((batch, n0 * n1)).astype(np.float32)
    t = cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [n0, n1], compute=cb.ComputeType.FP32, batch=batch,
                    inverse=inverse, normalize_inverse=inverse)
    got = run_plan(torch_gpu, lib, t, x, stream)
    want = oracle.fwht_f32(x, inverse=inverse, normalize=inverse)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("log_n,batch", [(16, 2), (20, 2), (21, 1)])
def test_inverse_divides_once_subnormal(torch_gpu, lib, stream, log_n, batch):
    # The reference divides by n once, after the last stage
    # (src/operator_traits.cuh:110): with outputs in the subnormal range a
    # per-pass 1/n_axis would round twice and differ from it.
    x = (np.random.default_rng(40 + log_n).standard_normal((batch, 1 << log_n)) * 2.0 ** -120).astype(np.float32)
    got = run_plan(torch_gpu, lib, fwht(1 << log_n, batch, inverse=True), x, stream)
    want = oracle.fwht_f32(x, inverse=True, normalize=True, threads=oracle.default_threads())
    assert np.count_nonzero((want != 0) & (np.abs(want) < np.finfo(np.float32).tiny)) > 1000
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("extents,inverse", [([4096, 64], True), ([64, 64, 64], False), ([64, 64, 64], True),
                                             ([128, 2, 256], True)])
def test_rank_n_column_passes(torch_gpu, lib, stream, extents, inverse):
    # The innermost axis as rows, every other axis as in-place column passes
    # of at most 2^7 rows (a 2^12 axis as two); per-axis normalisation.
    batch, n = 2, int(np.prod(extents))
    x = np.random.default_rng(33).standard_normal((batch, n)).astype(np.float32)
    t = cb.describe(cb.Operator.FWHT, cb.DataType.FP32, extents, compute=cb.ComputeType.FP32, batch=batch,
                    inverse=inverse, normalize_inverse=inverse)
    with cb.Plan(lib, t) as plan:
        assert "fwht-columns[" in plan.algorithm_name()
    got = run_plan(torch_gpu, lib, t, x, stream)
    want = oracle.fwht_f32(x, inverse=inverse, normalize=inverse)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_zero_extended_long_rows(torch_gpu, lib, stream):
    # 20000 logical points run at 2^15: the forward input is zero-extended,
    # the output holds all 2^15 points (reference docs/c_api.md:74-79).
    batch, n, padded = 2, 20000, 1 << 15
    x = np.random.default_rng(32).standard_normal((batch, n)).astype(np.float32)
    t = cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [n], compute=cb.ComputeType.FP32, batch=batch,
                    length_mode=cb.LengthMode.ZERO_EXTENDED_EMBEDDING)
    got = run_plan(torch_gpu, lib, t, x, stream).reshape(batch, padded)
    full = np.zeros((batch, padded), np.float32)
    full[:, :n] = x
    np.testing.assert_array_equal(got.view(np.uint32), oracle.fwht_f32(full).view(np.uint32))
