"""FWHT beyond one resident tile (n > 2^13): factored into axes of at most
2^12 points, lowest index bits first, which is the reference's stage order
(src/butterfly_reference.cpp:349-369), so results are bit-identical to the
oracle."""
import numpy as np
import pytest

import cubutterfly_amd as cb
import oracle
from gpu_util import run_plan

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
