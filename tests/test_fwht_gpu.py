"""FWHT parity on the GPU, through the C ABI, against the CPU oracle.

FP32 (C1) must be bit-exact: integer inputs make every sum exact, and random
float inputs pin the stage order (a different bit order rounds differently).
FP16 final storage (C5) must satisfy the max-abs <= 2e-3 contract; the kernel is
stage-ordered, so it is also checked bit for bit.
"""
import numpy as np
import pytest

import cubutterfly_amd as cb
import oracle
from cubutterfly_amd import workloads
from golden import make_full_size_hashes as golden
from gpu_util import run_plan

pytestmark = pytest.mark.gpu

THREADS = oracle.default_threads()


def fwht32(n, batch, **kw):
    return cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [n], compute=cb.ComputeType.FP32, batch=batch, **kw)


def fwht16(n, batch, scale, **kw):
    return cb.describe(cb.Operator.FWHT, cb.DataType.FP16, [n], compute=cb.ComputeType.FP32, batch=batch, output_scale=scale, output_rounding=cb.OutputRounding.FINAL_STORAGE, **kw)


def random_floats(rows, n, seed):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((rows, n)) * np.exp(rng.standard_normal((rows, n)) * 3)).astype(np.float32)


def test_c1_full_size_bit_exact(torch_gpu, lib, stream):
    print("case C1 fwht fp32 4096 x 4096", flush=True)
    x = workloads.fwht_integer_input(12, 4096, seed=1)
    got = run_plan(torch_gpu, lib, fwht32(4096, 4096), x, stream)
    np.testing.assert_array_equal(got, oracle.fwht_f32(x, threads=THREADS))
    assert golden.sha256(got) == golden.load()["c1"]["output_sha256"]


@pytest.mark.parametrize("log_n", list(range(1, 14)))
@pytest.mark.parametrize("batch", [1, 5, 64])
def test_fp32_random_floats_bit_exact(torch_gpu, lib, stream, log_n, batch):
    print(f"case fwht fp32 log_n={log_n} batch={batch}", flush=True)
    x = random_floats(batch, 1 << log_n, seed=log_n * 100 + batch)
    got = run_plan(torch_gpu, lib, fwht32(1 << log_n, batch), x, stream)
    np.testing.assert_array_equal(got.view(np.uint32), oracle.fwht_f32(x).view(np.uint32))


@pytest.mark.parametrize("log_n,batch", [(5, 129), (7, 1000), (12, 3), (13, 2)])
def test_fp32_inverse_normalised_in_place(torch_gpu, lib, stream, log_n, batch):
    x = random_floats(batch, 1 << log_n, seed=7)
    got = run_plan(torch_gpu, lib, fwht32(1 << log_n, batch, inverse=True, placement=cb.Placement.IN_PLACE), x, stream,
                   in_place=True)
    expected = oracle.fwht_f32(x, inverse=True, normalize=True)
    np.testing.assert_array_equal(got.view(np.uint32), expected.view(np.uint32))
    raw = run_plan(torch_gpu, lib, fwht32(1 << log_n, batch, inverse=True, normalize_inverse=False), x, stream)
    np.testing.assert_array_equal(raw.view(np.uint32), oracle.fwht_f32(x).view(np.uint32))


def check_fp16(got, expected):
    err = np.max(np.abs(got.astype(np.float32) - expected.astype(np.float32)))
    assert err <= 2e-3, f"max abs err {err}"
    mismatches = int(np.count_nonzero(got.view(np.uint16) != expected.view(np.uint16)))
    assert mismatches == 0, f"{mismatches} outputs differ from the stage-ordered oracle"


@pytest.mark.parametrize("rows,n", [(16384, 4096), (524288, 128)])
def test_c5_quarot_full_size(torch_gpu, lib, stream, rows, n):
    print(f"case C5 fwht fp16 {rows} x {n}", flush=True)
    scale = float(np.float32(1.0 / np.sqrt(n)))
    x = workloads.quarot_input(rows, n, seed=5)
    got = run_plan(torch_gpu, lib, fwht16(n, rows, scale), x, stream)
    check_fp16(got, oracle.fwht_f16_final(x, scale, threads=THREADS))
    assert golden.sha256(got) == golden.load()["c5a" if n == 4096 else "c5b"]["output_sha256"]


@pytest.mark.parametrize("log_n", [1, 3, 5, 6, 8, 11, 13])
@pytest.mark.parametrize("inverse,normalize,scale", [(False, False, 1.0), (True, True, 0.375), (True, False, -0.75)])
def test_fp16_contract_variants(torch_gpu, lib, stream, log_n, inverse, normalize, scale):
    n = 1 << log_n
    rng = np.random.default_rng(61013 + n)
    x = (rng.integers(-1024, 1025, (37, n)).astype(np.float32) / 1024).astype(np.float16)
    t = fwht16(n, 37, scale, inverse=inverse, normalize_inverse=normalize)
    got = run_plan(torch_gpu, lib, t, x, stream)
    check_fp16(got, oracle.fwht_f16_final(x, scale, inverse=inverse, normalize=normalize))
