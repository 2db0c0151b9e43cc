"""Bit-reversed logical orders of one-pass FFTs (n <= 2^14) in the kernel:
the input is read through the row bit reversal, the output keeps the DIF
result's own order (reference logical-order semantics, semantic_contract.cpp;
gather / scatter src/general_kernels.cu:475-535). Checked against the oracle
with the orders applied in numpy."""
import numpy as np
import pytest

import cubutterfly_amd as cb
import oracle
from gpu_util import run_plan

pytestmark = pytest.mark.gpu


def perm(log_n):
    n = 1 << log_n
    return np.array([int(format(i, f"0{log_n}b")[::-1], 2) if log_n else 0 for i in range(n)])


@pytest.mark.parametrize("log_n", [1, 4, 7, 10, 12, 13, 14])
@pytest.mark.parametrize("rin,rout", [(True, False), (False, True), (True, True)])
@pytest.mark.parametrize("inverse", [False, True])
def test_orders(torch_gpu, lib, stream, log_n, rin, rout, inverse):
    n = 1 << log_n
    batch = max(2, (1 << 16) >> log_n)
    rng = np.random.default_rng(log_n * 4 + rin * 2 + rout)
    x = (rng.standard_normal((batch, n)) + 1j * rng.standard_normal((batch, n))).astype(np.complex64)
    order = lambda rev: [cb.LogicalOrder.BIT_REVERSED if rev else cb.LogicalOrder.NATURAL]
    t = cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [n], compute=cb.ComputeType.FP32, batch=batch, inverse=inverse, input_orders=order(rin), output_orders=order(rout))
    with cb.Plan(lib, t) as plan:
        name = plan.algorithm_name()
        assert not name.startswith("semantic-boundary") and "-bitrev-" in name, name
        assert plan.workspace_size() == 0
    got = run_plan(torch_gpu, lib, t, x, stream).astype(np.complex128)
    p = perm(log_n)
    logical_in = x[:, p] if rin else x          # physical j holds logical bitrev(j)
    ref = oracle.fft_c64(logical_in, inverse=inverse, normalize=inverse,
                         threads=oracle.default_threads()).astype(np.complex128)
    if rout:
        ref = ref[:, p]
    err = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert err <= 1e-5, err


def test_round_trip_through_bit_reversed_spectrum(torch_gpu, lib, stream):
    # Forward with bit-reversed output, inverse with bit-reversed input: the
    # convolution-pipeline pattern, back to the input.
    n, batch = 1 << 14, 8
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((batch, n)) + 1j * rng.standard_normal((batch, n))).astype(np.complex64)
    fwd = cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [n], compute=cb.ComputeType.FP32, batch=batch, output_orders=[cb.LogicalOrder.BIT_REVERSED])
    inv = cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [n], compute=cb.ComputeType.FP32, batch=batch, inverse=True, input_orders=[cb.LogicalOrder.BIT_REVERSED])
    spectrum = run_plan(torch_gpu, lib, fwd, x, stream)
    back = run_plan(torch_gpu, lib, inv, spectrum, stream).astype(np.complex128)
    assert np.linalg.norm(back - x) / np.linalg.norm(x) <= 1e-5
