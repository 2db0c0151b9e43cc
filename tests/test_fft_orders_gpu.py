"""Bit-reversed logical orders of FFTs in the kernels: one-pass FFTs
(n <= 2^14) read the input through the row bit reversal and keep the DIF
result's own order on output; two- and three-pass FFTs write a bit-reversed
output from their final row pass, each row back where it was read (reference
logical-order semantics, semantic_contract.cpp; gather / scatter
src/general_kernels.cu:475-535). Checked against the oracle with the orders
applied in numpy."""
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


# Two-pass lengths 2^15..2^22 and the three-pass lengths 2^23, 2^24, with
# non-default splits that MEASURE may pick.
@pytest.mark.parametrize("log_n,batch,algorithm", [
    (15, 8, None), (16, 5, None), (16, 3, "fft-c64-two-pass-r16-7x9"), (19, 2, None), (20, 2, None),
    (22, 1, None), (23, 1, None), (24, 1, None), (21, 1, "fft-c64-three-pass-r16-6x7x8"),
    (24, 1, "fft-c64-three-pass-r16-7x9x8")])
@pytest.mark.parametrize("inverse", [False, True])
def test_multi_pass_bit_reversed_output(torch_gpu, lib, stream, log_n, batch, algorithm, inverse):
    n = 1 << log_n
    print(f"case fft bitrev-out n=2^{log_n} batch={batch} {algorithm} inverse={inverse}", flush=True)
    rng = np.random.default_rng(log_n + 100 * inverse)
    x = (rng.standard_normal((batch, n)) + 1j * rng.standard_normal((batch, n))).astype(np.complex64)
    t = cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [n], compute=cb.ComputeType.FP32, batch=batch,
                    inverse=inverse, output_orders=[cb.LogicalOrder.BIT_REVERSED])
    kw = {} if algorithm is None else {"algorithm": algorithm + "-bitrev-out"}
    with cb.Plan(lib, t, **kw) as plan:
        name = plan.algorithm_name()
    assert name.endswith("-bitrev-out") and "pass" in name and not name.startswith("semantic-boundary"), name
    got = run_plan(torch_gpu, lib, t, x, stream, **kw).astype(np.complex128)
    ref = (np.fft.ifft if inverse else np.fft.fft)(x.astype(np.complex128), axis=1)
    ref = ref[:, perm(log_n)]
    err = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert err <= 1e-5, err


def test_multi_pass_bit_reversed_input_uses_the_boundary(lib):
    # A bit-reversed input of a two-pass length gathers through the boundary.
    t = cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [1 << 16], compute=cb.ComputeType.FP32, batch=2,
                    input_orders=[cb.LogicalOrder.BIT_REVERSED])
    with cb.Plan(lib, t) as plan:
        assert plan.algorithm_name().startswith("semantic-boundary[fft-c64-two-pass-r16")


def test_multi_pass_round_trip_in_place(torch_gpu, lib, stream):
    # Forward 2^20 points to the bit-reversed spectrum (native), inverse from
    # it (through the boundary), in place: back to the input.
    n, batch = 1 << 20, 2
    rng = np.random.default_rng(12)
    x = (rng.standard_normal((batch, n)) + 1j * rng.standard_normal((batch, n))).astype(np.complex64)
    fwd = cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [n], compute=cb.ComputeType.FP32, batch=batch,
                      output_orders=[cb.LogicalOrder.BIT_REVERSED], placement=cb.Placement.IN_PLACE)
    inv = cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [n], compute=cb.ComputeType.FP32, batch=batch,
                      inverse=True, input_orders=[cb.LogicalOrder.BIT_REVERSED])
    spectrum = run_plan(torch_gpu, lib, fwd, x, stream, in_place=True)
    back = run_plan(torch_gpu, lib, inv, spectrum, stream).astype(np.complex128)
    assert np.linalg.norm(back - x) / np.linalg.norm(x) <= 1e-5
