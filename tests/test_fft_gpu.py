"""Complex FFT parity on the GPU through the C ABI.

The contract is rel-L2 <= 1e-5 per transform against the reference's own
output (COMPLEX_FP32 storage, FP32 compute): the oracle restates the
reference CPU path (reference_fft: bit reversal, radix-2 with double-precision
twiddles per butterfly, float storage; src/butterfly_reference.cpp:392-433),
and every length from 2^1 to 2^24 -- C3 at full size, 1 x 2^24 and
1024 x 2^14 -- is compared with it per transform at 1e-5. numpy's complex128
FFT of the same complex64 input is a second, independent truth at the same
tolerance, so a kernel that agrees with the oracle only because both share a
mistake fails too.
"""
import numpy as np
import pytest

import cubutterfly_amd as cb
import oracle
from cubutterfly_amd import workloads
from gpu_util import run_plan

pytestmark = pytest.mark.gpu

TOL = 1e-5


def fft(log_n, batch, **kw):
    return cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [1 << log_n], compute=cb.ComputeType.FP32, batch=batch, **kw)


def truth(x, inverse=False, normalize=False):
    a = x.astype(np.complex128)
    if not inverse:
        return np.fft.fft(a, axis=-1)
    y = np.fft.ifft(a, axis=-1)  # 1/n included
    return y if normalize else y * a.shape[-1]


def worst_rel_l2(got, expected):
    got = got.reshape(expected.shape).astype(np.complex128)
    num = np.linalg.norm(got - expected, axis=-1)
    den = np.maximum(np.linalg.norm(expected, axis=-1), 1e-30)
    return float(np.max(num / den))


@pytest.mark.parametrize("rows,log_n", [(1, 24), (1024, 14)])
def test_c3_full_size(torch_gpu, lib, stream, rows, log_n):
    print(f"case C3 fft c64 {rows} x 2^{log_n}", flush=True)
    x = workloads.complex_input(log_n, rows, seed=3).reshape(rows, 1 << log_n)
    got = run_plan(torch_gpu, lib, fft(log_n, rows), x, stream)
    err = worst_rel_l2(got, oracle.fft_c64(x, threads=oracle.default_threads()).astype(np.complex128))
    assert err <= TOL, f"rel-L2 vs the reference CPU path {err}"
    err = worst_rel_l2(got, truth(x))
    assert err <= TOL, f"rel-L2 vs complex128 {err}"
    # Round trip (forward and inverse errors add: a property, not the parity bar) through the normalised inverse returns the input.
    back = run_plan(torch_gpu, lib, fft(log_n, rows, inverse=True, placement=cb.Placement.IN_PLACE), got, stream, in_place=True)
    err = worst_rel_l2(back, x.astype(np.complex128))
    assert err <= 2 * TOL, f"round trip rel-L2 {err}"


@pytest.mark.parametrize("log_n", list(range(1, 25)))
def test_forward_every_length(torch_gpu, lib, stream, log_n):
    batch = 37 if log_n <= 12 else 3 if log_n <= 20 else 1
    print(f"case fft forward log_n={log_n} batch={batch}", flush=True)
    x = workloads.complex_input(log_n, batch, seed=log_n).reshape(batch, 1 << log_n)
    got = run_plan(torch_gpu, lib, fft(log_n, batch), x, stream)
    err = worst_rel_l2(got, truth(x))
    assert err <= TOL, f"rel-L2 vs complex128 {err}"
    ref = oracle.fft_c64(x, threads=oracle.default_threads())
    err = worst_rel_l2(got, ref.astype(np.complex128))
    assert err <= TOL, f"rel-L2 vs the reference CPU path {err}"


@pytest.mark.parametrize("log_n", [1, 4, 9, 12, 13, 14, 15, 17, 20, 23])
@pytest.mark.parametrize("normalize", [True, False])
def test_inverse(torch_gpu, lib, stream, log_n, normalize):
    batch = 5 if log_n <= 17 else 1
    print(f"case fft inverse log_n={log_n} normalize={normalize}", flush=True)
    x = workloads.complex_input(log_n, batch, seed=100 + log_n).reshape(batch, 1 << log_n)
    got = run_plan(torch_gpu, lib, fft(log_n, batch, inverse=True, normalize_inverse=normalize), x, stream)
    err = worst_rel_l2(got, truth(x, inverse=True, normalize=normalize))
    assert err <= TOL, f"rel-L2 vs complex128 {err}"
    ref = oracle.fft_c64(x, inverse=True, normalize=normalize, threads=oracle.default_threads())
    err = worst_rel_l2(got, ref.astype(np.complex128))
    assert err <= TOL, f"rel-L2 vs the reference CPU path {err}"


@pytest.mark.parametrize("log_n,batch", [(3, 1000), (11, 7), (14, 9), (16, 4), (19, 2)])
def test_in_place(torch_gpu, lib, stream, log_n, batch):
    x = workloads.complex_input(log_n, batch, seed=9).reshape(batch, 1 << log_n)
    got = run_plan(torch_gpu, lib, fft(log_n, batch, placement=cb.Placement.IN_PLACE), x, stream, in_place=True)
    assert worst_rel_l2(got, truth(x)) <= TOL


def test_special_inputs(torch_gpu, lib, stream):
    # Impulse -> constant, constant -> scaled impulse, single tone -> one bin.
    log_n, n = 16, 1 << 16
    x = np.zeros((3, n), np.complex64)
    x[0, 0] = 1
    x[1, :] = 1
    k = 12345
    x[2] = np.exp(2j * np.pi * k * np.arange(n) / n).astype(np.complex64)
    got = run_plan(torch_gpu, lib, fft(log_n, 3), x, stream).reshape(3, n)
    np.testing.assert_allclose(got[0], np.ones(n), atol=1e-6)
    expected = np.zeros(n)
    expected[0] = n
    np.testing.assert_allclose(got[1], expected, atol=1e-6 * n)
    tone = np.zeros(n)
    tone[k] = n
    np.testing.assert_allclose(got[2], tone, atol=2e-5 * n)


def test_two_pass_needs_workspace(torch_gpu, lib, stream):
    with cb.Plan(lib, fft(16, 2), stream=stream) as plan:
        assert plan.workspace_size() == 2 * (1 << 16) * 8
    with cb.Plan(lib, fft(14, 2), stream=stream) as plan:
        assert plan.workspace_size() == 0
