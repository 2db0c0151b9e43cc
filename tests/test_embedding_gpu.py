"""Zero-extended embedding on the GPU (reference docs/c_api.md:74-79;
src/c_api.cpp:5231-5245 pack, 5312-5325 scatter): the forward transform of
each row zero-padded to the next power of two, and the inverse cut back to
the logical length, against the oracle on padded rows (FWHT bit-exact, NTT
exact, FFT also against numpy's padded FFT)."""
import numpy as np
import pytest

import cubutterfly_amd as cb
import oracle
from gpu_util import run_plan

pytestmark = pytest.mark.gpu

Q = 998244353
EMB = cb.LengthMode.ZERO_EXTENDED_EMBEDDING


def pow2(n):
    p = 1
    while p < n:
        p *= 2
    return p


def pad(x, p):
    out = np.zeros(x.shape[:-1] + (p,), x.dtype)
    out[..., : x.shape[-1]] = x
    return out


@pytest.mark.parametrize("n", [3, 100, 1000, 5000])
def test_fwht_forward(torch_gpu, lib, stream, n):
    batch = 3
    x = np.random.default_rng(n).standard_normal((batch, n)).astype(np.float32)
    t = cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [n], compute=cb.ComputeType.FP32, batch=batch, length_mode=EMB)
    got = run_plan(torch_gpu, lib, t, x, stream)
    expected = oracle.fwht_f32(pad(x, pow2(n)))
    np.testing.assert_array_equal(got.reshape(batch, -1).view(np.uint32), expected.view(np.uint32))


def test_fwht_inverse_cuts(torch_gpu, lib, stream):
    n, batch = 100, 4
    y = np.random.default_rng(1).standard_normal((batch, 128)).astype(np.float32)
    t = cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [n], compute=cb.ComputeType.FP32, batch=batch, inverse=True, length_mode=EMB)
    got = run_plan(torch_gpu, lib, t, y, stream)
    expected = oracle.fwht_f32(y, inverse=True, normalize=True)[:, :n]
    np.testing.assert_array_equal(got.reshape(batch, n).view(np.uint32), expected.view(np.uint32))


@pytest.mark.parametrize("n", [5, 100, 3000, 40000])
@pytest.mark.parametrize("inverse", [False, True])
def test_fft(torch_gpu, lib, stream, n, inverse):
    batch, p = 2, pow2(n)
    rng = np.random.default_rng(n + inverse)
    m = p if inverse else n
    x = (rng.standard_normal((batch, m)) + 1j * rng.standard_normal((batch, m))).astype(np.complex64)
    t = cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [n], compute=cb.ComputeType.FP32, batch=batch, inverse=inverse, length_mode=EMB)
    got = run_plan(torch_gpu, lib, t, x, stream).reshape(batch, -1).astype(np.complex128)
    if inverse:
        ref = np.fft.ifft(x.astype(np.complex128), axis=-1)[:, :n]
    else:
        ref = np.fft.fft(x.astype(np.complex128), n=p, axis=-1)
    assert got.shape == ref.shape
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 1e-5


@pytest.mark.parametrize("n", [100, 5000])
@pytest.mark.parametrize("inverse", [False, True])
def test_ntt(torch_gpu, lib, stream, n, inverse):
    batch, p = 3, pow2(n)
    rng = np.random.default_rng(n)
    x = rng.integers(0, Q, (batch, p if inverse else n)).astype(np.uint32)
    t = cb.describe(cb.Operator.NTT, cb.DataType.UINT32, [n], compute=cb.ComputeType.UINT32, batch=batch, modulus=Q, word_bits=32, inverse=inverse, length_mode=EMB)
    got = run_plan(torch_gpu, lib, t, x, stream).reshape(batch, -1)
    if inverse:
        expected = oracle.ntt_cyclic(x.astype(np.uint64), Q, inverse=True)[:, :n]
    else:
        expected = oracle.ntt_cyclic(pad(x.astype(np.uint64), p), Q)
    np.testing.assert_array_equal(got.astype(np.uint64), expected)


@pytest.mark.parametrize("inverse", [False, True])
def test_rank2_fft(torch_gpu, lib, stream, inverse):
    shape, batch = (5, 12), 2
    phys = (8, 16)
    rng = np.random.default_rng(7)
    side = phys if inverse else shape
    x = (rng.standard_normal((batch,) + side) + 1j * rng.standard_normal((batch,) + side)).astype(np.complex64)
    t = cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, list(shape), compute=cb.ComputeType.FP32, batch=batch, inverse=inverse, length_mode=EMB)
    got = run_plan(torch_gpu, lib, t, x, stream).astype(np.complex128)
    if inverse:
        ref = np.fft.ifftn(x.astype(np.complex128), axes=(1, 2))[:, :5, :12]
    else:
        ref = np.fft.fftn(x.astype(np.complex128), s=phys, axes=(1, 2))
    got = got.reshape(ref.shape)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 1e-5


def test_strided_input(torch_gpu, lib, stream):
    # Forward input interleaved (stride 2), output packed at the padded length.
    n, batch = 100, 3
    rng = np.random.default_rng(3)
    flat = (rng.standard_normal(2 * n * batch) + 1j * rng.standard_normal(2 * n * batch)).astype(np.complex64)
    t = cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [n], compute=cb.ComputeType.FP32, batch=batch, length_mode=EMB, input_strides=[2], input_batch_stride=2 * n)
    span = 2 * n * (batch - 1) + 2 * (n - 1) + 1
    got = run_plan(torch_gpu, lib, t, flat[:span], stream).reshape(batch, 128).astype(np.complex128)
    rows = flat[: 2 * n * batch].reshape(batch, 2 * n)[:, ::2]
    ref = np.fft.fft(rows.astype(np.complex128), n=128, axis=-1)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 1e-5
