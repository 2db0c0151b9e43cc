"""NTT parity on the GPU through the C ABI: bit-exact against the CPU oracle.

C2 (negacyclic u32, n = 2^16, batch 64) at full size, plus cyclic/negacyclic
u32/u64 over lengths 2..2^20, both word sizes' lazy and strict arithmetic
(q below / above 2^30 and 2^62), bit-reversed layouts (the reference's
output-order contract, tests/test_c_api.c:920-1010), non-canonical inputs
(reduced like reference_ntt, src/reference.cpp:601-603) and in-place plans.
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
Q30 = workloads.C2_MODULUS            # 1073479681, tests/test_ntt.cpp:251
Q64 = 576460756061519873              # tests/test_c_api.c:934
QDEF = 1152921504606584833            # include/cuntt/ntt.hpp:17
Q63 = 9223372036752015361             # largest prime < 2^63 with 2^21 | q - 1 (strict u64 path)


def ntt(n, batch, q, bits, inverse=False, ring=cb.NttRing.CYCLIC, **kw):
    storage = cb.DataType.UINT32 if bits == 32 else cb.DataType.UINT64
    compute = cb.ComputeType.UINT32 if bits == 32 else cb.ComputeType.UINT64
    return cb.describe(cb.Operator.NTT, storage, [n], compute=compute, batch=batch, modulus=q, word_bits=bits, inverse=inverse, ntt_ring=ring, **kw)


def as_words(a, bits):
    return np.ascontiguousarray(a, dtype=np.uint32 if bits == 32 else np.uint64)


def bitrev_perm(log_n):
    idx = np.arange(1 << log_n)
    rev = np.zeros_like(idx)
    for b in range(log_n):
        rev |= ((idx >> b) & 1) << (log_n - 1 - b)
    return rev


def test_c2_negacyclic_full_size(torch_gpu, lib, stream):
    print("case C2 negacyclic u32 n=2^16 batch=64", flush=True)
    x = workloads.ntt_input(16, 64, Q30, seed=1).astype(np.uint32)
    neg = cb.NttRing.NEGACYCLIC
    fwd = run_plan(torch_gpu, lib, ntt(1 << 16, 64, Q30, 32, ring=neg), x, stream)
    expected = oracle.ntt_negacyclic(x.astype(np.uint64), Q30, threads=THREADS)
    np.testing.assert_array_equal(fwd.astype(np.uint64), expected)
    assert golden.sha256(fwd) == golden.load()["c2"]["output_sha256"]
    back = run_plan(torch_gpu, lib, ntt(1 << 16, 64, Q30, 32, inverse=True, ring=neg), fwd, stream)
    np.testing.assert_array_equal(back, x)
    inv_ref = oracle.ntt_negacyclic(x.astype(np.uint64), Q30, inverse=True, threads=THREADS)
    inv = run_plan(torch_gpu, lib, ntt(1 << 16, 64, Q30, 32, inverse=True, ring=neg), x, stream)
    np.testing.assert_array_equal(inv.astype(np.uint64), inv_ref)


CASES = [(q, bits, log_n, batch)
         for q, bits in [(Q30, 32), (2013265921, 32), (Q64, 64), (QDEF, 64), (Q63, 64)]
         for log_n, batch in [(1, 3), (4, 17), (7, 300), (10, 5), (12, 3), (13, 2), (14, 3), (16, 2),
                              (17, 1), (20, 1)]
         if (q - 1) % (2 << log_n) == 0]


@pytest.mark.parametrize("q,bits,log_n,batch", CASES)
@pytest.mark.parametrize("ring", [cb.NttRing.CYCLIC, cb.NttRing.NEGACYCLIC])
def test_ntt_matches_oracle(torch_gpu, lib, stream, q, bits, log_n, batch, ring):
    print(f"case ntt q={q} bits={bits} log_n={log_n} batch={batch} ring={int(ring)}", flush=True)
    x = as_words(workloads.ntt_input(log_n, batch, q, seed=log_n), bits)
    n = 1 << log_n
    ref_fn = oracle.ntt_negacyclic if ring == cb.NttRing.NEGACYCLIC else oracle.ntt_cyclic
    expected = ref_fn(x.astype(np.uint64), q, threads=THREADS)
    got = run_plan(torch_gpu, lib, ntt(n, batch, q, bits, ring=ring), x, stream)
    np.testing.assert_array_equal(got.astype(np.uint64), expected)
    back = run_plan(torch_gpu, lib, ntt(n, batch, q, bits, inverse=True, ring=ring), got, stream)
    np.testing.assert_array_equal(back, x)


@pytest.mark.parametrize("q,bits", [(998244353, 32), (Q64, 64)])
@pytest.mark.parametrize("log_n", [3, 9, 14, 16])
@pytest.mark.parametrize("inverse", [False, True])
def test_bit_reversed_layouts(torch_gpu, lib, stream, q, bits, log_n, inverse):
    # Reference contract: logical coordinate i of a BIT_REVERSED side lives at
    # reverse_bits(i) (cubutterfly.h:23-30; tests/test_c_api.c:972-977).
    batch = 2
    n = 1 << log_n
    perm = bitrev_perm(log_n)
    x = as_words(workloads.ntt_input(log_n, batch, q, seed=5), bits)
    natural = run_plan(torch_gpu, lib, ntt(n, batch, q, bits, inverse=inverse), x, stream)
    out_rev = run_plan(torch_gpu, lib, ntt(n, batch, q, bits, inverse=inverse,
                                           ntt_output_layout=cb.NttLayout.BIT_REVERSED), x, stream)
    np.testing.assert_array_equal(out_rev, natural[:, perm])
    in_rev = run_plan(torch_gpu, lib, ntt(n, batch, q, bits, inverse=inverse,
                                          input_orders=[cb.LogicalOrder.BIT_REVERSED],
                                          output_orders=[cb.LogicalOrder.NATURAL]), x[:, perm], stream)
    np.testing.assert_array_equal(in_rev, natural)


@pytest.mark.parametrize("q,bits,log_n", [(Q30, 32, 10), (Q30, 32, 16), (QDEF, 64, 16)])
def test_non_canonical_inputs_are_reduced(torch_gpu, lib, stream, q, bits, log_n):
    rng = np.random.default_rng(3)
    top = (1 << bits) - 1
    x = rng.integers(0, top, (2, 1 << log_n), dtype=np.uint64, endpoint=True)
    x[0, :4] = [top, top - 1, q, 2 * q]
    x = as_words(x, bits)
    got = run_plan(torch_gpu, lib, ntt(1 << log_n, 2, q, bits), x, stream)
    expected = oracle.ntt_cyclic(x.astype(np.uint64) % np.uint64(q), q)
    np.testing.assert_array_equal(got.astype(np.uint64), expected)


@pytest.mark.parametrize("log_n", [6, 16])
def test_in_place(torch_gpu, lib, stream, log_n):
    x = workloads.ntt_input(log_n, 4, Q30, seed=2).astype(np.uint32)
    t = ntt(1 << log_n, 4, Q30, 32, ring=cb.NttRing.NEGACYCLIC, placement=cb.Placement.IN_PLACE)
    got = run_plan(torch_gpu, lib, t, x, stream, in_place=True)
    np.testing.assert_array_equal(got.astype(np.uint64), oracle.ntt_negacyclic(x.astype(np.uint64), Q30))


def test_explicit_psi(torch_gpu, lib, stream):
    # A caller-chosen psi (here the cube of the default) defines w = psi^2.
    log_n, q = 8, Q30
    w = oracle.find_primitive_root(log_n, q)
    psi = pow(oracle.find_psi(log_n, q, w), 3, q)
    x = workloads.ntt_input(log_n, 3, q, seed=9)
    got = run_plan(torch_gpu, lib, ntt(1 << log_n, 3, q, 32, ring=cb.NttRing.NEGACYCLIC, ntt_psi=psi),
                   x.astype(np.uint32), stream)
    expected = oracle.rns(x, [q] * 3, [psi] * 3)  # natural-order negacyclic with explicit root
    np.testing.assert_array_equal(got.astype(np.uint64), expected)
