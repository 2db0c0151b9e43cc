"""Seeded random parity over the whole public surface, on the GPU: every
operator with random lengths and batches, strided, pitched and bit-reversed
sides (the semantic boundary, reference src/c_api.cpp:5064-5085), NTT
layouts and rings, in-place plans, long FWHTs (factored and FP32-promoted),
rank-2 / rank-3 composites, the zero-extended embedding, MEASURE selection
with its cache replay, and RNS plans through the RNS C ABI (random
domains, roots, polynomial slots, orders and placements; the layout rules of
the reference's tests/test_rns_ntt.cu:113-162). Each case is checked against the CPU oracle
(bit-exact for FWHT and NTT; FFT within rel-L2 1e-5 against numpy in
complex128), and every output element outside the output layout must keep
its sentinel. Cases are drawn from fixed seeds, so a failure names a case
that reproduces."""
import random

import numpy as np
import pytest

import cubutterfly_amd as cb
import oracle
from cubutterfly_amd import rns
from gpu_util import run_plan, to_device, to_host

pytestmark = pytest.mark.gpu

U32 = [998244353, 1073479681, 2013265921, 469762049]
U64 = [576460756061519873, 1152921504606584833, 1152921504577486849, 9223372036752015361]
ORDER = {False: cb.LogicalOrder.NATURAL, True: cb.LogicalOrder.BIT_REVERSED}


def two_adic(x):
    return (x & -x).bit_length() - 1


def bitrev(j, log_n):
    r = np.zeros_like(j)
    for b in range(log_n):
        r |= ((j >> b) & 1) << (log_n - 1 - b)
    return r


def batch_stride(n, stride, code):
    """code 0: the axis span; -p: the span plus p padding elements."""
    span = (n - 1) * stride + 1
    return span - code if code < 0 else span


def positions(n, batch, stride, code, rev):
    j = np.arange(n, dtype=np.int64)
    r = bitrev(j, n.bit_length() - 1) if rev else j
    return np.arange(batch, dtype=np.int64)[:, None] * batch_stride(n, stride, code) + r[None, :] * stride


def span(n, batch, stride, code):
    return (n - 1) * stride + (batch - 1) * batch_stride(n, stride, code) + 1


def execute(torch, lib, stream, t, x_flat, out_len, sentinel):
    x = to_device(torch, x_flat)
    y = to_device(torch, np.full(out_len, sentinel, dtype=x_flat.dtype))
    with cb.Plan(lib, t, stream=stream) as plan:
        assert plan.input_size() == x.numel() * x.element_size()
        assert plan.output_size() == y.numel() * y.element_size()
        ws = plan.workspace_size()
        buf = torch.empty(ws, dtype=torch.uint8, device="cuda") if ws else None
        if buf is not None:
            plan.set_workspace(buf, ws)
        plan.execute(x, y)
        torch.cuda.synchronize()
        name = plan.algorithm_name()
    return to_host(torch, y, x_flat.dtype), name


def layout_case(torch, lib, stream, rng, index):
    """One rank-1 plan with random sides; returns (description, ok)."""
    op = rng.choice(["fwht32", "fwht16", "fft", "ntt32", "ntt64"])
    batch = rng.randint(1, 5)
    sides = [(rng.choice([1, 1, 2, 3, 5]), rng.choice([0, 0, -rng.randint(1, 9)]), rng.random() < 0.4)
             for _ in range(2)]
    (si, bi, ri), (so, bo, ro) = sides
    data = np.random.default_rng(index)
    kw = {}
    if op == "fwht32":
        log_n = rng.randint(1, 17)
        storage, compute, dt, opc = cb.DataType.FP32, cb.ComputeType.FP32, np.float32, cb.Operator.FWHT
        inv = rng.random() < 0.3
        kw = dict(inverse=inv, normalize_inverse=inv and rng.random() < 0.5)
    elif op == "fwht16":
        log_n = rng.randint(1, 16)
        storage, compute, dt, opc = cb.DataType.FP16, cb.ComputeType.FP32, np.float16, cb.Operator.FWHT
        scale = float(np.float32(rng.choice([1.0, (1 << log_n) ** -0.5, 0.37])))
        kw = dict(output_scale=scale, output_rounding=cb.OutputRounding.FINAL_STORAGE)
    elif op == "fft":
        log_n = rng.randint(1, 16)
        storage, compute, dt, opc = cb.DataType.COMPLEX_FP32, cb.ComputeType.FP32, np.complex64, cb.Operator.FFT
        inv = rng.random() < 0.5
        kw = dict(inverse=inv, normalize_inverse=inv and rng.random() < 0.5)
    else:
        bits = 32 if op == "ntt32" else 64
        q = rng.choice(U32 if bits == 32 else U64)
        ring = rng.choice([cb.NttRing.CYCLIC, cb.NttRing.NEGACYCLIC])
        log_n = rng.randint(1, min(15, two_adic(q - 1) - (ring == cb.NttRing.NEGACYCLIC)))
        storage = cb.DataType.UINT32 if bits == 32 else cb.DataType.UINT64
        compute = cb.ComputeType.UINT32 if bits == 32 else cb.ComputeType.UINT64
        dt, opc = (np.uint32 if bits == 32 else np.uint64), cb.Operator.NTT
        kw = dict(modulus=q, word_bits=bits, ntt_ring=ring, inverse=rng.random() < 0.5)
    n = 1 << log_n
    n_in = span(n, batch, si, bi)
    if dt == np.complex64:
        x_flat = (data.standard_normal(n_in) + 1j * data.standard_normal(n_in)).astype(dt)
    elif dt in (np.uint32, np.uint64):
        x_flat = data.integers(0, kw["modulus"], n_in, dtype=np.uint64).astype(dt)
    elif dt == np.float16:
        x_flat = data.standard_normal(n_in).astype(dt)
    else:
        x_flat = (data.integers(-8, 9, n_in) + data.standard_normal(n_in)).astype(dt)
    rows = x_flat[positions(n, batch, si, bi, ri)]
    out_pos = positions(n, batch, so, bo, ro)
    out_len = span(n, batch, so, bo)
    t = cb.describe(opc, storage, [n], batch=batch, compute=compute, input_strides=[si],
                    input_batch_stride=batch_stride(n, si, bi), output_strides=[so],
                    output_batch_stride=batch_stride(n, so, bo), input_orders=[ORDER[ri]], output_orders=[ORDER[ro]],
                    **kw)
    sentinel = dt(3)
    got, name = execute(torch, lib, stream, t, x_flat, out_len, sentinel)
    desc = f"{op} n={n} batch={batch} in={sides[0]} out={sides[1]} {kw} [{name}]"
    mask = np.ones(out_len, bool)
    mask[out_pos.ravel()] = False
    if not np.all(got[mask] == sentinel):
        return desc + ": elements outside the output layout changed", False
    if op == "fwht32":
        want = oracle.fwht_f32(rows, inverse=kw["inverse"], normalize=kw["normalize_inverse"])
        return desc, np.array_equal(got[out_pos].view(np.uint32), want.view(np.uint32))
    if op == "fwht16":
        want = oracle.fwht_f16_final(rows, kw["output_scale"])
        return desc, np.array_equal(got[out_pos].view(np.uint16), want.view(np.uint16))
    if op == "fft":
        want = oracle.fft_c64(rows, inverse=kw["inverse"], normalize=kw["normalize_inverse"]).astype(np.complex128)
        err = np.linalg.norm(got[out_pos].astype(np.complex128) - want) / np.linalg.norm(want)
        return desc + f" rel-L2 {err:.2e}", err <= 1e-5
    ref = oracle.ntt_negacyclic if kw["ntt_ring"] == cb.NttRing.NEGACYCLIC else oracle.ntt_cyclic
    want = ref(rows.astype(np.uint64), kw["modulus"], inverse=kw["inverse"])
    return desc, np.array_equal(got[out_pos].astype(np.uint64), want)


def ntt_case(torch, lib, stream, rng, index):
    """Packed NTT with layout fields, rings and in-place plans up to 2^20 points."""
    bits = rng.choice([32, 64])
    q = rng.choice(U32 if bits == 32 else U64)
    ring = rng.choice([cb.NttRing.CYCLIC, cb.NttRing.NEGACYCLIC])
    log_n = rng.randint(1, min(20, two_adic(q - 1) - (ring == cb.NttRing.NEGACYCLIC)))
    batch = rng.randint(1, max(1, min(6, (1 << 20) >> log_n)))
    inv, lin, lout, in_place = rng.random() < 0.5, rng.random() < 0.4, rng.random() < 0.4, rng.random() < 0.3
    kw = dict(modulus=q, word_bits=bits, ntt_ring=ring, inverse=inv)
    if lin:
        kw["ntt_input_layout"] = cb.NttLayout.BIT_REVERSED
    if lout:
        kw["ntt_output_layout"] = cb.NttLayout.BIT_REVERSED
    if in_place:
        kw["placement"] = cb.Placement.IN_PLACE
    t = cb.describe(cb.Operator.NTT, cb.DataType.UINT32 if bits == 32 else cb.DataType.UINT64, [1 << log_n],
                    compute=cb.ComputeType.UINT32 if bits == 32 else cb.ComputeType.UINT64, batch=batch, **kw)
    logical = np.random.default_rng(index).integers(0, q, (batch, 1 << log_n), dtype=np.uint64)
    perm = bitrev(np.arange(1 << log_n), log_n)
    ref = oracle.ntt_negacyclic if ring == cb.NttRing.NEGACYCLIC else oracle.ntt_cyclic
    want = ref(logical, q, inverse=inv)
    want = want[:, perm] if lout else want
    stored = np.ascontiguousarray(logical[:, perm] if lin else logical)
    got = run_plan(torch, lib, t, stored.astype(np.uint32 if bits == 32 else np.uint64), stream, in_place=in_place)
    desc = f"u{bits} ntt q={q} ring={int(ring)} n=2^{log_n} batch={batch} inverse={inv} layouts=({lin},{lout}) " \
           f"in_place={in_place}"
    return desc, np.array_equal(got.astype(np.uint64), want)


def fft_case(torch, lib, stream, rng, index):
    """Packed FFT to 2^22 points with orders, normalisation and in-place plans."""
    log_n = rng.randint(1, 22)
    batch = rng.randint(1, max(1, min(5, (1 << 22) >> log_n)))
    inv = rng.random() < 0.5
    norm = inv and rng.random() < 0.5
    ri, ro = rng.random() < 0.3, rng.random() < 0.3
    in_place = rng.random() < 0.3 and ri == ro
    kw = dict(inverse=inv, normalize_inverse=norm)
    if in_place:
        kw["placement"] = cb.Placement.IN_PLACE
    t = cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [1 << log_n], compute=cb.ComputeType.FP32,
                    batch=batch, input_orders=[ORDER[ri]], output_orders=[ORDER[ro]], **kw)
    data = np.random.default_rng(index)
    shape = (batch, 1 << log_n)
    logical = (data.standard_normal(shape) + 1j * data.standard_normal(shape)).astype(np.complex64)
    perm = bitrev(np.arange(1 << log_n), log_n)
    want = (np.fft.ifft if inv else np.fft.fft)(logical.astype(np.complex128), axis=1)
    if inv and not norm:
        want = want * (1 << log_n)
    want = want[:, perm] if ro else want
    stored = np.ascontiguousarray(logical[:, perm] if ri else logical)
    got = run_plan(torch, lib, t, stored, stream, in_place=in_place).astype(np.complex128)
    err = np.linalg.norm(got - want) / np.linalg.norm(want)
    return f"fft n=2^{log_n} batch={batch} inverse={inv} normalize={norm} orders=({ri},{ro}) in_place={in_place} " \
           f"rel-L2 {err:.2e}", err <= 1e-5


def composite_case(torch, lib, stream, rng, index):
    """Rank 2 or 3: FFT against numpy fftn, FWHT (integer data, exact in any
    order) against the flat oracle, cyclic NTT against the oracle per axis."""
    op = rng.choice(["fft", "fwht", "ntt"])
    rank = rng.choice([2, 2, 3])
    logs = [rng.randint(1, 10) for _ in range(rank)]
    while sum(logs) > 20:
        k = rng.randrange(rank)
        logs[k] = max(1, logs[k] - 1)
    ext = [1 << l for l in logs]
    batch = rng.randint(1, 3)
    shape = (batch, *ext)
    inv = rng.random() < 0.5
    data = np.random.default_rng(index)
    desc = f"rank-{rank} {op} extents={ext} batch={batch} inverse={inv}"
    if op == "fft":
        x = (data.standard_normal(shape) + 1j * data.standard_normal(shape)).astype(np.complex64)
        t = cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, ext, compute=cb.ComputeType.FP32, batch=batch,
                        inverse=inv, normalize_inverse=inv)
        want = (np.fft.ifftn if inv else np.fft.fftn)(x.astype(np.complex128), axes=tuple(range(1, rank + 1)))
        got = run_plan(torch, lib, t, x, stream).astype(np.complex128)
        err = np.linalg.norm(got - want) / np.linalg.norm(want)
        return desc + f" rel-L2 {err:.2e}", err <= 1e-5
    if op == "fwht":
        x = data.integers(-4, 5, shape).astype(np.float32)
        t = cb.describe(cb.Operator.FWHT, cb.DataType.FP32, ext, compute=cb.ComputeType.FP32, batch=batch)
        want = oracle.fwht_f32(x.reshape(batch, -1)).reshape(shape)
        return desc, np.array_equal(run_plan(torch, lib, t, x, stream).reshape(shape), want)
    q = 998244353
    x = data.integers(0, q, shape, dtype=np.uint64)
    t = cb.describe(cb.Operator.NTT, cb.DataType.UINT32, ext, compute=cb.ComputeType.UINT32, batch=batch,
                    modulus=q, word_bits=32, inverse=inv)
    want = x.copy()
    for axis in range(1, rank + 1):
        moved = np.moveaxis(want, axis, -1)
        flat = np.ascontiguousarray(moved.reshape(-1, moved.shape[-1]))
        want = np.moveaxis(oracle.ntt_cyclic(flat, q, inverse=inv).reshape(moved.shape), -1, axis)
    got = run_plan(torch, lib, t, x.astype(np.uint32), stream).reshape(shape).astype(np.uint64)
    return desc, np.array_equal(got, want)


def embedding_case(torch, lib, stream, rng, index):
    """The zero-extended embedding (reference docs/c_api.md:74-79): each axis
    runs at its next power of two; the forward takes the logical extents and
    returns the padded ones, the inverse the reverse. Checked against the
    transform of the zero-padded input (forward) and the cut transform of the
    padded input (inverse)."""
    op = rng.choice(["fft", "fwht", "ntt"])
    rank = rng.choice([1, 1, 2])
    logical = [rng.randint(3, 5000 if rank == 1 else 300) for _ in range(rank)]
    padded = [1 << (e - 1).bit_length() for e in logical]
    batch = rng.randint(1, 3)
    inverse = rng.random() < 0.5
    data = np.random.default_rng(index)
    in_ext, out_ext = (padded, logical) if inverse else (logical, padded)
    shape_in = (batch, *in_ext)
    axes = tuple(range(1, rank + 1))
    if op == "fft":
        x = (data.standard_normal(shape_in) + 1j * data.standard_normal(shape_in)).astype(np.complex64)
        t = cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, logical, compute=cb.ComputeType.FP32,
                        batch=batch, inverse=inverse, normalize_inverse=inverse,
                        length_mode=cb.LengthMode.ZERO_EXTENDED_EMBEDDING)
    elif op == "fwht":
        x = data.integers(-4, 5, shape_in).astype(np.float32)
        t = cb.describe(cb.Operator.FWHT, cb.DataType.FP32, logical, compute=cb.ComputeType.FP32, batch=batch,
                        length_mode=cb.LengthMode.ZERO_EXTENDED_EMBEDDING, inverse=inverse)
    else:
        q = 998244353
        x = data.integers(0, q, shape_in, dtype=np.uint64).astype(np.uint32)
        t = cb.describe(cb.Operator.NTT, cb.DataType.UINT32, logical, compute=cb.ComputeType.UINT32, batch=batch,
                        modulus=q, word_bits=32, inverse=inverse, length_mode=cb.LengthMode.ZERO_EXTENDED_EMBEDDING)
    full = np.zeros((batch, *padded), dtype=x.dtype)
    full[(slice(None),) + tuple(slice(0, e) for e in in_ext)] = x
    if op == "fft":
        want = (np.fft.ifftn if inverse else np.fft.fftn)(full.astype(np.complex128), axes=axes)
    elif op == "fwht":
        # normalize_inverse defaults to true; integer data and a power-of-two
        # 1/n keep every order of the additions exact
        want = oracle.fwht_f32(full.reshape(batch, -1), inverse=inverse, normalize=inverse).reshape(full.shape)
    else:
        want = full.astype(np.uint64)
        for axis in axes:
            moved = np.moveaxis(want, axis, -1)
            flat = np.ascontiguousarray(moved.reshape(-1, moved.shape[-1]))
            want = np.moveaxis(oracle.ntt_cyclic(flat, q, inverse=inverse).reshape(moved.shape), -1, axis)
    want = want[(slice(None),) + tuple(slice(0, e) for e in out_ext)]
    got = run_plan(torch, lib, t, np.ascontiguousarray(x), stream).reshape((batch, *out_ext))
    desc = f"embedded {op} logical={logical} batch={batch} inverse={inverse}"
    if op == "fft":
        err = np.linalg.norm(got.astype(np.complex128) - want) / np.linalg.norm(want)
        return desc + f" rel-L2 {err:.2e}", err <= 1e-5
    if op == "fwht":
        return desc, np.array_equal(got, want)
    return desc, np.array_equal(got.astype(np.uint64), want)


def measure_case(torch, lib, stream, rng, index):
    """MEASURE on a random packed rank-1 request with a fresh selection cache:
    the measured plan matches the oracle, and a DEFAULT plan on the same
    cache replays the same lowering from it."""
    import tempfile
    op = rng.choice(["fft", "fwht32", "fwht16", "ntt32", "ntt64"])
    data = np.random.default_rng(index)
    if op == "fft":
        log_n = rng.randint(10, 20)
        batch = max(1, (1 << 18) >> log_n)
        t = cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [1 << log_n], compute=cb.ComputeType.FP32,
                        batch=batch)
        x = (data.standard_normal((batch, 1 << log_n)) + 1j * data.standard_normal((batch, 1 << log_n))).astype(
            np.complex64)
    elif op.startswith("fwht"):
        log_n = rng.randint(5, 13)
        batch = max(1, (1 << 18) >> log_n)
        if op == "fwht32":
            t = cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [1 << log_n], compute=cb.ComputeType.FP32, batch=batch)
            x = data.standard_normal((batch, 1 << log_n)).astype(np.float32)
        else:
            scale = float(np.float32((1 << log_n) ** -0.5))
            t = cb.describe(cb.Operator.FWHT, cb.DataType.FP16, [1 << log_n], compute=cb.ComputeType.FP32,
                            batch=batch, output_scale=scale, output_rounding=cb.OutputRounding.FINAL_STORAGE)
            x = data.standard_normal((batch, 1 << log_n)).astype(np.float16)
    else:
        bits = 32 if op == "ntt32" else 64
        q = U32[0] if bits == 32 else U64[2]
        log_n = rng.randint(8, 17)
        batch = max(1, (1 << 18) >> log_n)
        t = cb.describe(cb.Operator.NTT, cb.DataType.UINT32 if bits == 32 else cb.DataType.UINT64, [1 << log_n],
                        compute=cb.ComputeType.UINT32 if bits == 32 else cb.ComputeType.UINT64, batch=batch,
                        modulus=q, word_bits=bits, ntt_ring=cb.NttRing.NEGACYCLIC)
        x = data.integers(0, q, (batch, 1 << log_n), dtype=np.uint64).astype(np.uint32 if bits == 32 else np.uint64)
    with tempfile.TemporaryDirectory() as tmp:
        cache = f"{tmp}/selection.tsv"
        with cb.Plan(lib, t, policy=cb.AlgorithmPolicy.MEASURE, stream=stream, cache_path=cache) as plan:
            chosen = plan.algorithm_name()
            measured = plan.selection_source() == cb.SelectionSource.RUNTIME_MEASURED
        with cb.Plan(lib, t, stream=stream, cache_path=cache) as plan:
            replayed = plan.algorithm_name() == chosen and plan.selection_source() == cb.SelectionSource.USER_CACHE
        got = run_plan(torch, lib, t, x, stream, algorithm=chosen)
    desc = f"measure {op} n=2^{log_n} batch={batch} -> {chosen} (measured {measured}, replayed {replayed})"
    if op == "fft":
        want = np.fft.fft(x.astype(np.complex128), axis=1)
        err = np.linalg.norm(got.astype(np.complex128) - want) / np.linalg.norm(want)
        ok = err <= 1e-5
    elif op == "fwht32":
        ok = np.array_equal(got.view(np.uint32), oracle.fwht_f32(x).view(np.uint32))
    elif op == "fwht16":
        ok = np.array_equal(got.view(np.uint16), oracle.fwht_f16_final(x, scale).view(np.uint16))
    else:
        ok = np.array_equal(got.astype(np.uint64), oracle.ntt_negacyclic(x.astype(np.uint64), q))
    return desc, ok and measured and replayed


RNS_SENTINEL = np.uint64(0xFEDCBA9876543210)


def rns_case(torch, lib, stream, rng, index):
    """An RNS plan: 1-3 domains (primes from 2^59 to above 2^62, roots an odd
    power of a primitive root), 1-5 polynomials in permuted slots of padded
    rows, random orders, ring, direction and placement; sentinel words around
    every slot must survive (out of place) or keep the input (in place)."""
    log_n = rng.randint(12, 17)
    n = 1 << log_n
    negacyclic = rng.random() < 0.6
    inverse, in_rev, out_rev, in_place = (rng.random() < 0.5 for _ in range(4))
    root_bits = log_n + int(negacyclic)
    primes = [q for q in U64 if two_adic(q - 1) >= root_bits]
    domains = []
    for _ in range(rng.randint(1, 3)):
        q = rng.choice(primes)
        domains.append((q, pow(oracle.find_primitive_root(root_bits, q), rng.choice([1, 3, 5, 7, 9, 11]), q)))
    count = rng.randint(1, 5)
    slots = count + rng.randint(0, 2)
    pad, base = rng.randint(0, 40), rng.randint(0, 20)
    ins, outs = rng.sample(range(slots), count), rng.sample(range(slots), count)
    polys = [{"domain": rng.randrange(len(domains)), "input_offset": i * (n + pad) + base,
              "output_offset": o * (n + pad) + base} for i, o in zip(ins, outs)]
    cfg = rns.request(log_n, domains, polynomials=polys, inverse=inverse,
                      ring="negacyclic" if negacyclic else "cyclic",
                      input_order="bit_reversed" if in_rev else "natural",
                      output_order="bit_reversed" if out_rev else "natural")
    words = slots * (n + pad) + base + 7
    data = np.full(words, RNS_SENTINEL)
    values = np.random.default_rng(index)
    for poly in polys:
        q = domains[poly["domain"]][0]
        data[poly["input_offset"]:poly["input_offset"] + n] = values.integers(0, q, n, dtype=np.uint64)
    want = data.copy() if in_place else np.full(words, RNS_SENTINEL)
    for poly in polys:
        q, root = domains[poly["domain"]]
        row = data[poly["input_offset"]:poly["input_offset"] + n]
        want[poly["output_offset"]:poly["output_offset"] + n] = oracle.rns(
            row[None], [q], [root], negacyclic=negacyclic, inverse=inverse, input_bit_reversed=in_rev,
            output_bit_reversed=out_rev)[0]
    x = to_device(torch, data)
    y = x if in_place else to_device(torch, np.full(words, RNS_SENTINEL))
    with rns.RnsPlan(lib, cfg) as plan:
        plan.prepare(stream, in_place=in_place, repetitions=1)
        plan.execute(x, y, stream)
        torch.cuda.synchronize()
        mapping = plan.info()["mapping"]["algorithm"]
    got = to_host(torch, y, np.uint64)
    desc = (f"rns n=2^{log_n} negacyclic={negacyclic} inverse={inverse} orders=({in_rev},{out_rev}) "
            f"in_place={in_place} domains={domains} polynomials={polys} [{mapping}]")
    return desc, np.array_equal(got, want)


KINDS = {"layouts": (layout_case, 120), "ntt": (ntt_case, 50), "fft": (fft_case, 40),
         "composites": (composite_case, 30), "embedding": (embedding_case, 30), "measure": (measure_case, 12),
         "rns": (rns_case, 25)}


@pytest.mark.parametrize("seed", [7, 11])
@pytest.mark.parametrize("kind", list(KINDS))
def test_random_cases(torch_gpu, lib, stream, kind, seed):
    case, count = KINDS[kind]
    rng = random.Random(f"{kind}-{seed}")
    failures = []
    for index in range(count):
        desc, ok = case(torch_gpu, lib, stream, rng, 1000 * seed + index)
        if not ok:
            failures.append(f"case {index}: {desc}")
    assert not failures, "\n".join(failures)
