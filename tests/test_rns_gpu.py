"""RNS NTT parity on the GPU through the RNS C ABI, bit-exact against the oracle.

C4 at full size (32 limbs of 60-bit primes, n = 2^16, forward natural ->
bit-reversed, inverse bit-reversed -> natural), and the reference's own
regression layout (tests/test_rns_ntt.cu:113-162): two domains with explicit
roots primitive^3 / primitive^5, five polynomials in permuted slots of
n + 17 words at offset 11, sentinel words around every slot, both placements
and all four order combinations, plus graph replay and the prepared-cache
contract.
"""
import json

import numpy as np
import pytest

import cubutterfly_amd as cb
import oracle
from cubutterfly_amd import rns, workloads
from golden import make_full_size_hashes as golden
from gpu_util import to_device, to_host

pytestmark = pytest.mark.gpu

SENTINEL = np.uint64(0xFEDCBA9876543210)
PRIMES = [1152921504577486849, 576460756061519873]  # tests/test_rns_ntt.cu:19


@pytest.fixture(scope="module")
def rlib():
    return cb.Native()


def bitrev_perm(log_n):
    idx = np.arange(1 << log_n)
    rev = np.zeros_like(idx)
    for b in range(log_n):
        rev |= ((idx >> b) & 1) << (log_n - 1 - b)
    return rev


def run(torch, rlib, cfg, host_in, out_words, in_place, stream_obj):
    stream = stream_obj.cuda_stream
    x = to_device(torch, host_in)
    y = x if in_place else to_device(torch, np.full(out_words, SENTINEL))
    with rns.RnsPlan(rlib, cfg) as plan:
        plan.prepare(stream, in_place=in_place)
        plan.execute(x, y, stream)
        torch.cuda.synchronize()
        info = plan.info()
    return to_host(torch, y, np.uint64), info


def test_c4_full_size_round_trip(torch_gpu, rlib):
    print("case C4 rns 32 limbs x 2^16", flush=True)
    log_n, n = 16, 1 << 16
    moduli = workloads.c4_moduli()
    roots = [oracle.find_primitive_root(log_n + 1, q) for q in moduli]
    x = np.stack([workloads.ntt_input(log_n, 1, q, seed=1, channel=i)[0] for i, q in enumerate(moduli)])
    stream = torch_gpu.cuda.Stream()
    fwd_cfg = rns.request(log_n, list(zip(moduli, roots)))
    got, info = run(torch_gpu, rlib, fwd_cfg, x.ravel(), x.size, False, stream)
    expected = oracle.rns(x, moduli, roots, output_bit_reversed=True, threads=oracle.default_threads())
    np.testing.assert_array_equal(got.reshape(32, n), expected)
    assert golden.sha256(got.reshape(32, n)) == golden.load()["c4"]["output_sha256"]
    assert info["prepared"] and info["placement"] == "separate"
    inv_cfg = rns.request(log_n, list(zip(moduli, roots)), inverse=True)
    back, _ = run(torch_gpu, rlib, inv_cfg, got, x.size, True, stream)
    np.testing.assert_array_equal(back.reshape(32, n), x)


@pytest.mark.parametrize("inverse", [False, True])
def test_prepare_sweeps_the_candidates(torch_gpu, rlib, inverse):
    # Prepare times every mapping the gfx950 engine offers this request --
    # lazy and strict Shoup arithmetic (the 60-bit primes leave two spare
    # bits), 16- and 32-column tiles, the neighbouring splits 7 / 9 of the 16
    # index bits, Barrett products -- and executes the fastest; the result
    # stays bit-exact.
    print(f"case rns prepare sweep inverse={inverse}", flush=True)
    log_n, n, limbs = 16, 1 << 16, 4
    moduli = workloads.c4_moduli()[:limbs]
    roots = [oracle.find_primitive_root(log_n + 1, q) for q in moduli]
    x = np.stack([workloads.ntt_input(log_n, 1, q, seed=2, channel=i)[0] for i, q in enumerate(moduli)])
    cfg = rns.request(log_n, list(zip(moduli, roots)), inverse=inverse)
    stream = torch_gpu.cuda.Stream()
    xd = to_device(torch_gpu, x.ravel())
    yd = torch_gpu.empty_like(xd)
    with rns.RnsPlan(rlib, cfg) as plan:
        plan.prepare(stream.cuda_stream, repetitions=2)
        plan.execute(xd, yd, stream.cuda_stream)
        torch_gpu.cuda.synchronize()
        info = plan.info()
    mappings = [c["mapping"] for c in info["candidates"]]
    assert mappings == ["lazy-c16", "lazy-c32", "lazy-c16-h7", "lazy-c16-h9",
                        "strict-c16", "strict-c32", "strict-c16-h7", "strict-c16-h9",
                        "barrett-c16"]
    assert all(c["kernel_ms"] > 0 for c in info["candidates"])
    assert info["selected"] in mappings and info["source"] == "uncached_candidate_sweep"
    assert info["kernel_ms"] > 0 and info["mapping"]["algorithm"] in [c["algorithm"] for c in info["candidates"]]
    expected = oracle.rns(x, moduli, roots, inverse=inverse, input_bit_reversed=inverse,
                          output_bit_reversed=not inverse, threads=oracle.default_threads())
    np.testing.assert_array_equal(to_host(torch_gpu, yd, np.uint64).reshape(limbs, n), expected)


def wide_domain(log_n, negacyclic):
    """The reference's large-modulus fixture (tests/test_rns_ntt.cu:856-867):
    the first prime 2^62 + 1 + 8192 k, with the 7th power of its primitive
    root of the transform's order as the explicit root. 4q exceeds the word,
    so only fully reduced arithmetic applies."""
    q = (1 << 62) + 1
    while not oracle.is_prime(q):
        q += 8192
    root_bits = log_n + (1 if negacyclic else 0)
    root = pow(oracle.find_primitive_root(root_bits, q), 7, q)
    assert pow(root, 1 << root_bits, q) == 1 and pow(root, 1 << (root_bits - 1), q) == q - 1
    return q, root


def reference_layout(log_n, negacyclic, inverse, in_rev, out_rev, wide=False):
    """Config and input of tests/test_rns_ntt.cu:113-162 (`wide`: domain 0
    replaced by the large-modulus fixture, :856-868)."""
    n = 1 << log_n
    root_bits = log_n + (1 if negacyclic else 0)
    domains = []
    for d, q in enumerate(PRIMES):
        root = pow(oracle.find_primitive_root(root_bits, q), 3 if d == 0 else 5, q)
        domains.append((q, root))
    if wide:
        domains[0] = wide_domain(log_n, negacyclic)
    slots = [(1, 3, 5), (0, 0, 2), (0, 6, 0), (1, 2, 6), (0, 5, 3)]  # (domain, input slot, output slot)
    polys = [{"domain": d, "input_offset": i * (n + 17) + 11, "output_offset": o * (n + 17) + 11}
             for d, i, o in slots]
    cfg = rns.request(log_n, domains, polynomials=polys, inverse=inverse, ring="negacyclic" if negacyclic else "cyclic",
                     input_order="bit_reversed" if in_rev else "natural",
                     output_order="bit_reversed" if out_rev else "natural")
    words = 7 * (n + 17) + 29
    data = np.full(words, SENTINEL)
    rng = np.random.default_rng(log_n * 7 + int(inverse))
    for p in polys:
        q = domains[p["domain"]][0]
        row = rng.integers(0, q, n, dtype=np.uint64)
        row[:3] = [0, q - 1, q // 2]
        data[p["input_offset"]:p["input_offset"] + n] = row
    return cfg, domains, polys, data


def expected_layout(cfg, domains, polys, data, in_place):
    n = 1 << cfg["log_n"]
    out = data.copy() if in_place else np.full(data.size, SENTINEL)
    perm = bitrev_perm(cfg["log_n"])
    for p in polys:
        q, root = domains[p["domain"]]
        phys = data[p["input_offset"]:p["input_offset"] + n]
        y = oracle.rns(phys[None], [q], [root], negacyclic=cfg["ring"] == "negacyclic", inverse=cfg["inverse"],
                       input_bit_reversed=cfg["input_order"] == "bit_reversed",
                       output_bit_reversed=cfg["output_order"] == "bit_reversed")[0]
        out[p["output_offset"]:p["output_offset"] + n] = y
    return out


@pytest.mark.parametrize("log_n", [12, 14, 16])
@pytest.mark.parametrize("negacyclic", [True, False])
@pytest.mark.parametrize("inverse", [False, True])
@pytest.mark.parametrize("in_rev,out_rev", [(False, True), (True, False), (False, False), (True, True)])
@pytest.mark.parametrize("in_place", [False, True])
def test_reference_layout(torch_gpu, rlib, log_n, negacyclic, inverse, in_rev, out_rev, in_place):
    print(f"case rns layout log_n={log_n} neg={negacyclic} inv={inverse} in_rev={in_rev} "
          f"out_rev={out_rev} in_place={in_place}", flush=True)
    cfg, domains, polys, data = reference_layout(log_n, negacyclic, inverse, in_rev, out_rev)
    got, _ = run(torch_gpu, rlib, cfg, data, data.size, in_place, torch_gpu.cuda.Stream())
    np.testing.assert_array_equal(got, expected_layout(cfg, domains, polys, data, in_place))


# The reference's further cases (tests/test_rns_ntt.cu:853-868): log n 18
# (cyclic forward, natural -> bit-reversed), log n 20 (negacyclic inverse,
# bit-reversed -> natural) and the large-modulus domain at log n 12, through
# the RNS plan in both placements.
EDGE_CASES = [(18, False, False, False, True, False), (20, True, True, True, False, False),
              (12, True, True, True, False, True)]


@pytest.mark.parametrize("log_n,negacyclic,inverse,in_rev,out_rev,wide", EDGE_CASES)
@pytest.mark.parametrize("in_place", [False, True])
def test_reference_edge_cases(torch_gpu, rlib, log_n, negacyclic, inverse, in_rev, out_rev, wide, in_place):
    print(f"case rns edge log_n={log_n} neg={negacyclic} inv={inverse} in_rev={in_rev} out_rev={out_rev} "
          f"wide={wide} in_place={in_place}", flush=True)
    cfg, domains, polys, data = reference_layout(log_n, negacyclic, inverse, in_rev, out_rev, wide)
    got, info = run(torch_gpu, rlib, cfg, data, data.size, in_place, torch_gpu.cuda.Stream())
    np.testing.assert_array_equal(got, expected_layout(cfg, domains, polys, data, in_place))
    if wide:  # 4q > 2^64: no lazy candidate
        assert domains[0][0] > 1 << 62
        assert all(c["mapping"].startswith("strict") for c in info["candidates"])


def test_graph_replay_matches_eager(torch_gpu, rlib):
    # Captured executions replayed several times, with eager work between
    # replays, must equal the eager result every time.
    cfg, domains, polys, data = reference_layout(14, True, False, False, True)
    stream = torch_gpu.cuda.Stream()
    x = to_device(torch_gpu, data)
    y = to_device(torch_gpu, np.full(data.size, SENTINEL))
    blank = y.clone()
    expected = expected_layout(cfg, domains, polys, data, False)
    with rns.RnsPlan(rlib, cfg) as plan:
        plan.prepare(stream.cuda_stream)
        graph = torch_gpu.cuda.CUDAGraph()
        with torch_gpu.cuda.graph(graph, stream=stream):
            plan.execute(x, y, stream.cuda_stream)
        for _ in range(3):
            y.copy_(blank)  # eager work between replays
            torch_gpu.cuda.synchronize()
            with torch_gpu.cuda.stream(stream):
                graph.replay()
            torch_gpu.cuda.synchronize()
            np.testing.assert_array_equal(to_host(torch_gpu, y, np.uint64), expected)


def test_prepare_cache_contract(torch_gpu, rlib, tmp_path):
    cfg, _, _, _ = reference_layout(12, True, False, False, True)
    stream = torch_gpu.cuda.Stream().cuda_stream
    with rns.RnsPlan(rlib, cfg) as plan:
        with pytest.raises(cb.AbiError):  # REQUIRE without a record
            plan.prepare(stream, cache_dir=tmp_path, cache="require")
    with rns.RnsPlan(rlib, cfg) as plan:
        plan.prepare(stream, cache_dir=tmp_path, cache="prefer")
        first = plan.info()
        assert not first["cache_hit"] and first["kernel_ms"] > 0
        with pytest.raises(cb.AbiError):
            plan.prepare(stream)  # already prepared
    records = list(tmp_path.glob("rns-v1-*.json"))
    assert len(records) == 1 and records[0].stem == first["cache_key"]
    record = json.loads(records[0].read_text())
    assert record["selected"] == first["selected"] and record["source"] == "candidate_sweep"
    # One pass: arithmetic only (lazy, strict and Barrett products).
    assert [c["mapping"] for c in record["candidates"]] == ["lazy-c16", "strict-c16", "barrett-c16"]
    assert record["validation"] == "finalists_bit_exact_against_static_plan"
    with rns.RnsPlan(rlib, cfg) as plan:
        plan.prepare(stream, cache_dir=tmp_path, cache="require")
        hit = plan.info()
        assert hit["cache_hit"] and hit["kernel_ms"] == first["kernel_ms"]
        assert hit["selected"] == first["selected"] and hit["candidates"] == first["candidates"]
    # A record that selects no mapping of the request is refused.
    tampered = dict(record, selected="lazy-c64")
    records[0].write_text(json.dumps(tampered))
    with rns.RnsPlan(rlib, cfg) as plan:
        with pytest.raises(cb.AbiError) as info:
            plan.prepare(stream, cache_dir=tmp_path, cache="require")
        assert "selects no mapping" in str(info.value)
    # A record whose identity differs is refused, not replayed.
    record["identity"]["placement"] = "in_place"
    records[0].write_text(json.dumps(record))
    with rns.RnsPlan(rlib, cfg) as plan:
        with pytest.raises(cb.AbiError) as info:
            plan.prepare(stream, cache_dir=tmp_path, cache="prefer")
        assert "describes another request" in str(info.value)


def test_execute_contract(torch_gpu, rlib):
    cfg, _, _, data = reference_layout(12, True, False, False, True)
    x = to_device(torch_gpu, data)
    y = to_device(torch_gpu, data)
    with rns.RnsPlan(rlib, cfg) as plan:
        with pytest.raises(cb.AbiError) as info:
            plan.execute(x, y)  # not prepared
        assert info.value.status == 1
        plan.prepare()
        with pytest.raises(cb.AbiError) as info:
            plan.execute(x, x)  # aliasing differs from the prepared placement
        assert info.value.status == 1 and "placement" in info.value.detail


def test_prepare_refuses_stream_capture(torch_gpu, rlib):
    # Preparation times kernels on private buffers, which a capturing stream
    # cannot do (reference src/rns_ntt.cu:89-94): status 1, plan unprepared.
    cfg, _, _, data = reference_layout(12, True, False, False, True)
    s = torch_gpu.cuda.Stream()
    with rns.RnsPlan(rlib, cfg) as plan:
        graph = torch_gpu.cuda.CUDAGraph()
        with torch_gpu.cuda.graph(graph, stream=s):
            with pytest.raises(cb.AbiError) as info:
                plan.prepare(s.cuda_stream)
        assert info.value.status == 1 and "capture" in info.value.detail
        assert not plan.info()["prepared"]
        plan.prepare(s.cuda_stream)  # outside capture it prepares normally
        assert plan.info()["prepared"]


def test_prepare_that_cannot_allocate_leaves_the_plan_intact(torch_gpu, rlib):
    # One polynomial at word offset 2^36 (a 512 GiB input extent): Prepare's
    # sweep cannot allocate its buffers and fails with a runtime status; the
    # plan stays unprepared and intact -- Prepare may be called again, and
    # Execute still refuses it (the reference's allocation-failure contract,
    # tests/test_rns_mapping_failure.cu, src/rns_ntt.cu:761-785).
    log_n = 12
    q = PRIMES[0]
    root = oracle.find_primitive_root(log_n + 1, q)
    offset = 1 << 36
    cfg = rns.request(log_n, [(q, root)], polynomials=[{"domain": 0, "input_offset": offset,
                                                         "output_offset": 0}])
    stream = torch_gpu.cuda.Stream().cuda_stream
    with rns.RnsPlan(rlib, cfg) as plan:
        for _ in range(2):
            with pytest.raises(cb.AbiError) as e:
                plan.prepare(stream)
            assert e.value.status == 2
            assert plan.info()["prepared"] is False
        x = to_device(torch_gpu, np.zeros(1 << log_n, np.uint64))
        y = to_device(torch_gpu, np.zeros(1 << log_n, np.uint64))
        with pytest.raises(cb.AbiError) as e:
            plan.execute(x, y, stream)
        assert e.value.status == 1
