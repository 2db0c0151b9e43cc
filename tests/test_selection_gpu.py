"""MEASURE and the selection cache on the GPU (reference src/c_api.cpp:
722-764 cache records, 1420-1885 candidate searches): measured candidates,
cache replay under DEFAULT, last-record-wins, unterminated and stale records,
explicit selection of every candidate, and parity of each candidate with the
oracle."""
import re

import numpy as np
import pytest

import cubutterfly_amd as cb
import oracle
from gpu_util import run_plan

pytestmark = pytest.mark.gpu

Q30 = 1073479681  # 2^30 - 2^18 + 1: lazy reduction fits, so strict is a candidate too


def fft(log_n, batch, inverse=False):
    return cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [1 << log_n], compute=cb.ComputeType.FP32, batch=batch, inverse=inverse)


def ntt(log_n, batch, inverse=False):
    return cb.describe(cb.Operator.NTT, cb.DataType.UINT32, [1 << log_n], compute=cb.ComputeType.UINT32, batch=batch, modulus=Q30, word_bits=32, ntt_ring=cb.NttRing.NEGACYCLIC, inverse=inverse)


def measured(plan):
    """Candidate names listed in a MEASURE plan's selection reason."""
    reason = plan.selection_reason()
    assert "measured " in reason, reason
    return re.findall(r"([\w-]+)=[0-9.]+ ms", reason.split("measured ", 1)[1])


def records(path):
    text = path.read_text()
    return [line.split("\t") for line in text.splitlines()]


def fft_ok(torch, lib, t, stream, log_n, batch, inverse, **plan_args):
    rng = np.random.default_rng(log_n)
    x = (rng.standard_normal((batch, 1 << log_n)) + 1j * rng.standard_normal((batch, 1 << log_n))).astype(np.complex64)
    got = run_plan(torch, lib, t, x, stream, **plan_args).astype(np.complex128)
    ref = oracle.fft_c64(x, inverse=inverse, normalize=inverse, threads=oracle.default_threads()).astype(np.complex128)
    err = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert err <= 1e-5, err


def test_measure_records_and_default_replays(torch_gpu, lib, stream, tmp_path):
    cache = tmp_path / "selection.tsv"
    t = fft(16, 8)
    with cb.Plan(lib, t, policy=cb.AlgorithmPolicy.MEASURE, stream=stream,
                 cache_path=cache) as plan:
        assert plan.selection_source() == cb.SelectionSource.RUNTIME_MEASURED
        names = measured(plan)
        assert len(names) >= 2 and plan.algorithm_name() in names
        chosen = plan.algorithm_name()
    recs = records(cache)
    assert len(recs) == 1 and recs[0][1] == chosen
    key = recs[0][0]
    with cb.Plan(lib, t, cache_path=cache) as plan:
        assert plan.selection_source() == cb.SelectionSource.USER_CACHE
        assert plan.algorithm_name() == chosen
    # The last record for a key wins.
    other = next(n for n in names if n != chosen)
    with open(cache, "a") as f:
        f.write(f"{key}\t{other}\n")
    with cb.Plan(lib, t, cache_path=cache) as plan:
        assert plan.algorithm_name() == other
        assert plan.selection_source() == cb.SelectionSource.USER_CACHE
    fft_ok(torch_gpu, lib, t, stream, 16, 8, False, algorithm=other)
    # An unterminated final record is not replayed.
    with open(cache, "a") as f:
        f.write(f"{key}\t{chosen}")
    with cb.Plan(lib, t, cache_path=cache) as plan:
        assert plan.algorithm_name() == other
    # A record naming no lowering of the request falls back to the model.
    with open(cache, "a") as f:
        f.write(f"\n{key}\tno-such-lowering\n")
    with cb.Plan(lib, t, cache_path=cache) as plan:
        assert plan.selection_source() == cb.SelectionSource.STATIC_MODEL
        assert plan.algorithm_name() == "fft-c64-two-pass-r16"
        assert "ignored cache record" in plan.selection_reason()
    # Without a cache path DEFAULT is the static model.
    with cb.Plan(lib, t) as plan:
        assert plan.selection_source() == cb.SelectionSource.STATIC_MODEL


@pytest.mark.parametrize("log_n", [13, 14, 15, 16, 18, 20, 22, 23, 24])
@pytest.mark.parametrize("inverse", [False, True])
def test_every_fft_candidate_matches_the_oracle(torch_gpu, lib, stream, tmp_path, log_n, inverse):
    batch = 1 << max(0, 18 - log_n)
    t = fft(log_n, batch, inverse)
    with cb.Plan(lib, t, policy=cb.AlgorithmPolicy.MEASURE, stream=stream,
                 cache_path=tmp_path / "c.tsv") as plan:
        names = measured(plan)
    # The static model's choice comes first: radix-32 one-pass tiles up to
    # 2^14 (radix-16 tiles are the other candidate), three passes from 2^23.
    first = ("fft-c64-resident-r32" if log_n <= 14 else
             "fft-c64-three-pass-r16" if log_n >= 23 else "fft-c64-two-pass-r16")
    assert names[0].startswith(first)
    if log_n <= 14:
        assert names == ["fft-c64-resident-r32", "fft-c64-resident-r16"]
    for name in names:
        opts = {"algorithm": name}
        with cb.Plan(lib, t, **opts) as plan:
            assert plan.algorithm_name() == name
            assert plan.selection_source() == cb.SelectionSource.EXPLICIT
        fft_ok(torch_gpu, lib, t, stream, log_n, batch, inverse, **opts)


QDEF = 1152921504606584833  # include/cuntt/ntt.hpp:17; 2^18 | q - 1
Q2_21 = 1152921504577486849  # tests/test_rns_ntt.cu:19; 2^21 | q - 1 (negacyclic up to 2^20 points)


def modulus(bits, log_n):
    return Q30 if bits == 32 else QDEF if log_n <= 17 else Q2_21


def ntt_words(log_n, batch, bits, inverse):
    if bits == 32:
        return ntt(log_n, batch, inverse)
    return cb.describe(cb.Operator.NTT, cb.DataType.UINT64, [1 << log_n], compute=cb.ComputeType.UINT64, batch=batch,
                       modulus=modulus(bits, log_n), word_bits=64, ntt_ring=cb.NttRing.NEGACYCLIC, inverse=inverse)


# u64 adds 2^18 and 2^20, where its 32-column tiles are MEASURE candidates
# (the 30-bit u32 modulus has no 2^19-th roots of unity).
NTT_CANDIDATE_CASES = [(b, l) for b in (32, 64) for l in (10, 13, 14, 15, 16, 17)] + [(64, 18), (64, 20)]


@pytest.mark.parametrize("bits,log_n", NTT_CANDIDATE_CASES)
@pytest.mark.parametrize("inverse", [False, True])
def test_every_ntt_candidate_matches_the_oracle(torch_gpu, lib, stream, tmp_path, bits, log_n, inverse):
    print(f"case ntt candidates u{bits} log_n={log_n} inverse={inverse}", flush=True)
    batch = 4
    t = ntt_words(log_n, batch, bits, inverse)
    with cb.Plan(lib, t, policy=cb.AlgorithmPolicy.MEASURE, stream=stream,
                 cache_path=tmp_path / "c.tsv") as plan:
        names = measured(plan)
    # Lazy and strict; two-pass lengths add 32-column tiles (the static choice,
    # listed first, for u32 at 2^16) and at 2^15..2^17 the neighbouring
    # splits of the high and low bits; Barrett products last.
    base = f"ntt-u{bits}-negacyclic-" + ("two-pass-r16" if log_n > 12 else "resident-r16")
    expected = [base, base + "-strict"] + ([base + "-c32"] if log_n >= 13 else [])
    if log_n == 16 and bits == 32:
        expected = expected[-1:] + expected[:-1]
    l1 = min(8, log_n // 2)
    if 15 <= log_n <= 17:
        expected += [f"{base}-h{l1 - 1}", f"{base}-h{l1 + 1}"]
    expected.append(base + "-barrett")  # every modulus here is below 2^(word bits - 2)
    assert names == expected
    q = modulus(bits, log_n)
    rng = np.random.default_rng(log_n)
    words = np.uint32 if bits == 32 else np.uint64
    x = rng.integers(0, np.iinfo(words).max, (batch, 1 << log_n), dtype=np.uint64, endpoint=True).astype(words)
    expected = oracle.ntt_negacyclic(x.astype(np.uint64) % np.uint64(q), q, inverse=inverse).astype(words)
    for name in names:
        got = run_plan(torch_gpu, lib, t, x, stream, algorithm=name)
        np.testing.assert_array_equal(got, expected, err_msg=name)


def test_measure_composite_children(torch_gpu, lib, stream, tmp_path):
    cache = tmp_path / "c.tsv"
    t = cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [64, 1 << 15], compute=cb.ComputeType.FP32, batch=1)
    with cb.Plan(lib, t, policy=cb.AlgorithmPolicy.MEASURE, stream=stream,
                 cache_path=cache) as plan:
        assert plan.selection_source() == cb.SelectionSource.RUNTIME_MEASURED
        assert plan.algorithm_name().startswith("rank2-transpose[")
    assert len(records(cache)) == 2  # one record per axis plan
    with cb.Plan(lib, t, cache_path=cache) as plan:
        assert plan.selection_source() == cb.SelectionSource.USER_CACHE


def test_unknown_explicit_name_is_not_supported(torch_gpu, lib):
    opts = {"algorithm": "fft-c64-two-pass-r16-3x13"}
    with pytest.raises(cb.AbiError) as e:
        cb.Plan(lib, fft(16, 1), **opts)
    assert e.value.status == cb.Status.NOT_SUPPORTED


def test_plan_trace(torch_gpu, lib, stream, tmp_path, monkeypatch):
    # CUBUTTERFLY_PLAN_TRACE=<path>: JSON lines per search event (reference
    # src/plan_search_trace.hpp:17-60).
    import json
    trace = tmp_path / "trace.jsonl"
    monkeypatch.setenv("CUBUTTERFLY_PLAN_TRACE", str(trace))
    with cb.Plan(lib, fft(16, 2), policy=cb.AlgorithmPolicy.MEASURE, stream=stream,
                 cache_path=tmp_path / "c.tsv") as plan:
        chosen = plan.algorithm_name()
    rows = [json.loads(line) for line in trace.read_text().splitlines()]
    assert {r["schema"] for r in rows} == {"cubutterfly-plan-search-trace-v1"}
    phases = [r["phase"] for r in rows]
    assert phases[0] == "inventory" and phases[-1] == "selected"
    # Candidates are timed in interleaved rounds, each scored by its median block.
    assert rows[0]["timing_protocol"] == "interleaved-rounds"
    assert rows[0]["rounds"] >= 3 and rows[0]["calls_per_round"] >= 1
    results = [r for r in rows if r["phase"] == "result"]
    assert len(results) == rows[0]["candidate_count"] and all(r["kernel_ms"] > 0 for r in results)
    assert rows[-1]["algorithm"] == chosen


def test_measure_rotates_large_buffers(torch_gpu, lib, stream, tmp_path, monkeypatch):
    # Transforms of 16 MiB or more are timed over rotating buffer sets whose
    # inputs alone exceed twice the 256 MB Infinity Cache (C3b's 128 MiB
    # input: 5 sets); small ones on one set.
    import json
    for log_n, batch, sets in ((16, 2, 1), (14, 1024, 5)):
        trace = tmp_path / f"trace{log_n}.jsonl"
        monkeypatch.setenv("CUBUTTERFLY_PLAN_TRACE", str(trace))
        with cb.Plan(lib, fft(log_n, batch), policy=cb.AlgorithmPolicy.MEASURE,
                     stream=stream, cache_path=tmp_path / "c.tsv") as plan:
            assert plan.selection_source() == cb.SelectionSource.RUNTIME_MEASURED
        rows = [json.loads(line) for line in trace.read_text().splitlines()]
        assert rows[0]["phase"] == "inventory" and rows[0]["buffer_sets"] == sets


def _rows(flat, batch, pitch, n):
    return np.stack([flat[b * pitch: b * pitch + n] for b in range(batch)])


@pytest.mark.parametrize("case", ["fwht-c1p", "ntt-pitched"])
def test_measure_of_pitched_rows_sizes_scratch_by_the_span(torch_gpu, lib, stream, tmp_path, monkeypatch, case):
    # A pitched leaf addresses row b at b * pitch, (batch - 1) * pitch + n
    # elements per side: MEASURE's scratch buffers must span that much, and
    # the measured plan must compute what the EXPLICIT plan of the same
    # lowering computes.
    import json
    from gpu_util import to_device, to_host
    rng = np.random.default_rng(11)
    if case == "fwht-c1p":
        n, batch, pitch, dtype = 4096, 4096, 4096 + 64, np.float32
        t = cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [n], batch, compute=cb.ComputeType.FP32,
                        input_strides=[1], input_batch_stride=pitch, output_strides=[1], output_batch_stride=pitch)
        x = rng.integers(-8, 9, (batch - 1) * pitch + n).astype(np.float32)
    else:
        n, batch, pitch, dtype = 1 << 16, 4, (1 << 16) + 256, np.uint32
        t = cb.describe(cb.Operator.NTT, cb.DataType.UINT32, [n], batch, compute=cb.ComputeType.UINT32,
                        modulus=Q30, word_bits=32, ntt_ring=cb.NttRing.NEGACYCLIC, input_strides=[1],
                        input_batch_stride=pitch, output_strides=[1], output_batch_stride=pitch)
        x = rng.integers(0, Q30, (batch - 1) * pitch + n, dtype=np.uint64).astype(np.uint32)
    span = x.size * x.itemsize
    trace = tmp_path / "trace.jsonl"
    monkeypatch.setenv("CUBUTTERFLY_PLAN_TRACE", str(trace))
    results = {}
    for label, args in (("measure", {"policy": cb.AlgorithmPolicy.MEASURE, "cache_path": tmp_path / "c.tsv"}),
                        ("explicit", None)):
        if args is None:
            args = {"algorithm": results["measure"][0]}
        xd = to_device(torch_gpu, x)
        yd = torch_gpu.zeros_like(xd)
        with cb.Plan(lib, t, stream=stream, **args) as plan:
            assert plan.input_size() == plan.output_size() == span
            ws = plan.workspace_size()
            if ws:
                plan.set_workspace(torch_gpu.empty(ws, dtype=torch_gpu.uint8, device="cuda"), ws)
            plan.execute(xd, yd)
            torch_gpu.cuda.synchronize()
            results[label] = (plan.algorithm_name(), _rows(to_host(torch_gpu, yd, dtype), batch, pitch, n))
    inventory = json.loads(trace.read_text().splitlines()[0])
    assert inventory["phase"] == "inventory"
    assert inventory["input_bytes"] == span and inventory["output_bytes"] == span
    assert inventory["scratch_bytes"] >= inventory["buffer_sets"] * 2 * span
    assert results["measure"][0].endswith("-pitched")
    np.testing.assert_array_equal(results["measure"][1], results["explicit"][1])
    if case == "fwht-c1p":
        np.testing.assert_array_equal(results["explicit"][1], oracle.fwht_f32(_rows(x, batch, pitch, n), threads=16))
    else:
        expected = oracle.ntt_negacyclic(_rows(x, batch, pitch, n).astype(np.uint64), Q30)
        np.testing.assert_array_equal(results["explicit"][1].astype(np.uint64), expected)


def test_measure_refuses_stream_capture(torch_gpu, lib):
    # MEASURE times candidates on the device, which a capturing stream cannot
    # do: plan creation reports NOT_SUPPORTED and the capture stays valid.
    s = torch_gpu.cuda.Stream()
    graph = torch_gpu.cuda.CUDAGraph()
    with torch_gpu.cuda.graph(graph, stream=s):
        with pytest.raises(cb.AbiError) as e:
            cb.Plan(lib, fft(16, 1), policy=cb.AlgorithmPolicy.MEASURE, stream=s.cuda_stream)
        assert e.value.status == cb.Status.NOT_SUPPORTED and "capture" in e.value.detail


def test_measure_without_room_for_scratch_keeps_the_static_model(torch_gpu, lib, stream, tmp_path):
    # A request larger than the device (20 Mi rows of 4096 FP32 points, 320 GiB
    # each way): MEASURE cannot allocate its timing buffers, so the plan keeps
    # the static model's lowering and says why, instead of failing (the
    # reference's tuner falls back the same way when a candidate cannot run).
    t = cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [4096], 20 << 20, compute=cb.ComputeType.FP32)
    with cb.Plan(lib, t) as plan:
        static = plan.algorithm_name()
    with cb.Plan(lib, t, policy=cb.AlgorithmPolicy.MEASURE, stream=stream, cache_path=tmp_path / "c.tsv") as plan:
        assert plan.algorithm_name() == static
        assert plan.selection_source() != cb.SelectionSource.RUNTIME_MEASURED
        assert "MEASURE skipped: could not allocate" in plan.selection_reason()
    assert not (tmp_path / "c.tsv").exists() or (tmp_path / "c.tsv").read_text() == ""
    # The failed allocation is reported by the plan, not left in the HIP
    # runtime for the caller's next call to find.
    torch_gpu.zeros(16, device="cuda").add_(1)
    torch_gpu.cuda.synchronize()
