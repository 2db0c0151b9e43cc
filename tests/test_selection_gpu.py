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
    return cb.Transform(op=cb.Operator.FFT, storage=cb.DataType.COMPLEX_FP32, compute=cb.ComputeType.FP32,
                        extents=[1 << log_n], batch=batch, inverse=inverse)


def ntt(log_n, batch, inverse=False):
    return cb.Transform(op=cb.Operator.NTT, storage=cb.DataType.UINT32, compute=cb.ComputeType.UINT32,
                        extents=[1 << log_n], batch=batch, modulus=Q30, word_bits=32,
                        ring=cb.NttRing.NEGACYCLIC, inverse=inverse)


def measured(plan):
    """Candidate names listed in a MEASURE plan's selection reason."""
    reason = plan.selection_reason()
    assert "measured " in reason, reason
    return re.findall(r"([\w-]+)=[0-9.]+ ms", reason.split("measured ", 1)[1])


def records(path):
    text = path.read_text()
    return [line.split("\t") for line in text.splitlines()]


def fft_ok(torch, lib, t, stream, log_n, batch, inverse, options=None):
    rng = np.random.default_rng(log_n)
    x = (rng.standard_normal((batch, 1 << log_n)) + 1j * rng.standard_normal((batch, 1 << log_n))).astype(np.complex64)
    got = run_plan(torch, lib, t, x, stream, options=options).astype(np.complex128)
    ref = oracle.fft_c64(x, inverse=inverse, normalize=inverse, threads=oracle.default_threads()).astype(np.complex128)
    err = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert err <= 1e-5, err


def test_measure_records_and_default_replays(torch_gpu, lib, stream, tmp_path):
    cache = tmp_path / "selection.tsv"
    t = fft(16, 8)
    with cb.Plan(lib, t, options=cb.PlanOptions(policy=cb.AlgorithmPolicy.MEASURE), stream=stream,
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
    fft_ok(torch_gpu, lib, t, stream, 16, 8, False, options=cb.PlanOptions(mapping=other))
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


@pytest.mark.parametrize("log_n", [15, 16, 18, 20, 22, 23, 24])
@pytest.mark.parametrize("inverse", [False, True])
def test_every_fft_candidate_matches_the_oracle(torch_gpu, lib, stream, tmp_path, log_n, inverse):
    batch = 1 << max(0, 18 - log_n)
    t = fft(log_n, batch, inverse)
    with cb.Plan(lib, t, options=cb.PlanOptions(policy=cb.AlgorithmPolicy.MEASURE), stream=stream,
                 cache_path=tmp_path / "c.tsv") as plan:
        names = measured(plan)
    # The static model's choice comes first: three passes from 2^23.
    assert names[0].startswith("fft-c64-three-pass-r16" if log_n >= 23 else "fft-c64-two-pass-r16")
    for name in names:
        opts = cb.PlanOptions(policy=cb.AlgorithmPolicy.EXPLICIT, mapping=name)
        with cb.Plan(lib, t, options=opts) as plan:
            assert plan.algorithm_name() == name
            assert plan.selection_source() == cb.SelectionSource.EXPLICIT
        fft_ok(torch_gpu, lib, t, stream, log_n, batch, inverse, options=opts)


@pytest.mark.parametrize("log_n", [10, 13, 14, 16, 17])
@pytest.mark.parametrize("inverse", [False, True])
def test_ntt_strict_candidate(torch_gpu, lib, stream, tmp_path, log_n, inverse):
    batch = 4
    t = ntt(log_n, batch, inverse)
    with cb.Plan(lib, t, options=cb.PlanOptions(policy=cb.AlgorithmPolicy.MEASURE), stream=stream,
                 cache_path=tmp_path / "c.tsv") as plan:
        names = measured(plan)
    # Lazy and strict; u32 two-pass lengths add 32-column tiles, the static
    # choice (listed first) at 2^16.
    base = "ntt-u32-negacyclic-" + ("two-pass-r16" if log_n > 12 else "resident-r16")
    expected = [base, base + "-strict"] + ([base + "-c32"] if log_n >= 13 else [])
    if log_n == 16:
        expected = expected[-1:] + expected[:-1]
    assert names == expected
    rng = np.random.default_rng(log_n)
    x = rng.integers(0, 1 << 32, (batch, 1 << log_n), dtype=np.uint64).astype(np.uint32)
    expected = oracle.ntt_negacyclic(x.astype(np.uint64) % Q30, Q30, inverse=inverse).astype(np.uint32)
    for name in names:
        opts = cb.PlanOptions(policy=cb.AlgorithmPolicy.EXPLICIT, mapping=name)
        got = run_plan(torch_gpu, lib, t, x, stream, options=opts)
        np.testing.assert_array_equal(got, expected, err_msg=name)


def test_measure_composite_children(torch_gpu, lib, stream, tmp_path):
    cache = tmp_path / "c.tsv"
    t = cb.Transform(op=cb.Operator.FFT, storage=cb.DataType.COMPLEX_FP32, compute=cb.ComputeType.FP32,
                     extents=[64, 1 << 15], batch=1)
    with cb.Plan(lib, t, options=cb.PlanOptions(policy=cb.AlgorithmPolicy.MEASURE), stream=stream,
                 cache_path=cache) as plan:
        assert plan.selection_source() == cb.SelectionSource.RUNTIME_MEASURED
        assert plan.algorithm_name().startswith("rank2-transpose[")
    assert len(records(cache)) == 2  # one record per axis plan
    with cb.Plan(lib, t, cache_path=cache) as plan:
        assert plan.selection_source() == cb.SelectionSource.USER_CACHE


def test_unknown_explicit_name_is_not_supported(torch_gpu, lib):
    opts = cb.PlanOptions(policy=cb.AlgorithmPolicy.EXPLICIT, mapping="fft-c64-two-pass-r16-3x13")
    with pytest.raises(cb.Error) as e:
        cb.Plan(lib, fft(16, 1), options=opts)
    assert e.value.status == cb.Status.NOT_SUPPORTED


def test_plan_trace(torch_gpu, lib, stream, tmp_path, monkeypatch):
    # CUBUTTERFLY_PLAN_TRACE=<path>: JSON lines per search event (reference
    # src/plan_search_trace.hpp:17-60).
    import json
    trace = tmp_path / "trace.jsonl"
    monkeypatch.setenv("CUBUTTERFLY_PLAN_TRACE", str(trace))
    with cb.Plan(lib, fft(16, 2), options=cb.PlanOptions(policy=cb.AlgorithmPolicy.MEASURE), stream=stream,
                 cache_path=tmp_path / "c.tsv") as plan:
        chosen = plan.algorithm_name()
    rows = [json.loads(line) for line in trace.read_text().splitlines()]
    assert {r["schema"] for r in rows} == {"cubutterfly-plan-search-trace-v1"}
    phases = [r["phase"] for r in rows]
    assert phases[0] == "inventory" and phases[-1] == "selected"
    results = [r for r in rows if r["phase"] == "result"]
    assert len(results) == rows[0]["candidate_count"] and all(r["kernel_ms"] > 0 for r in results)
    assert rows[-1]["algorithm"] == chosen


def test_measure_rotates_large_buffers(torch_gpu, lib, stream, tmp_path, monkeypatch):
    # Transforms of 16 MiB or more are timed over rotating buffer sets whose
    # footprint exceeds twice the 256 MB Infinity Cache (C3b's 128 MiB: 3
    # sets); small ones on one set.
    import json
    for log_n, batch, sets in ((16, 2, 1), (14, 1024, 3)):
        trace = tmp_path / f"trace{log_n}.jsonl"
        monkeypatch.setenv("CUBUTTERFLY_PLAN_TRACE", str(trace))
        with cb.Plan(lib, fft(log_n, batch), options=cb.PlanOptions(policy=cb.AlgorithmPolicy.MEASURE),
                     stream=stream, cache_path=tmp_path / "c.tsv") as plan:
            assert plan.selection_source() == cb.SelectionSource.RUNTIME_MEASURED
        rows = [json.loads(line) for line in trace.read_text().splitlines()]
        assert rows[0]["phase"] == "inventory" and rows[0]["buffer_sets"] == sets
