"""bench.py's host-side contract (no GPU needed): the buffer rotation that
keeps the Infinity Cache out of the measurement, the one-GPU refusal, the
BASELINE configurations it times, and their algorithmic bytes."""
import importlib.util
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


@pytest.mark.parametrize("input_mib,sets", [(64, 9), (128, 5), (16, 33), (1024, 3), (256, 3)])
def test_rotation_puts_inputs_beyond_the_infinity_cache(bench, input_mib, sets):
    # An input is read again only after more than twice the cache's bytes of
    # other inputs: outputs (nontemporal stores) may not evict it.
    got = bench._rotation(input_mib << 20)
    assert got == sets
    assert got >= 3 and (got - 1) * (input_mib << 20) >= 2 * bench.MALL_BYTES


def test_more_than_one_gpu_is_refused():
    done = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                          timeout=120)
    assert done.returncode == 2
    assert "one GPU" in done.stderr


def test_baseline_configurations_and_bytes(bench):
    # BASELINE.json's five configurations, the FFT and FP16 ones with two
    # shapes each: seven timed lines.
    configs = json.loads((ROOT / "BASELINE.json").read_text())["configs"]
    assert len(configs) == 5
    assert "n=2^24" in configs[2] and "n=2^14" in configs[2]
    assert "4096" in configs[4] and "128" in configs[4]
    assert list(bench.BASELINE_CONFIGS) == ["c1", "c2", "c3a", "c3b", "c4", "c5a", "c5b"]
    assert bench.DEFAULT_HEADLINE in bench.BASELINE_CONFIGS
    # Compulsory read + write of the caller's data per call: C1 2 x 64 MiB,
    # C2 / C4 2 x 16 MiB per direction, C3 / C5 2 x 128 MiB.
    expected = {"c1": 134217728, "c2": 67108864, "c3a": 268435456, "c3b": 268435456, "c4": 67108864,
                "c5a": 268435456, "c5b": 268435456}
    for name, nbytes in expected.items():
        assert bench.WORKLOADS[name]().bytes_per_call == nbytes, name


def test_batch_override_scales_the_workload(bench):
    # `--batch` rebuilds one configuration at another batch: the compulsory
    # bytes scale with it and the transform stays the same.
    assert sorted(bench.BATCHED) == ["c1", "c2", "c3b", "c5a", "c5b"]
    for name, standard in [("c1", 4096), ("c2", 64), ("c3b", 1024), ("c5a", 16384), ("c5b", 524288)]:
        base = bench.WORKLOADS[name]()
        assert bench.BATCHED[name](standard).bytes_per_call == base.bytes_per_call, name
        assert bench.BATCHED[name](2 * standard).bytes_per_call == 2 * base.bytes_per_call, name


@pytest.mark.parametrize("args", [["--batch", "128"], ["--workload", "c4", "--batch", "64"],
                                  ["--workload", "c2", "--batch", "0"]])
def test_batch_override_needs_a_batched_workload(args):
    done = subprocess.run([sys.executable, str(ROOT / "bench.py")] + args, capture_output=True, text=True,
                          timeout=120)
    assert done.returncode == 2
    assert "--batch needs" in done.stderr
