"""The full-size golden hashes (tests/golden/full_size_hashes.json) against
the seeded generators and the CPU oracle: a change to either (an input rule,
a root convention, the stage order, the FP16 narrowing) moves a hash. The
GPU full-size tests compare the device outputs with the same hashes."""
import pytest

from golden import make_full_size_hashes as golden


@pytest.mark.parametrize("name", sorted(golden.CONFIGS))
def test_generators_and_oracle_reproduce_the_hashes(name):
    want = golden.load()[name]
    x, y = golden.CONFIGS[name]()
    assert list(x.shape) == want["shape"] and str(x.dtype) == want["dtype"]
    assert golden.sha256(x) == want["input_sha256"]
    assert golden.sha256(y) == want["output_sha256"]
