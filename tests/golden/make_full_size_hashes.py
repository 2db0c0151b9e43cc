"""Writes full_size_hashes.json: SHA-256 of the inputs and of the expected
outputs of the bit-exact BASELINE configurations at full size, from the
seeded generators (cubutterfly_amd/workloads.py) and the CPU oracle
(oracle/). Each hash covers the C-contiguous little-endian bytes of one
array:

* C1: fp32 [4096][4096] integer input, its unnormalised forward FWHT;
* C2: u32 [64][65536] (q = 1073479681), the forward negacyclic NTT
  (natural order), whose inverse is the input again;
* C4: u64 [32][65536] over the 32 C4 primes, the forward negacyclic RNS NTT
  (natural -> bit-reversed), whose inverse is the input again;
* C5a / C5b: fp16 [16384][4096] / [524288][128] QuaRot-style input, the
  forward FWHT with output scale 1/sqrt(n) and final-storage rounding
  (bit-exact on the default lowering).

Run: python tests/golden/make_full_size_hashes.py (CPU only, a few seconds).
The tests recompute these from the generators and the oracle
(tests/test_golden_hashes.py) and compare the GPU outputs with them
(the full-size tests in tests/test_fwht_gpu.py, test_ntt_gpu.py,
test_rns_gpu.py)."""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PATH = os.path.join(HERE, "full_size_hashes.json")


def sha256(a):
    return hashlib.sha256(np.ascontiguousarray(a).astype(a.dtype.newbyteorder("<"), copy=False).tobytes()).hexdigest()


def c1():
    import oracle
    from cubutterfly_amd import workloads
    x = workloads.fwht_integer_input(12, 4096, seed=1)
    return x, oracle.fwht_f32(x, threads=oracle.default_threads())


def c2():
    import oracle
    from cubutterfly_amd import workloads
    q = workloads.C2_MODULUS
    x = workloads.ntt_input(16, 64, q, seed=1).astype(np.uint32)
    y = oracle.ntt_negacyclic(x.astype(np.uint64), q, threads=oracle.default_threads()).astype(np.uint32)
    return x, y


def c4():
    import oracle
    from cubutterfly_amd import workloads
    moduli = workloads.c4_moduli()
    roots = [oracle.find_primitive_root(17, q) for q in moduli]
    x = np.stack([workloads.ntt_input(16, 1, q, seed=1, channel=i)[0] for i, q in enumerate(moduli)])
    return x, oracle.rns(x, moduli, roots, output_bit_reversed=True, threads=oracle.default_threads())


def c5(rows, n):
    import oracle
    from cubutterfly_amd import workloads
    x = workloads.quarot_input(rows, n, seed=5)
    scale = float(np.float32(1.0 / np.sqrt(n)))
    return x, oracle.fwht_f16_final(x, scale, threads=oracle.default_threads())


CONFIGS = {"c1": c1, "c2": c2, "c4": c4, "c5a": lambda: c5(16384, 4096), "c5b": lambda: c5(524288, 128)}


def compute():
    out = {}
    for name, make in CONFIGS.items():
        x, y = make()
        out[name] = {"input_sha256": sha256(x), "output_sha256": sha256(y), "shape": list(x.shape),
                     "dtype": str(x.dtype)}
    return out


def load():
    with open(PATH) as f:
        return json.load(f)


if __name__ == "__main__":
    data = compute()
    with open(PATH, "w") as f:
        json.dump(data, f, indent=1, sort_keys=True)
        f.write("\n")
    print(json.dumps(data, indent=1, sort_keys=True))
