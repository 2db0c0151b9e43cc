"""Plans created from several host threads at once, on the GPU: FFT and NTT
plans upload their twiddle tables at creation, and plans made concurrently
(one handle each) must execute bit-identically to plans made one at a time."""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

import cubutterfly_amd as cb
from gpu_util import to_device, to_host

pytestmark = pytest.mark.gpu

CASES = [
    (cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [1 << 16], 4, compute=cb.ComputeType.FP32),
     np.complex64),
    (cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [512, 2048], 1, compute=cb.ComputeType.FP32),
     np.complex64),
    (cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [1 << 12], 64, compute=cb.ComputeType.FP32,
                 inverse=True), np.complex64),
    (cb.describe(cb.Operator.NTT, cb.DataType.UINT64, [1 << 16], 8, compute=cb.ComputeType.UINT64,
                 modulus=1152921504606584833, word_bits=64, ntt_ring=cb.NttRing.NEGACYCLIC), np.uint64),
    (cb.describe(cb.Operator.NTT, cb.DataType.UINT32, [1 << 14], 16, compute=cb.ComputeType.UINT32,
                 modulus=998244353, word_bits=32, inverse=True), np.uint32),
]


def host_input(desc, dtype, seed):
    count = int(np.prod(desc["shape"])) * desc["batch"]
    rng = np.random.default_rng(seed)
    if dtype == np.complex64:
        return (rng.standard_normal(count) + 1j * rng.standard_normal(count)).astype(dtype)
    return rng.integers(0, desc["modulus"], count, dtype=np.uint64).astype(dtype)


def execute(torch, plan, host, dtype):
    x = to_device(torch, host)
    y = torch.empty_like(x)
    ws_bytes = plan.workspace_size()
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    if ws_bytes:
        plan.set_workspace(ws, ws_bytes)
    plan.execute(x, y)
    torch.cuda.synchronize()
    return to_host(torch, y, dtype)


def test_concurrently_created_plans_match_serial_ones(torch_gpu, lib):
    stream = torch_gpu.cuda.current_stream().cuda_stream
    inputs = [host_input(d, t, i) for i, (d, t) in enumerate(CASES)]
    serial = []
    for (desc, dtype), host in zip(CASES, inputs):
        with cb.Plan(lib, desc, stream=stream) as plan:
            serial.append((plan.algorithm_name(), execute(torch_gpu, plan, host, dtype)))
    # Four plans of every case, created by eight threads at once.
    with ThreadPoolExecutor(max_workers=8) as pool:
        plans = list(pool.map(lambda d: cb.Plan(lib, d, stream=stream), [d for d, _ in CASES] * 4))
    try:
        for k, plan in enumerate(plans):
            i = k % len(CASES)
            dtype = CASES[i][1]
            name, want = serial[i]
            assert plan.algorithm_name() == name
            got = execute(torch_gpu, plan, inputs[i], dtype)
            bits = np.uint64 if dtype == np.complex64 else dtype
            np.testing.assert_array_equal(got.view(bits), want.view(bits), err_msg=f"plan {k} ({name})")
    finally:
        for plan in plans:
            plan.close()
