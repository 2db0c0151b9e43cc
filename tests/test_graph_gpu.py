"""Plans captured into a HIP graph (torch.cuda.graph) and replayed several
times, with eager work between replays, match their eager results on every
replay: one-, two- and three-pass FFT, one- and two-pass NTT, FWHT (packed and
pitched; the lane-swap and MFMA lowerings too), a semantic-boundary plan and
rank-2 compositions (transposing rows, column passes). Execution
allocates nothing and records no memset, so capture is legal for every plan
(reference execution semantics, docs/c_api.md:29-33)."""
import numpy as np
import pytest

import cubutterfly_amd as cb
from gpu_util import to_device, to_host

pytestmark = pytest.mark.gpu

Q30 = 1073479681


def fft(n, batch, **kw):
    return cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [n] if isinstance(n, int) else n, compute=cb.ComputeType.FP32, batch=batch, **kw)


def ntt(n, batch, **kw):
    return cb.describe(cb.Operator.NTT, cb.DataType.UINT32, [n], compute=cb.ComputeType.UINT32, batch=batch, modulus=Q30, word_bits=32, ntt_ring=cb.NttRing.NEGACYCLIC, **kw)


def fwht(n, batch, **kw):
    return cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [n], compute=cb.ComputeType.FP32, batch=batch, **kw)


def fwht16(n, batch, **kw):
    return cb.describe(cb.Operator.FWHT, cb.DataType.FP16, [n], compute=cb.ComputeType.FP32, batch=batch, output_scale=n ** -0.5, output_rounding=cb.OutputRounding.FINAL_STORAGE, **kw)


CASES = {
    "fft-one-pass": (fft(1 << 12, 16), np.complex64, 1 << 16),
    "fft-two-pass": (fft(1 << 16, 2), np.complex64, 1 << 17),
    "fft-three-pass": (fft(1 << 23, 1), np.complex64, 1 << 23),
    "ntt-one-pass": (ntt(1 << 10, 32), np.uint32, 1 << 15),
    "ntt-two-pass": (ntt(1 << 16, 4, inverse=True), np.uint32, 1 << 18),
    "ntt-two-pass-forward": (ntt(1 << 16, 4), np.uint32, 1 << 18),
    "fwht-fp16-wide": (fwht16(4096, 64), np.float16, 1 << 18),
    "fwht": (fwht(4096, 32), np.float32, 1 << 17),
    "fwht-pitched": (fwht(1024, 8, input_strides=[1], input_batch_stride=1040, output_strides=[1],
                          output_batch_stride=1040), np.float32, 7 * 1040 + 1024),
    "boundary": (fft(256, 6, input_strides=[6], input_batch_stride=1), np.complex64, 6 * 256),
    "rank2": (fft([64, 128], 2), np.complex64, 2 * 64 * 128),
    "rank2-columns": (fft([512, 2048], 2), np.complex64, 2 * 512 * 2048),
    "fwht-fp16-lanes": (fwht16(128, 4096 + 7), np.float16, (4096 + 7) * 128),
    "fwht-fp32-lanes": (fwht(256, 300), np.float32, 300 * 256),
    "fwht-fp16-mfma": (fwht16(4096, 64, arithmetic_policy=cb.ArithmeticPolicy.ALLOW_FP16_MMA), np.float16, 1 << 18),
    "fwht-fp16-short": (fwht16(256, 16 * 40 + 3), np.float16, (16 * 40 + 3) * 256),
    "fwht-factored": (fwht(1 << 16, 3), np.float32, 3 << 16),
    "fwht-fp16-promoted": (fwht16(1 << 16, 3), np.float16, 3 << 16),
    "fwht-long-bit-reversed": (fwht(1 << 16, 2, input_orders=[cb.LogicalOrder.BIT_REVERSED],
                                    output_orders=[cb.LogicalOrder.NATURAL]), np.float32, 2 << 16),
}

# Explicit lowerings of some cases (the others use the default).
ALGORITHMS = {"fwht-fp16-lanes": "fwht-fp16-fp32-lanes-r64", "fwht-fp32-lanes": "fwht-fp32-lanes-r64",
              "fwht-fp16-mfma": "fwht-fp16-mfma16", "fwht-fp16-short": "fwht-fp16-fp32-resident-r32"}


def host_data(dtype, size, seed):
    rng = np.random.default_rng(seed)
    if np.dtype(dtype).kind == "c":
        return (rng.standard_normal(size) + 1j * rng.standard_normal(size)).astype(dtype)
    if np.dtype(dtype).kind == "u":
        return rng.integers(0, Q30, size).astype(dtype)
    return rng.standard_normal(size).astype(dtype)


@pytest.mark.parametrize("case", list(CASES))
def test_replays_match_eager(torch_gpu, lib, case):
    t, dtype, span = CASES[case]
    torch = torch_gpu
    stream = torch.cuda.Stream()
    kw = {"algorithm": ALGORITHMS[case]} if case in ALGORITHMS else {}
    with cb.Plan(lib, t, stream=stream.cuda_stream, **kw) as plan:
        if kw:
            assert plan.algorithm_name() == kw["algorithm"]
        out_span = plan.output_size() // np.dtype(dtype).itemsize
        assert plan.input_size() == span * np.dtype(dtype).itemsize
        ws_bytes = plan.workspace_size()
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
        if ws_bytes:
            plan.set_workspace(ws, ws_bytes)
        x = to_device(torch, host_data(dtype, span, 1))
        y = to_device(torch, np.zeros(out_span, dtype))
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            plan.execute(x, y)
        torch.cuda.synchronize()
        for replay in range(3):
            data = host_data(dtype, span, 10 + replay)
            x.copy_(to_device(torch, data))          # eager work between replays
            y.zero_()
            torch.cuda.synchronize()
            with torch.cuda.stream(stream):
                graph.replay()
            torch.cuda.synchronize()
            got = to_host(torch, y, dtype).copy()
            # The same plan, eagerly, on the same input.
            y.zero_()
            torch.cuda.synchronize()
            with torch.cuda.stream(stream):
                plan.execute(x, y)
            torch.cuda.synchronize()
            eager = to_host(torch, y, dtype)
            bits = {2: np.uint16, 4: np.uint32, 8: np.uint64}[np.dtype(dtype).itemsize] if np.dtype(dtype).kind != "c" else np.uint64
            np.testing.assert_array_equal(got.view(bits), eager.view(bits), err_msg=f"{case} replay {replay}")


@pytest.mark.parametrize("case", ["fft-two-pass", "rank2-columns", "fwht-fp16-promoted"])
def test_execute_steady_matches_execute(torch_gpu, lib, case):
    # cubutterflyExecuteSteady (reference src/c_api.cpp:5390-5411): the same
    # results as cubutterflyExecute, also after the handle's stream changes
    # between calls, and the same pointer checks.
    t, dtype, span = CASES[case]
    torch = torch_gpu
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    with cb.Plan(lib, t, stream=streams[0].cuda_stream) as plan:
        ws_bytes = plan.workspace_size()
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
        if ws_bytes:
            plan.set_workspace(ws, ws_bytes)
        out_span = plan.output_size() // np.dtype(dtype).itemsize
        x = to_device(torch, host_data(dtype, span, 4))
        y_exec = to_device(torch, np.zeros(out_span, dtype))
        plan.execute(x, y_exec)
        torch.cuda.synchronize()
        want = to_host(torch, y_exec, dtype)
        bits = np.uint64 if np.dtype(dtype).kind == "c" else {2: np.uint16, 4: np.uint32}[np.dtype(dtype).itemsize]
        for call, s in enumerate([streams[0], streams[0], streams[1], streams[0]]):
            lib("SetStream", plan.context, s.cuda_stream)
            y = to_device(torch, np.zeros(out_span, dtype))
            plan.execute_steady(x, y)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(to_host(torch, y, dtype).view(bits), want.view(bits), err_msg=f"call {call}")
        with pytest.raises(cb.AbiError) as e:
            plan.execute_steady(x, x)  # an out-of-place plan refuses aliased pointers
        assert e.value.status == cb.Status.INVALID_VALUE
