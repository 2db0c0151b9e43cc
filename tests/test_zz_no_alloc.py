"""cubutterflyExecuteNoAlloc against cubutterflyExecute on the GPU: the
no-allocation entry point takes the plan's workspace from the library's
static device array and must produce exactly what the bound-workspace entry
point produces -- two calls in a row, the second with a smaller input, so a
stale first-call image in the shared array would show. Plans whose workspace
exceeds the array are rejected before any work is queued."""
import ctypes as ct

import numpy as np
import pytest

import cubutterfly_amd as cb
from cubutterfly_amd import native, workloads
from gpu_util import to_device, to_host

pytestmark = pytest.mark.gpu

Q30 = workloads.C2_MODULUS
LIMIT = 32 << 20


def ntt(log_n, batch, inverse=False):
    return cb.describe(cb.Operator.NTT, cb.DataType.UINT32, [1 << log_n], batch, compute=cb.ComputeType.UINT32,
                       modulus=Q30, word_bits=32, inverse=inverse, ntt_ring=cb.NttRing.NEGACYCLIC)


def fft(log_n, batch):
    return cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [1 << log_n], batch, compute=cb.ComputeType.FP32)


def both(torch, lib, stream, desc, host, dtype):
    """(Execute output, ExecuteNoAlloc output) of one plan on `host`; the
    outputs are sized by the plan (the zero-extended embedding changes it)."""
    x = to_device(torch, host)
    with cb.Plan(lib, desc, stream=stream) as plan:
        ws_bytes = plan.workspace_size()
        assert 0 < ws_bytes <= LIMIT
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
        plan.set_workspace(ws, ws_bytes)
        assert plan.input_size() == x.numel() * x.element_size()
        out_elems = plan.output_size() // x.element_size()
        y_bound = torch.full((out_elems,), -1, dtype=x.dtype, device="cuda")
        plan.execute(x, y_bound)
        y_static = torch.full((out_elems,), -1, dtype=x.dtype, device="cuda")
        lib("ExecuteNoAlloc", plan.context, plan.handle, x.data_ptr(), y_static.data_ptr())
        torch.cuda.synchronize()
    return to_host(torch, y_bound, dtype), to_host(torch, y_static, dtype)


def fill_scratch(torch, lib, stream):
    """C2's forward through ExecuteNoAlloc: leaves 16 MiB of non-zero
    intermediate words in the shared array for the next plan to find."""
    host = workloads.ntt_input(16, 64, Q30, seed=11).astype(np.uint32)
    bound, static = both(torch, lib, stream, ntt(16, 64), host, np.uint32)
    np.testing.assert_array_equal(static, bound)


def test_header_states_the_limit():
    text = (native.INCLUDE / "cubutterfly" / "cubutterfly_mi355x.h").read_text()
    assert "#define CUBUTTERFLY_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)" in text


def test_ntt_two_calls_second_smaller(torch_gpu, lib, stream):
    # C2's forward (16 MiB workspace), then an 8-polynomial forward and an
    # inverse (2 MiB): bit-exact against the bound-workspace entry point.
    print("case no-alloc ntt 2^16 x 64 then x 8", flush=True)
    for batch, inverse in ((64, False), (8, False), (8, True)):
        host = workloads.ntt_input(16, batch, Q30, seed=batch).astype(np.uint32)
        bound, static = both(torch_gpu, lib, stream, ntt(16, batch, inverse), host, np.uint32)
        np.testing.assert_array_equal(static, bound)


def test_fft_two_calls_second_smaller(torch_gpu, lib, stream):
    print("case no-alloc fft 2^20 x 2 then 2^15 x 3", flush=True)
    for log_n, batch in ((20, 2), (15, 3)):
        host = workloads.complex_input(log_n, batch, seed=log_n).reshape(batch, 1 << log_n)
        bound, static = both(torch_gpu, lib, stream, fft(log_n, batch), host, np.complex64)
        np.testing.assert_array_equal(static.view(np.uint64), bound.view(np.uint64))


def test_plans_without_workspace_and_oversized_plans(torch_gpu, lib, stream):
    host = workloads.fwht_integer_input(12, 64, seed=2)
    x = to_device(torch_gpu, host)
    d = cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [4096], 64, compute=cb.ComputeType.FP32)
    with cb.Plan(lib, d, stream=stream) as plan:
        assert plan.workspace_size() == 0
        y1, y2 = torch_gpu.empty_like(x), torch_gpu.empty_like(x)
        plan.execute(x, y1)
        lib("ExecuteNoAlloc", plan.context, plan.handle, x.data_ptr(), y2.data_ptr())
        torch_gpu.cuda.synchronize()
        np.testing.assert_array_equal(to_host(torch_gpu, y2, np.float32), to_host(torch_gpu, y1, np.float32))
    # 2^22-point FFT x 2: 64 MiB of workspace, beyond the array. Rejected
    # before queuing anything (the pointers are never touched).
    with cb.Plan(lib, fft(22, 2), stream=stream) as plan:
        assert plan.workspace_size() > LIMIT
        status = lib.fn("ExecuteNoAlloc")(plan.context, plan.handle, ct.c_void_p(0x1000), ct.c_void_p(0x2000))
        assert status == cb.Status.INVALID_VALUE and "workspace" in lib.last_error()
    # The pointer and placement rules of cubutterflyExecute hold too.
    with cb.Plan(lib, ntt(16, 2), stream=stream) as plan:
        status = lib.fn("ExecuteNoAlloc")(plan.context, plan.handle, ct.c_void_p(0x1000), ct.c_void_p(0x1000))
        assert status == cb.Status.INVALID_VALUE


def test_composite_embedding_and_boundary_plans_after_a_larger_plan(torch_gpu, lib, stream):
    # Rank-2 FFT (row plan, transposes, workspace ping-pong buffers; column
    # passes and a natural-order row pass), the
    # zero-extended embedding (gather with zero fill, padded transform), a
    # strided boundary plan and long FWHTs (the FP32 promotion's buffer, a
    # bit-reversed boundary around a factored plan), each run right after a larger plan filled the
    # shared array with non-zero data: no plan may read a word it did not
    # write first, so both entry points agree bit for bit.
    rng = np.random.default_rng(5)
    cases = [
        ("rank-2 fft 64 x 2^13", cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [64, 1 << 13],
                                            compute=cb.ComputeType.FP32, batch=1), (64 << 13,), np.complex64),
        ("rank-2 fft 64 x 128, batch 2", cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [64, 128],
                                              compute=cb.ComputeType.FP32, batch=2), (2 * 64 * 128,), np.complex64),
        ("rank-2 fft 16 x 4096, batch 2 (one column pass)",
         cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [16, 4096], compute=cb.ComputeType.FP32, batch=2),
         (2 * 16 * 4096,), np.complex64),
        ("rank-2 fft 512 x 2048 (two column passes)",
         cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [512, 2048], compute=cb.ComputeType.FP32, batch=1),
         (512 * 2048,), np.complex64),
        ("zero-extended fft 3000 x 4", cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [3000],
                                                  compute=cb.ComputeType.FP32, batch=4,
                                                  length_mode=cb.LengthMode.ZERO_EXTENDED_EMBEDDING),
         (4 * 3000,), np.complex64),
        ("zero-extended fwht 1000 x 5", cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [1000],
                                                   compute=cb.ComputeType.FP32, batch=5,
                                                   length_mode=cb.LengthMode.ZERO_EXTENDED_EMBEDDING),
         (5 * 1000,), np.float32),
        ("strided fwht 2^12 x 8, rows interleaved", cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [4096],
                                                               compute=cb.ComputeType.FP32, batch=8,
                                                               input_strides=[8], input_batch_stride=1),
         (8 * 4096,), np.float32),
        ("fp16 fwht 2^16 x 3 (FP32 promotion)",
         cb.describe(cb.Operator.FWHT, cb.DataType.FP16, [1 << 16], compute=cb.ComputeType.FP32, batch=3,
                     output_scale=float(np.float32((1 << 16) ** -0.5)),
                     output_rounding=cb.OutputRounding.FINAL_STORAGE), (3 << 16,), np.float16),
        ("fwht 2^16 x 2, bit-reversed input (boundary, factored)",
         cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [1 << 16], compute=cb.ComputeType.FP32, batch=2,
                     input_orders=[cb.LogicalOrder.BIT_REVERSED], output_orders=[cb.LogicalOrder.NATURAL]),
         (2 << 16,), np.float32),
    ]
    for name, desc, shape, dtype in cases:
        print(f"case no-alloc {name} after C2's forward", flush=True)
        fill_scratch(torch_gpu, lib, stream)
        if dtype == np.complex64:
            host = (rng.standard_normal(shape) + 1j * rng.standard_normal(shape)).astype(np.complex64)
        else:
            host = rng.standard_normal(shape).astype(dtype)
        bound, static = both(torch_gpu, lib, stream, desc, host, dtype)
        width = {np.complex64: np.uint64, np.float32: np.uint32, np.float16: np.uint16}[dtype]
        np.testing.assert_array_equal(static.view(width), bound.view(width), err_msg=name)
