"""FWHT on pitched rows: the FWHT kernels read and write rows a pitch apart
(unit element stride, natural order) without a boundary plan. Every case
checks the whole output buffer: the transformed rows bit-exact against the
oracle, every padding element untouched (reference layout semantics,
semantic_contract.cpp:55-123; stage order src/butterfly_reference.cpp:349-369)."""
import numpy as np
import pytest

import cubutterfly_amd as cb
import oracle
from gpu_util import to_device, to_host

pytestmark = pytest.mark.gpu


def run(torch, lib, stream, n, batch, in_pitch, out_pitch, fp16=False, inverse=False, in_place=False, seed=0):
    dtype = np.float16 if fp16 else np.float32
    rng = np.random.default_rng(seed)
    span_in = (batch - 1) * in_pitch + n
    span_out = (batch - 1) * out_pitch + n
    x = rng.standard_normal(span_in).astype(dtype)
    rows = np.stack([x[b * in_pitch: b * in_pitch + n] for b in range(batch)])
    kw = dict(output_rounding=cb.OutputRounding.FINAL_STORAGE,
              output_scale=n ** -0.5) if fp16 else {}
    t = cb.describe(cb.Operator.FWHT, cb.DataType.FP16 if fp16 else cb.DataType.FP32, [n], compute=cb.ComputeType.FP32, batch=batch, input_strides=[1], input_batch_stride=in_pitch, output_strides=[1], output_batch_stride=out_pitch, inverse=inverse, placement=int(in_place), **kw)
    sentinel = dtype(-3.0)
    xd = to_device(torch, x)
    yd = xd if in_place else to_device(torch, np.full(span_out, sentinel, dtype))
    with cb.Plan(lib, t, stream=stream) as plan:
        name = plan.algorithm_name()
        assert plan.workspace_size() == 0 or not name.endswith("-pitched")
        if plan.workspace_size():
            ws = torch.empty(plan.workspace_size(), dtype=torch.uint8, device="cuda")
            plan.set_workspace(ws, plan.workspace_size())
        plan.execute(xd, yd)
        torch.cuda.synchronize()
    got = to_host(torch, yd, dtype)
    expected = x.copy() if in_place else np.full(span_out, sentinel, dtype)
    if fp16:
        result = oracle.fwht_f16_final(rows, n ** -0.5, inverse=inverse, normalize=inverse)
    else:
        result = oracle.fwht_f32(rows, inverse=inverse, normalize=inverse)
    for b in range(batch):
        expected[b * out_pitch: b * out_pitch + n] = result[b]
    bits = np.uint16 if fp16 else np.uint32
    np.testing.assert_array_equal(got.view(bits), expected.view(bits))
    return name


@pytest.mark.parametrize("log_n", [4, 5, 7, 10, 12, 13])
@pytest.mark.parametrize("batch", [1 + 1, 37, 300])
def test_fp32(torch_gpu, lib, stream, log_n, batch):
    n = 1 << log_n
    name = run(torch_gpu, lib, stream, n, batch, n + 12, n + 4, seed=log_n)
    # 2^13-point FP32 rows default to the 32-register kernel.
    assert name == ("fwht-fp32-resident-r32-pitched" if log_n == 13 else "fwht-fp32-resident-r16-pitched")


@pytest.mark.parametrize("log_n", [4, 7, 11, 12, 13])
def test_fp16_final(torch_gpu, lib, stream, log_n):
    n = 1 << log_n
    name = run(torch_gpu, lib, stream, n, 45, n + 24, n + 8, fp16=True, seed=log_n)
    # FP16 rows of 2^11 to 2^13 points default to the 32-register kernel.
    wide = 11 <= log_n <= 13
    assert name == ("fwht-fp16-fp32-resident-r32-pitched" if wide else "fwht-fp16-fp32-resident-r16-pitched")


def test_inverse_normalised(torch_gpu, lib, stream):
    run(torch_gpu, lib, stream, 256, 70, 256 + 64, 256 + 4, inverse=True)


def test_in_place_same_pitch(torch_gpu, lib, stream):
    name = run(torch_gpu, lib, stream, 64, 200, 80, 80, in_place=True)
    assert name.endswith("-pitched")


def test_ineligible_layouts_use_the_boundary(torch_gpu, lib, stream):
    # Pitch not a 16-byte multiple, n below 16, in-place pitch change.
    assert run(torch_gpu, lib, stream, 64, 9, 66, 64 + 4).startswith("semantic-boundary[")
    assert run(torch_gpu, lib, stream, 8, 9, 12, 8).startswith("semantic-boundary[")
    assert run(torch_gpu, lib, stream, 64, 9, 80, 80).endswith("-pitched")


def test_many_tiles(torch_gpu, lib, stream):
    # 1250 row tiles of 32 rows: more workgroups than the GPU holds at once.
    run(torch_gpu, lib, stream, 128, 40000, 128 + 16, 128 + 16)
