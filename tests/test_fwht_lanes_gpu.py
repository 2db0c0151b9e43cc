"""The 64-elements-per-lane FWHT lowering (`fwht-fp16-fp32-lanes-r64`,
`fwht-fp32-lanes-r64`: rows of 2^5..2^8 points, element bits 4 and 5
through gfx950's lane swaps, no LDS): bit-exact against the stage-ordered oracle
(src/butterfly_reference.cpp:349-369; FP16 final-storage contract
tests/test_fwht_final_storage.py:28-40) on packed and pitched rows, partial
last waves, in and out of place, forward and normalised inverse, selected
explicitly and listed for MEASURE."""
import numpy as np
import pytest

import cubutterfly_amd as cb
import oracle
from gpu_util import run_plan, to_device, to_host

pytestmark = pytest.mark.gpu


def transform(log_n, batch, fp16, inverse=False, in_place=False, **layout):
    kw = dict(output_rounding=cb.OutputRounding.FINAL_STORAGE,
              output_scale=(1 << log_n) ** -0.5) if fp16 else {}
    return cb.describe(cb.Operator.FWHT, cb.DataType.FP16 if fp16 else cb.DataType.FP32, [1 << log_n],
                       compute=cb.ComputeType.FP32, batch=batch, inverse=inverse, placement=int(in_place), **kw,
                       **layout)


def lanes_name(fp16, pitched=False):
    return ("fwht-fp16-fp32-lanes-r64" if fp16 else "fwht-fp32-lanes-r64") + ("-pitched" if pitched else "")


def inputs(log_n, batch, fp16, seed):
    rng = np.random.default_rng(seed)
    if fp16:
        x = rng.standard_normal((batch, 1 << log_n))
        x[:, rng.integers(0, 1 << log_n, 5)] *= 50.0  # outlier channels, as in the C5 workload
        return x.astype(np.float16)
    return (rng.integers(-8, 9, (batch, 1 << log_n)) + rng.standard_normal((batch, 1 << log_n))).astype(np.float32)


def expected(x, log_n, fp16, inverse):
    if fp16:
        return oracle.fwht_f16_final(x, (1 << log_n) ** -0.5, inverse=inverse, normalize=inverse)
    return oracle.fwht_f32(x, inverse=inverse, normalize=inverse)


def bits(a):
    return a.view(np.uint16 if a.dtype == np.float16 else np.uint32)


@pytest.mark.parametrize("fp16", [True, False])
@pytest.mark.parametrize("log_n", [5, 6, 7, 8])
@pytest.mark.parametrize("inverse", [False, True])
def test_packed(torch_gpu, lib, stream, fp16, log_n, inverse):
    # 4096 / n rows per wave, 4 waves per workgroup: the batch leaves the last
    # wave partial and the last workgroup with idle waves.
    batch = 3 * (4096 >> log_n) * 4 + 5
    x = inputs(log_n, batch, fp16, seed=log_n + 10 * fp16)
    t = transform(log_n, batch, fp16, inverse=inverse)
    name = lanes_name(fp16)
    with cb.Plan(lib, t, algorithm=name) as plan:
        assert plan.algorithm_name() == name
        assert plan.workspace_size() == 0
        assert plan.mapping()["lds_bytes"] == 0
    got = run_plan(torch_gpu, lib, t, x, stream, algorithm=name)
    np.testing.assert_array_equal(bits(got), bits(expected(x, log_n, fp16, inverse)))


@pytest.mark.parametrize("fp16", [True, False])
@pytest.mark.parametrize("log_n,batch", [(5, 1), (7, 3), (8, 17), (7, 524288)])
def test_small_and_full_batches(torch_gpu, lib, stream, fp16, log_n, batch):
    # One row (one partial wave) up to C5b's full 524288 x 128.
    x = inputs(log_n, batch, fp16, seed=batch)
    t = transform(log_n, batch, fp16)
    got = run_plan(torch_gpu, lib, t, x, stream, algorithm=lanes_name(fp16))
    np.testing.assert_array_equal(bits(got), bits(expected(x, log_n, fp16, False)))


@pytest.mark.parametrize("fp16", [True, False])
def test_in_place(torch_gpu, lib, stream, fp16):
    log_n, batch = 8, 97
    x = inputs(log_n, batch, fp16, seed=5)
    t = transform(log_n, batch, fp16, in_place=True)
    got = run_plan(torch_gpu, lib, t, x, stream, in_place=True, algorithm=lanes_name(fp16))
    np.testing.assert_array_equal(bits(got), bits(expected(x, log_n, fp16, False)))


@pytest.mark.parametrize("fp16", [True, False])
@pytest.mark.parametrize("log_n", [5, 6, 7, 8])
def test_pitched(torch_gpu, lib, stream, fp16, log_n):
    n, batch = 1 << log_n, 41
    in_pitch, out_pitch = n + 64, n + 8
    dtype = np.float16 if fp16 else np.float32
    rows = inputs(log_n, batch, fp16, seed=log_n)
    x = np.zeros((batch - 1) * in_pitch + n, dtype)
    for b in range(batch):
        x[b * in_pitch: b * in_pitch + n] = rows[b]
    sentinel = dtype(-3.0)
    t = transform(log_n, batch, fp16, input_strides=[1], input_batch_stride=in_pitch, output_strides=[1],
                  output_batch_stride=out_pitch)
    xd = to_device(torch_gpu, x)
    yd = to_device(torch_gpu, np.full((batch - 1) * out_pitch + n, sentinel, dtype))
    name = lanes_name(fp16, pitched=True)
    with cb.Plan(lib, t, algorithm=name, stream=stream) as plan:
        assert plan.algorithm_name() == name
        plan.execute(xd, yd)
        torch_gpu.cuda.synchronize()
    got = to_host(torch_gpu, yd, dtype)
    want = np.full_like(got, sentinel)
    result = expected(rows, log_n, fp16, False)
    for b in range(batch):
        want[b * out_pitch: b * out_pitch + n] = result[b]
    np.testing.assert_array_equal(bits(got), bits(want))


def test_measure_lists_the_lane_lowering(torch_gpu, lib, stream, tmp_path):
    t = transform(7, 4096, True)
    with cb.Plan(lib, t, policy=cb.AlgorithmPolicy.MEASURE, stream=stream,
                 cache_path=tmp_path / "c.tsv") as plan:
        reason = plan.selection_reason()
        name = plan.algorithm_name()
    assert "fwht-fp16-fp32-resident-r16=" in reason and "fwht-fp16-fp32-lanes-r64=" in reason, reason
    assert name in ("fwht-fp16-fp32-resident-r16", "fwht-fp16-fp32-resident-r32", "fwht-fp16-fp32-lanes-r64")


@pytest.mark.parametrize("log_n,pitch", [(4, 0), (9, 0), (12, 0), (8, 1 << 26)])
def test_other_shapes_refuse_the_lane_lowering(lib, log_n, pitch):
    # Rows of 2^5..2^8 points, a wave's pitched rows within 31-bit byte offsets.
    layout = dict(input_strides=[1], input_batch_stride=pitch, output_strides=[1],
                  output_batch_stride=pitch) if pitch else {}
    pitched = pitch != 0
    with pytest.raises(cb.AbiError) as e:
        cb.Plan(lib, transform(log_n, 8, True, **layout), algorithm=lanes_name(True, pitched))
    assert e.value.status == cb.Status.NOT_SUPPORTED

