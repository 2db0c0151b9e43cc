"""The 32-register FWHT lowering (`fwht-fp16-fp32-resident-r32` for FP16
rows of 2^11..2^14 points, `fwht-fp32-resident-r32` for FP32 rows of the
same lengths, without the walking form; the only lowering of 2^14-point
rows, one row per 512-thread workgroup with a 67.6 KB LDS image): bit-exact against the stage-ordered
oracle (src/butterfly_reference.cpp:349-369; FP16 final-storage contract
tests/test_fwht_final_storage.py:28-40) on packed and pitched rows, in and
out of place, forward and normalised inverse, selected explicitly and by
MEASURE."""
import json

import numpy as np
import pytest

import cubutterfly_amd as cb
import oracle
from gpu_util import run_plan, to_device, to_host

pytestmark = pytest.mark.gpu


def transform(log_n, batch, fp16, inverse=False, in_place=False, **layout):
    kw = dict(output_rounding=cb.OutputRounding.FINAL_STORAGE,
              output_scale=(1 << log_n) ** -0.5) if fp16 else {}
    return cb.describe(cb.Operator.FWHT, cb.DataType.FP16 if fp16 else cb.DataType.FP32, [1 << log_n], compute=cb.ComputeType.FP32, batch=batch, inverse=inverse, placement=int(in_place), **kw, **layout)


def explicit(name):
    return {"algorithm": name}


def wide_name(fp16=True, pitched=False):
    return ("fwht-fp16-fp32-resident-r32" if fp16 else "fwht-fp32-resident-r32") + ("-pitched" if pitched else "")


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
@pytest.mark.parametrize("log_n", [11, 12, 13, 14, 15])
@pytest.mark.parametrize("inverse", [False, True])
def test_packed(torch_gpu, lib, stream, fp16, log_n, inverse):
    batch = 300 + log_n
    x = inputs(log_n, batch, fp16, seed=log_n + 10 * fp16)
    t = transform(log_n, batch, fp16, inverse=inverse)
    with cb.Plan(lib, t, **explicit(wide_name(fp16))) as plan:
        assert plan.algorithm_name() == wide_name(fp16)
        assert plan.workspace_size() == 0
    got = run_plan(torch_gpu, lib, t, x, stream, **explicit(wide_name(fp16)))
    np.testing.assert_array_equal(bits(got), bits(expected(x, log_n, fp16, inverse)))


@pytest.mark.parametrize("fp16", [True, False])
def test_in_place(torch_gpu, lib, stream, fp16):
    log_n, batch = 12, 97
    x = inputs(log_n, batch, fp16, seed=5)
    t = transform(log_n, batch, fp16, in_place=True)
    got = run_plan(torch_gpu, lib, t, x, stream, in_place=True, **explicit(wide_name(fp16)))
    np.testing.assert_array_equal(bits(got), bits(expected(x, log_n, fp16, False)))


@pytest.mark.parametrize("fp16", [True, False])
@pytest.mark.parametrize("log_n", [11, 13, 14, 15])
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
    with cb.Plan(lib, t, **explicit(wide_name(fp16, pitched=True)), stream=stream) as plan:
        assert plan.algorithm_name() == wide_name(fp16, pitched=True)
        plan.execute(xd, yd)
        torch_gpu.cuda.synchronize()
    got = to_host(torch_gpu, yd, dtype)
    want = np.full_like(got, sentinel)
    result = expected(rows, log_n, fp16, False)
    for b in range(batch):
        want[b * out_pitch: b * out_pitch + n] = result[b]
    np.testing.assert_array_equal(bits(got), bits(want))


def test_measure_lists_both_lowerings(torch_gpu, lib, stream, tmp_path):
    t = transform(12, 256, True)
    with cb.Plan(lib, t, policy=cb.AlgorithmPolicy.MEASURE, stream=stream,
                 cache_path=tmp_path / "c.tsv") as plan:
        reason = plan.selection_reason()
        name = plan.algorithm_name()
    assert "fwht-fp16-fp32-resident-r16=" in reason and "fwht-fp16-fp32-resident-r32=" in reason, reason
    assert name in ("fwht-fp16-fp32-resident-r16", "fwht-fp16-fp32-resident-r32",
                    "fwht-fp16-fp32-resident-r32-persistent")


@pytest.mark.parametrize("log_n,fp16", [(10, True), (16, True), (10, False), (16, False)])
def test_other_shapes_refuse_the_wide_lowering(lib, log_n, fp16):
    # Only rows of 2^11..2^15 points, and FP16 rows of 2^7, 2^8 (the
    # short-row kernel).
    with pytest.raises(cb.AbiError) as e:
        cb.Plan(lib, transform(log_n, 8, fp16), **explicit(wide_name(fp16)))
    assert e.value.status == cb.Status.NOT_SUPPORTED


def test_fp32_rows_refuse_the_walking_form(lib):
    # Two 32-word prefetch buffers would spill the registers.
    with pytest.raises(cb.AbiError) as e:
        cb.Plan(lib, transform(12, 8, False), **explicit(wide_name(False).replace("-r32", "-r32-persistent")))
    assert e.value.status == cb.Status.NOT_SUPPORTED


@pytest.mark.parametrize("fp16", [True])
@pytest.mark.parametrize("log_n,batch", [(11, 5003), (12, 2 * 4096 + 7), (13, 1500)])
def test_persistent_walk(torch_gpu, lib, stream, fp16, log_n, batch):
    # More rows than resident workgroups: each walks several rows with the
    # next row's loads in flight (odd counts end the walk on either buffer).
    name = wide_name(fp16).replace("-r32", "-r32-persistent")
    x = inputs(log_n, batch, fp16, seed=batch)
    t = transform(log_n, batch, fp16)
    with cb.Plan(lib, t, **explicit(name)) as plan:
        assert plan.algorithm_name() == name
        grid = plan.mapping()["grid"]
    assert grid < batch
    got = run_plan(torch_gpu, lib, t, x, stream, **explicit(name))
    np.testing.assert_array_equal(bits(got), bits(expected(x, log_n, fp16, False)))
