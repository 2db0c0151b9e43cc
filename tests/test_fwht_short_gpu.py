"""The 32-register FWHT lowering on short FP16 rows
(`fwht-fp16-fp32-resident-r32` for rows of 2^7 and 2^8 points: 4096-element
tiles of whole rows, one swizzled LDS exchange): bit-exact against the
stage-ordered oracle (src/butterfly_reference.cpp:349-369; FP16
final-storage contract tests/test_fwht_final_storage.py:28-40) on packed
and pitched rows, partial last tiles, in and out of place, forward and
normalised inverse, selected explicitly and listed for MEASURE."""
import numpy as np
import pytest

import cubutterfly_amd as cb
import oracle
from gpu_util import run_plan, to_device, to_host

pytestmark = pytest.mark.gpu


def transform(log_n, batch, inverse=False, in_place=False, fp16=True, **layout):
    kw = dict(output_rounding=cb.OutputRounding.FINAL_STORAGE,
              output_scale=(1 << log_n) ** -0.5) if fp16 else {}
    return cb.describe(cb.Operator.FWHT, cb.DataType.FP16 if fp16 else cb.DataType.FP32, [1 << log_n],
                       compute=cb.ComputeType.FP32, batch=batch, inverse=inverse, placement=int(in_place), **kw,
                       **layout)


def short_name(pitched=False):
    return "fwht-fp16-fp32-resident-r32" + ("-pitched" if pitched else "")


def inputs(log_n, batch, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((batch, 1 << log_n))
    x[:, rng.integers(0, 1 << log_n, 5)] *= 50.0  # outlier channels, as in the C5 workload
    return x.astype(np.float16)


def expected(x, log_n, inverse):
    return oracle.fwht_f16_final(x, (1 << log_n) ** -0.5, inverse=inverse, normalize=inverse)


def bits(a):
    return a.view(np.uint16)


@pytest.mark.parametrize("log_n", [7, 8])
@pytest.mark.parametrize("inverse", [False, True])
def test_packed(torch_gpu, lib, stream, log_n, inverse):
    # 4096 / n rows per tile; the batch leaves the last tile partial.
    batch = 37 * (4096 >> log_n) + 3
    x = inputs(log_n, batch, seed=log_n)
    t = transform(log_n, batch, inverse=inverse)
    with cb.Plan(lib, t, algorithm=short_name()) as plan:
        assert plan.algorithm_name() == short_name()
        assert plan.workspace_size() == 0
        m = plan.mapping()
        assert (m["tile_elements"], m["threads_per_block"], m["phases"]) == (4096, 128, 2)
        assert m["tiles"] == m["grid"] == -(-batch // (4096 >> log_n))
    got = run_plan(torch_gpu, lib, t, x, stream, algorithm=short_name())
    np.testing.assert_array_equal(bits(got), bits(expected(x, log_n, inverse)))


@pytest.mark.parametrize("log_n,batch", [(7, 1), (7, 31), (8, 16), (7, 524288)])
def test_small_and_full_batches(torch_gpu, lib, stream, log_n, batch):
    # One row (one partial tile), exactly one tile, up to C5b's 524288 x 128.
    x = inputs(log_n, batch, seed=batch)
    t = transform(log_n, batch)
    got = run_plan(torch_gpu, lib, t, x, stream, algorithm=short_name())
    np.testing.assert_array_equal(bits(got), bits(expected(x, log_n, False)))


def test_in_place(torch_gpu, lib, stream):
    log_n, batch = 7, 97
    x = inputs(log_n, batch, seed=5)
    t = transform(log_n, batch, in_place=True)
    got = run_plan(torch_gpu, lib, t, x, stream, in_place=True, algorithm=short_name())
    np.testing.assert_array_equal(bits(got), bits(expected(x, log_n, False)))


@pytest.mark.parametrize("log_n", [7, 8])
def test_pitched(torch_gpu, lib, stream, log_n):
    n, batch = 1 << log_n, 41
    in_pitch, out_pitch = n + 64, n + 8
    rows = inputs(log_n, batch, seed=log_n)
    x = np.zeros((batch - 1) * in_pitch + n, np.float16)
    for b in range(batch):
        x[b * in_pitch: b * in_pitch + n] = rows[b]
    sentinel = np.float16(-3.0)
    t = transform(log_n, batch, input_strides=[1], input_batch_stride=in_pitch, output_strides=[1],
                  output_batch_stride=out_pitch)
    xd = to_device(torch_gpu, x)
    yd = to_device(torch_gpu, np.full((batch - 1) * out_pitch + n, sentinel, np.float16))
    with cb.Plan(lib, t, algorithm=short_name(pitched=True), stream=stream) as plan:
        assert plan.algorithm_name() == short_name(pitched=True)
        plan.execute(xd, yd)
        torch_gpu.cuda.synchronize()
    got = to_host(torch_gpu, yd, np.float16)
    want = np.full_like(got, sentinel)
    result = expected(rows, log_n, False)
    for b in range(batch):
        want[b * out_pitch: b * out_pitch + n] = result[b]
    np.testing.assert_array_equal(bits(got), bits(want))


def test_measure_lists_the_short_row_lowering(torch_gpu, lib, stream, tmp_path):
    t = transform(7, 4096)
    with cb.Plan(lib, t, policy=cb.AlgorithmPolicy.MEASURE, stream=stream,
                 cache_path=tmp_path / "c.tsv") as plan:
        reason = plan.selection_reason()
    assert "fwht-fp16-fp32-resident-r32=" in reason, reason
    assert "fwht-fp16-fp32-resident-r32-persistent" not in reason, reason


@pytest.mark.parametrize("log_n,fp16,pitch", [(6, True, 0), (9, True, 0), (7, False, 0), (8, True, 1 << 26)])
def test_other_shapes_refuse_the_short_row_lowering(lib, log_n, fp16, pitch):
    # FP16 rows of 2^7 and 2^8 points, a tile's pitched span within 31-bit byte offsets.
    layout = dict(input_strides=[1], input_batch_stride=pitch, output_strides=[1],
                  output_batch_stride=pitch) if pitch else {}
    name = ("fwht-fp16-fp32-resident-r32" if fp16 else "fwht-fp32-resident-r32") + ("-pitched" if pitch else "")
    with pytest.raises(cb.AbiError) as e:
        cb.Plan(lib, transform(log_n, 8, fp16=fp16, **layout), algorithm=name)
    assert e.value.status == cb.Status.NOT_SUPPORTED
