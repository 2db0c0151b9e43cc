"""Rank-2 and higher plans on the CPU host: lowering choice, schedule,
workspace and the executable subset (reference rank-two lowering,
src/c_api.cpp:4578-4650; FWHT plans allocate nothing at creation, so their
shapes are checkable without a device)."""
import json

import pytest

import cubutterfly_amd as cb


def fwht(extents, **kw):
    return cb.describe(cb.Operator.FWHT, cb.DataType.FP32, list(extents), compute=cb.ComputeType.FP32, **kw)


def schedule(plan):
    return plan.mapping()["schedule"]


def test_rank2_fwht_is_one_kronecker_plan(lib):
    with cb.Plan(lib, fwht([8, 16], batch=3)) as plan:
        name = plan.algorithm_name()
        assert name.startswith("rank2-kronecker[fwht-fp32")
        assert name.endswith("+direct-input+direct-output")
        assert plan.workspace_size() == 0
        assert plan.physical_extents() == [8, 16]
        assert plan.input_size() == plan.output_size() == 3 * 128 * 4
        steps = schedule(plan)
        assert len(steps) == 1 and steps[0]["step"] == "axis"


def test_normalised_inverse_fwht_composes_per_axis(lib):
    with cb.Plan(lib, fwht([8, 16], batch=2, inverse=True)) as plan:
        assert plan.algorithm_name().startswith("rank2-transpose[fwht-fp32")
        steps = schedule(plan)
        # Axis 1 (contiguous) first, transpose, axis 0, transpose back.
        assert [s["step"] for s in steps] == ["axis", "transpose", "axis", "transpose"]
        assert [s["axis"] for s in steps if s["step"] == "axis"] == [1, 0]
        assert (steps[1]["blocks"], steps[1]["rows"], steps[1]["cols"]) == (2, 8, 16)
        assert (steps[3]["blocks"], steps[3]["rows"], steps[3]["cols"]) == (2, 16, 8)
        assert plan.workspace_size() == 2 * 2 * 128 * 4


def test_rank3_schedule_restores_axis_order(lib):
    with cb.Plan(lib, fwht([4, 8, 2], inverse=True)) as plan:
        assert plan.algorithm_name().startswith("rankN-composite[")
        steps = schedule(plan)
        assert [s["axis"] for s in steps if s["step"] == "axis"] == [2, 1, 0]
        # Simulate the axis order through the transposes: each moves the
        # block's row axis after its column axes.
        extents = {0: 4, 1: 8, 2: 2}
        order = [0, 1, 2]
        for s in steps:
            if s["step"] == "axis":
                assert order[-1] == s["axis"]
                continue
            rows = s["rows"]
            # the moved axis is the first one whose extent matches the rows and
            # whose trailing product matches the columns
            for pos, axis in enumerate(order):
                tail = 1
                for other in order[pos + 1:]:
                    tail *= extents[other]
                if extents[axis] == rows and tail == s["cols"] and tail > 1:
                    order = order[:pos] + order[pos + 1:] + [axis]
                    break
            else:
                pytest.fail(f"transpose {s} moves no axis of {order}")
        assert order == [0, 1, 2]


def test_large_rank2_fwht_uses_column_passes(lib):
    # 2^16 points exceed one resident FWHT plan: the rows of axis 1, then axis
    # 0 as one in-place column pass (no transposes, no workspace).
    with cb.Plan(lib, fwht([128, 512])) as plan:
        assert plan.algorithm_name() == (
            "rank2-fwht-columns[fwht-fp32-resident-r16,fwht-fp32-columns-l7]+direct-input+direct-output")
        assert plan.workspace_size() == 0
        steps = schedule(plan)
        assert [s["step"] for s in steps] == ["axis", "columns"]
        assert (steps[1]["axis"], steps[1]["rows"], steps[1]["cols"], steps[1]["blocks"]) == (0, 128, 512, 1)
        assert steps[1]["scale"] == 1.0


def test_rank2_fwht_of_2_15_points_flattens(lib):
    # One 2^15-point row plan (the 32-register kernel) covers H(128) (x) H(256).
    with cb.Plan(lib, fwht([128, 256])) as plan:
        assert plan.algorithm_name() == "rank2-kronecker[fwht-fp32-resident-r32]+direct-input+direct-output"


def test_normalised_rank2_fwht_scales_each_axis(lib):
    # Axis 0 of 2^12 points splits into two column passes of 2^6 rows, lowest
    # bits first; per-axis normalisation divides by 2^12 after the second.
    with cb.Plan(lib, fwht([4096, 64], batch=2, inverse=True)) as plan:
        steps = schedule(plan)
        assert [s["step"] for s in steps] == ["axis", "columns", "columns"]
        assert [(s["rows"], s["cols"], s["blocks"]) for s in steps[1:]] == [(64, 64, 2 * 64), (64, 64 * 64, 2)]
        assert [s["scale"] for s in steps[1:]] == [1.0, 2.0 ** -12]


def test_short_inner_axis_keeps_transposes(lib):
    # Rows under 64 elements would make column passes read short segments.
    with cb.Plan(lib, fwht([1024, 32], inverse=True)) as plan:
        assert plan.algorithm_name().startswith("rank2-transpose[")


def test_strided_rank2_gathers_and_scatters(lib):
    t = fwht([8, 8], batch=2, input_strides=[16, 1], input_batch_stride=128)
    with cb.Plan(lib, t) as plan:
        name = plan.algorithm_name()
        assert "+direct-input" not in name and name.endswith("+direct-output")
        assert plan.input_size() == (128 + 7 * 16 + 8) * 4
        assert plan.workspace_size() == 2 * 8 * 8 * 4  # gathered buffer only
        assert plan.mapping()["direct_input_boundary"] is False


def test_rank2_orders_need_the_boundary(lib):
    t = fwht([8, 8], output_orders=[cb.LogicalOrder.NATURAL, cb.LogicalOrder.BIT_REVERSED])
    with cb.Plan(lib, t) as plan:
        assert plan.algorithm_name().endswith("+direct-input")


def test_rank2_not_supported_cases(lib):
    fp16 = cb.describe(cb.Operator.FWHT, cb.DataType.FP16, [8, 8], compute=cb.ComputeType.FP32, output_rounding=cb.OutputRounding.FINAL_STORAGE)
    negacyclic = cb.describe(cb.Operator.NTT, cb.DataType.UINT32, [8, 8], compute=cb.ComputeType.UINT32, modulus=998244353, word_bits=32, ntt_ring=cb.NttRing.NEGACYCLIC)
    odd = fwht([8, 1])
    for t in (fp16, negacyclic, odd):
        with pytest.raises(cb.AbiError) as e:
            cb.Plan(lib, t)
        assert e.value.status == cb.Status.NOT_SUPPORTED, lib.last_error()


# ---- the per-axis oracle composition the GPU tests compare against --------

import numpy as np  # noqa: E402

import oracle  # noqa: E402


def along(x, axis, f):
    """Apply the row-wise oracle `f` along `axis` of x [batch, *extents]."""
    moved = np.moveaxis(x, axis, -1)
    shape = moved.shape
    out = f(np.ascontiguousarray(moved).reshape(-1, shape[-1])).reshape(shape)
    return np.ascontiguousarray(np.moveaxis(out, -1, axis))


def compose(x, f):
    """Innermost axis first, as the reference's axis schedule."""
    for axis in range(x.ndim - 1, 0, -1):
        x = along(x, axis, f)
    return x


def test_ntt_composition_matches_brute_force_2d_dft():
    # X[k0, k1] = sum x[j0, j1] w0^(j0 k0) w1^(j1 k1) mod q, roots by the
    # reference rule for each axis length.
    q, n0, n1 = 998244353, 4, 8
    rng = np.random.default_rng(1)
    x = rng.integers(0, q, (2, n0, n1)).astype(np.uint64)
    w0, w1 = oracle.find_primitive_root(2, q), oracle.find_primitive_root(3, q)
    brute = np.zeros_like(x)
    for b in range(2):
        for k0 in range(n0):
            for k1 in range(n1):
                acc = 0
                for j0 in range(n0):
                    for j1 in range(n1):
                        acc += int(x[b, j0, j1]) * pow(w0, j0 * k0, q) * pow(w1, j1 * k1, q)
                brute[b, k0, k1] = acc % q
    got = compose(x, lambda rows: oracle.ntt_cyclic(rows, q))
    np.testing.assert_array_equal(got, brute)
    back = compose(got, lambda rows: oracle.ntt_cyclic(rows, q, inverse=True))
    np.testing.assert_array_equal(back, x)


def test_fft_composition_matches_numpy_fftn():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((2, 8, 16, 4)) + 1j * rng.standard_normal((2, 8, 16, 4))).astype(np.complex64)
    got = compose(x, oracle.fft_c64).astype(np.complex128)
    ref = np.fft.fftn(x.astype(np.complex128), axes=(1, 2, 3))
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-6


def test_fwht_composition_is_the_flat_transform():
    # Kronecker identity H(n0 n1) = H(n0) (x) H(n1), with the same rounding:
    # the innermost-first composition equals the flat rank-1 oracle bit for bit.
    rng = np.random.default_rng(3)
    x = rng.standard_normal((3, 16, 32)).astype(np.float32)
    got = compose(x, oracle.fwht_f32)
    flat = oracle.fwht_f32(x.reshape(3, -1)).reshape(x.shape)
    np.testing.assert_array_equal(got.view(np.uint32), flat.view(np.uint32))
    # An outermost-first order rounds differently for generic data, so the
    # axis order is what fixes the bits.
    other = along(along(x, 1, oracle.fwht_f32), 2, oracle.fwht_f32)
    assert not np.array_equal(other.view(np.uint32), flat.view(np.uint32))


@pytest.mark.parametrize("log_n,extents", [
    (16, [16, 4096]), (19, [128, 4096]), (20, [128, 8192]), (21, [128, 16384]), (22, [128, 32768]),
    (23, [64, 32, 4096]), (26, [128, 128, 4096]), (27, [128, 128, 8192]), (28, [128, 128, 16384]),
    (29, [128, 128, 32768]), (30, [64, 64, 64, 4096]),
])
def test_long_fwht_is_factored(lib, log_n, extents):
    # FWHT beyond 2^15 points: a resident row of 2^12 points (up to 2^15
    # where that saves a pass), then axes of at most 2^7 points, lowest bits
    # innermost, each one in-place column pass.
    n = 1 << log_n
    t = cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [n], compute=cb.ComputeType.FP32, batch=2)
    with cb.Plan(lib, t) as plan:
        # Rows of 2^13 points and more: the 32-register kernel.
        row = "resident-r32" if extents[-1] >= 8192 else "resident-r16"
        assert plan.algorithm_name().startswith(f"fwht-factored[fwht-fp32-{row},fwht-fp32-columns-l")
        assert plan.physical_extents() == [n]
        assert plan.input_size() == plan.output_size() == 2 * n * 4
        assert plan.workspace_size() == 0
        m = plan.mapping()
        assert m["extents"] == extents
        steps = m["schedule"]
        assert [s["step"] for s in steps] == ["axis"] + ["columns"] * (len(extents) - 1)
        assert steps[0]["axis"] == len(extents) - 1
        cols = extents[-1]
        for s, e in zip(steps[1:], reversed(extents[:-1])):
            assert (s["rows"], s["cols"], s["blocks"]) == (e, cols, 2 * n // (e * cols))
            cols *= e


def test_long_fwht_inverse_divides_once(lib):
    # A rank-1 FWHT divides by n after its last stage: the last column pass
    # multiplies by 2^-16 (the GPU tests pin the values, subnormal ones too).
    t = cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [1 << 16], compute=cb.ComputeType.FP32, inverse=True)
    with cb.Plan(lib, t) as plan:
        steps = plan.mapping()["schedule"]
        assert [s["scale"] for s in steps[1:]] == [2.0 ** -16]


def test_long_fp16_fwht_is_promoted(lib):
    # FP16 final-storage rows beyond 2^15 points: widened into an FP32 buffer
    # of the workspace, the factored FP32 plan, one narrowing (the reference's
    # FP32 promotion, src/butterfly.cu:1452-1470).
    n, batch = 1 << 16, 3
    t = cb.describe(cb.Operator.FWHT, cb.DataType.FP16, [n], compute=cb.ComputeType.FP32, batch=batch,
                    output_scale=n ** -0.5, output_rounding=cb.OutputRounding.FINAL_STORAGE)
    with cb.Plan(lib, t) as plan:
        assert plan.algorithm_name().startswith("fwht-fp16-promoted[fwht-factored[")
        assert plan.input_size() == plan.output_size() == batch * n * 2
        m = plan.mapping()
        assert m["kind"] == "fp32-promotion" and m["fp32_buffer_bytes"] == batch * n * 4
        assert m["narrowing"] == "last-column-pass"
        assert m["child"]["extents"] == [16, 4096]
        assert plan.workspace_size() >= batch * n * 4
    # Strided or bit-reversed sides gather to packed rows first.
    strided = cb.describe(cb.Operator.FWHT, cb.DataType.FP16, [n], compute=cb.ComputeType.FP32, batch=batch,
                          input_strides=[2], input_batch_stride=2 * n, output_rounding=cb.OutputRounding.FINAL_STORAGE)
    with cb.Plan(lib, strided) as plan:
        assert plan.algorithm_name().startswith("semantic-boundary[fwht-fp16-promoted[")


def test_long_fwht_strided_sides_use_the_boundary(lib):
    # Pitched or element-strided FP32 rows: the rank-1 boundary (16-byte
    # chunks for pitched rows) around the packed factored plan.
    n = 1 << 16
    for kw in (dict(input_strides=[1], input_batch_stride=n + 64), dict(output_strides=[2], output_batch_stride=2 * n)):
        t = cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [n], compute=cb.ComputeType.FP32, batch=3, **kw)
        with cb.Plan(lib, t) as plan:
            assert plan.algorithm_name().startswith("semantic-boundary[fwht-factored[")


def test_long_fwht_bit_reversed_orders_use_the_boundary(lib):
    # A whole-length bit reversal does not factor into per-axis reversals:
    # the boundary gathers to natural order, and the packed child factors.
    t = cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [1 << 16], compute=cb.ComputeType.FP32, batch=2,
                    input_orders=[cb.LogicalOrder.BIT_REVERSED], output_orders=[cb.LogicalOrder.NATURAL])
    with cb.Plan(lib, t) as plan:
        assert plan.algorithm_name().startswith("semantic-boundary[fwht-factored[")
