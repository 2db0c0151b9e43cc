"""Semantic boundary (strided sides, FWHT / FFT logical orders) on the CPU:
plan shapes, sizes and layout validation (FWHT plans: FFT and NTT plans
upload tables at creation and are covered by the GPU tests). The rules follow the reference's
boundary plan (src/c_api.cpp:2969-2993, 3085-3130) and its layout normaliser
(src/semantic_contract.cpp:55-123): empty strides are packed, a zero batch
stride is the axis span, and a layout with repeated addresses is invalid.
"""
import json

import pytest

import cubutterfly_amd as cb


def status_of(fn, *args):
    try:
        fn(*args)
    except cb.AbiError as e:
        return e.status
    return 0


def fwht(n=8, batch=2, **kw):
    return cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [n], compute=cb.ComputeType.FP32, batch=batch, **kw)


def align16(b):
    return (b + 15) // 16 * 16


def test_strided_input_uses_the_boundary(lib):
    t = fwht(n=8, batch=3, input_strides=[2], input_batch_stride=20)
    with cb.Plan(lib, t) as plan:
        assert plan.algorithm_name() == "semantic-boundary[fwht-fp32-resident-r16]"
        assert plan.input_size() == ((8 - 1) * 2 + (3 - 1) * 20 + 1) * 4
        assert plan.output_size() == 8 * 3 * 4
        assert plan.workspace_size() == 2 * align16(8 * 3 * 4)
        m = plan.mapping()
        assert m["kind"] == "semantic-boundary" and m["input_stride"] == 2 and m["input_batch_stride"] == 20
        assert m["child"]["operator"] == "fwht"
        assert m["direct_input"] is False and m["direct_output"] is True


@pytest.mark.parametrize("reversed_input", [True, False])
def test_packed_natural_side_skips_its_move(lib, reversed_input):
    # One bit-reversed side: the other, packed in natural order, is read or
    # written by the packed plan itself.
    orders = {"input_orders" if reversed_input else "output_orders": [cb.LogicalOrder.BIT_REVERSED]}
    with cb.Plan(lib, fwht(n=1024, batch=4, **orders)) as plan:
        m = plan.mapping()
        assert plan.algorithm_name().startswith("semantic-boundary[")
        assert m["direct_input"] is (not reversed_input) and m["direct_output"] is reversed_input


def test_default_batch_stride_is_the_axis_span(lib):
    with cb.Plan(lib, fwht(n=8, batch=2, output_strides=[3])) as plan:
        assert plan.mapping()["output_batch_stride"] == (8 - 1) * 3 + 1
        assert plan.output_size() == ((8 - 1) * 3 + (8 - 1) * 3 + 1 + 1) * 4


def test_packed_plans_stay_direct(lib):
    with cb.Plan(lib, fwht(n=8, batch=2, input_strides=[1], input_batch_stride=8)) as plan:
        assert plan.algorithm_name() == "fwht-fp32-resident-r16"


@pytest.mark.parametrize("strides,batch_stride,batch,n", [
    ([1], 4, 2, 8),        # batches overlap (stride 4 < span 8)
    ([2], 1, 4, 8),        # 2 a = b: (element 1, batch 0) == (element 0, batch 2)
    ([3], 6, 3, 4),        # batch 1 element 0 == batch 0 element 2
])
def test_overlapping_layouts_are_invalid(lib, strides, batch_stride, batch, n):
    t = fwht(n=n, batch=batch, input_strides=strides, input_batch_stride=batch_stride)
    assert status_of(cb.Plan, lib, t) == cb.Status.INVALID_VALUE


@pytest.mark.parametrize("strides,batch_stride,batch,n", [
    ([4], 1, 4, 8),        # interleaved batches
    ([2], 1, 2, 8),        # two interleaved rows
    ([1], 9, 3, 8),        # gaps between rows
])
def test_disjoint_layouts_are_valid(lib, strides, batch_stride, batch, n):
    assert status_of(cb.Plan, lib, fwht(n=n, batch=batch, input_strides=strides,
                                        input_batch_stride=batch_stride)) == 0


def test_zero_stride_is_invalid(lib):
    assert status_of(cb.Plan, lib, fwht(input_strides=[0])) == cb.Status.INVALID_VALUE
