"""Zero-extended embedding plans on the CPU host (reference
docs/c_api.md:74-79, semantic_contract.cpp:43-53): each axis runs at its next
power of two; the forward input and the inverse output keep the logical
extents; sizes and physical extents are queryable. FWHT plans allocate
nothing at creation, so their shapes are checkable without a device."""
import json

import pytest

import cubutterfly_amd as cb


def fwht(extents, **kw):
    return cb.describe(cb.Operator.FWHT, cb.DataType.FP32, list(extents), compute=cb.ComputeType.FP32, length_mode=cb.LengthMode.ZERO_EXTENDED_EMBEDDING, **kw)


def test_forward_sizes_and_names(lib):
    with cb.Plan(lib, fwht([100], batch=3)) as plan:
        assert plan.physical_extents() == [128]
        assert plan.input_size() == 3 * 100 * 4
        assert plan.output_size() == 3 * 128 * 4
        assert plan.algorithm_name() == "zero-extended[fwht-fp32-resident-r16]+direct-output"
        assert plan.workspace_size() == 3 * 128 * 4  # the zero-filled input
        m = plan.mapping()
        assert m["zero_extended"] is True and m["input_extents"] == [100] and m["output_extents"] == [128]


def test_inverse_reverses_the_extents(lib):
    with cb.Plan(lib, fwht([100], batch=3, inverse=True)) as plan:
        assert plan.input_size() == 3 * 128 * 4
        assert plan.output_size() == 3 * 100 * 4
        assert plan.algorithm_name().startswith("zero-extended[") and "+direct-input" in plan.algorithm_name()


def test_rank2_embedding(lib):
    with cb.Plan(lib, fwht([5, 12], batch=2)) as plan:
        assert plan.physical_extents() == [8, 16]
        assert plan.input_size() == 2 * 60 * 4 and plan.output_size() == 2 * 128 * 4
        assert plan.algorithm_name().startswith("rank2-kronecker[")


def test_power_of_two_extent_is_unchanged(lib):
    with cb.Plan(lib, fwht([64], batch=2)) as plan:
        assert plan.physical_extents() == [64]
        assert plan.input_size() == plan.output_size() == 2 * 64 * 4


def test_orders_need_power_of_two_side_extents(lib):
    bad = fwht([100], input_orders=[cb.LogicalOrder.BIT_REVERSED])
    with pytest.raises(cb.AbiError) as e:
        cb.Plan(lib, bad)
    assert e.value.status == cb.Status.INVALID_VALUE
    ok = fwht([100], output_orders=[cb.LogicalOrder.BIT_REVERSED])  # the padded side
    with cb.Plan(lib, ok) as plan:
        assert "+direct-output" not in plan.algorithm_name()


def test_not_supported_embeddings(lib):
    fp16 = cb.describe(cb.Operator.FWHT, cb.DataType.FP16, [100], compute=cb.ComputeType.FP32, output_rounding=cb.OutputRounding.FINAL_STORAGE, length_mode=cb.LengthMode.ZERO_EXTENDED_EMBEDDING)
    for t in (fp16, fwht([1])):
        with pytest.raises(cb.AbiError) as e:
            cb.Plan(lib, t)
        assert e.value.status == cb.Status.NOT_SUPPORTED, lib.last_error()
