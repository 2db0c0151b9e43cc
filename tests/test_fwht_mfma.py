"""Selection of the MFMA Hadamard-block FP16 FWHT (no GPU needed). Under
ALLOW_FP16_MMA the default stays the bit-exact stage-ordered VALU kernel (the
reference keeps its native selection unless a calibrated MMA profile wins,
src/mapping_selector.cpp:13-44); the MFMA kernel is taken by name and is a
MEASURE candidate; STRICT never uses it (reference
include/cubutterfly/cubutterfly.h:86-90)."""
import pytest

import cubutterfly_amd as cb

MMA = cb.ArithmeticPolicy.ALLOW_FP16_MMA
MFMA = "fwht-fp16-mfma16"


def fp16(n, batch, policy=MMA, **kw):
    return cb.describe(cb.Operator.FWHT, cb.DataType.FP16, [n], batch, compute=cb.ComputeType.FP32,
                       output_scale=n ** -0.5, output_rounding=cb.OutputRounding.FINAL_STORAGE,
                       arithmetic_policy=policy, **kw)


@pytest.mark.parametrize("n,batch", [(4096, 16384), (128, 524288), (2, 3), (16, 5), (512, 7)])
def test_allow_mma_default_is_the_stage_ordered_kernel(lib, n, batch):
    with cb.Plan(lib, fp16(n, batch, policy=cb.ArithmeticPolicy.STRICT)) as strict:
        expected = strict.algorithm_name()
    with cb.Plan(lib, fp16(n, batch)) as plan:
        assert plan.algorithm_name() == expected
        assert plan.algorithm_name() != MFMA
        reason = plan.selection_reason()
        assert "stage-ordered VALU kernel kept as the default" in reason and MFMA in reason


@pytest.mark.parametrize("n,batch", [(4096, 16384), (128, 524288), (2, 3), (16, 5), (512, 7)])
def test_allow_mma_explicit_name_selects_the_mfma_kernel(lib, n, batch):
    with cb.Plan(lib, fp16(n, batch), algorithm=MFMA) as plan:
        assert plan.algorithm_name() == MFMA
        m = plan.mapping()
        assert m["lds_bytes"] == 0 and m["tile_elements"] == 4096
        assert m["tiles"] == -(-n * batch // 4096)
        assert m["mfma_per_tile"] == (48 if n > 16 else 16)
        reason = plan.selection_reason()
        assert "MFMA" in reason and "one fp16 ulp" in reason and "inf or NaN" in reason


def test_strict_never_uses_mfma(lib):
    with cb.Plan(lib, fp16(4096, 64, policy=cb.ArithmeticPolicy.STRICT)) as plan:
        assert plan.algorithm_name() == "fwht-fp16-fp32-resident-r32"
    with pytest.raises(cb.AbiError) as e:
        cb.Plan(lib, fp16(4096, 64, policy=cb.ArithmeticPolicy.STRICT), algorithm=MFMA)
    assert e.value.status == cb.Status.NOT_SUPPORTED and "ALLOW_FP16_MMA" in e.value.detail


def test_explicit_valu_lowering_under_allow_mma(lib):
    with cb.Plan(lib, fp16(4096, 64), algorithm="fwht-fp16-fp32-resident-r16") as plan:
        assert plan.algorithm_name() == "fwht-fp16-fp32-resident-r16"


def test_uncovered_requests_name_the_valu_fallback(lib):
    # 2^13-point rows exceed the 4096-element wave tile; pitched rows are not covered.
    with cb.Plan(lib, fp16(8192, 4)) as plan:
        assert plan.algorithm_name().startswith("fwht-fp16-fp32-resident")
        assert "stage-ordered VALU kernel used" in plan.selection_reason()
    pitched = fp16(256, 8, input_strides=[1], input_batch_stride=272, output_strides=[1], output_batch_stride=272)
    with cb.Plan(lib, pitched) as plan:
        assert plan.algorithm_name().endswith("-pitched")
        assert "stage-ordered VALU kernel used" in plan.selection_reason()
    with pytest.raises(cb.AbiError) as e:
        cb.Plan(lib, fp16(8192, 4), algorithm=MFMA)
    assert e.value.status == cb.Status.NOT_SUPPORTED
