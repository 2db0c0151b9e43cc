"""C-ABI checks that need no GPU: the library loads, exports every symbol the
headers declare, and the descriptor / validation / error contract behaves like
the reference (tests/test_c_api.c, src/c_api.cpp:121-163, 3252-3500)."""
import ctypes as ct
import json
import re
from pathlib import Path

import pytest

import cubutterfly_amd as cb

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    names = set()
    for header in (ROOT / "include").rglob("*.h"):
        text = header.read_text()
        names.update(re.findall(r"\b(cubutterfly\w+)\s*\(", text))
    return names


def test_every_declared_symbol_is_exported(lib):
    names = declared_symbols()
    assert len(names) >= 50
    missing = [n for n in sorted(names) if getattr(lib._dll, n, None) is None]
    assert not missing, missing


def test_version_and_status_strings(lib):
    assert lib.version() == (0, 9, 3)
    assert lib.status_string(cb.Status.SUCCESS) == "success"
    assert lib.status_string(cb.Status.NOT_SUPPORTED) == "not supported"
    assert lib.status_string(99) == "unknown status"


def fwht(n=4096, batch=4096, **kw):
    return cb.Transform(op=cb.Operator.FWHT, storage=cb.DataType.FP32, compute=cb.ComputeType.FP32,
                        extents=[n], batch=batch, **kw)


def test_fwht_plan_sizes_and_introspection(lib):
    with cb.Plan(lib, fwht()) as plan:
        assert plan.input_size() == plan.output_size() == 4096 * 4096 * 4
        assert plan.workspace_size() == 0
        assert plan.algorithm_name() == "fwht-fp32-resident-r16"
        mapping = json.loads(plan.mapping_json())
        assert mapping["log_n"] == 12 and mapping["tiles"] == 4096 and 1 <= mapping["grid"] <= 4096
        assert plan.selection_source() == cb.SelectionSource.STATIC_MODEL
        d = json.loads(plan.descriptor_json())
        assert d["shape"] == [4096] and d["batch"] == 4096 and d["operator"] == int(cb.Operator.FWHT)


def test_fp16_final_storage_plan(lib):
    t = cb.Transform(op=cb.Operator.FWHT, storage=cb.DataType.FP16, compute=cb.ComputeType.FP32,
                     extents=[128], batch=524288, output_scale=128 ** -0.5,
                     output_rounding=cb.OutputRounding.FINAL_STORAGE)
    with cb.Plan(lib, t) as plan:
        assert plan.input_size() == 524288 * 128 * 2
        assert plan.algorithm_name() == "fwht-fp16-fp32-resident-r16"


def test_fp16_4096_point_rows_default_to_32_registers(lib):
    # C5a's shape: one 2^12-point row per workgroup of 128 threads x 32 registers.
    t = cb.Transform(op=cb.Operator.FWHT, storage=cb.DataType.FP16, compute=cb.ComputeType.FP32,
                     extents=[4096], batch=16384, output_scale=1 / 64,
                     output_rounding=cb.OutputRounding.FINAL_STORAGE)
    with cb.Plan(lib, t) as plan:
        assert plan.algorithm_name() == "fwht-fp16-fp32-resident-r32"
        mapping = json.loads(plan.mapping_json())
        assert mapping["threads_per_block"] == 128 and mapping["registers_per_thread"] == 32
        assert mapping["tiles"] == mapping["grid"] == 16384 and mapping["phases"] == 3


def status_of(fn, *args):
    try:
        fn(*args)
    except cb.Error as e:
        return e.status
    return 0


def test_invalid_descriptors_are_rejected(lib):
    # Non-power-of-two FWHT extent: INVALID_VALUE (semantic rule).
    assert status_of(cb.Plan, lib, fwht(n=100)) == cb.Status.INVALID_VALUE
    # Output epilogue on FP32 storage: INVALID_VALUE (src/butterfly.cu:573-576).
    assert status_of(cb.Plan, lib, fwht(output_scale=0.5)) == cb.Status.INVALID_VALUE
    # NTT needs integer storage.
    t = cb.Transform(op=cb.Operator.NTT, storage=cb.DataType.FP32, extents=[8])
    assert status_of(cb.Plan, lib, t) == cb.Status.INVALID_VALUE
    # Word bits must match storage.
    t = cb.Transform(op=cb.Operator.NTT, storage=cb.DataType.UINT32, compute=cb.ComputeType.UINT32,
                     extents=[8], modulus=998244353, word_bits=64)
    assert status_of(cb.Plan, lib, t) == cb.Status.INVALID_VALUE
    # Zero batch is rejected at SetShape.
    assert status_of(cb.Plan, lib, fwht(batch=0)) == cb.Status.INVALID_VALUE


def test_unsupported_lowerings_report_not_supported(lib):
    two_d = cb.Transform(op=cb.Operator.FWHT, storage=cb.DataType.FP16, compute=cb.ComputeType.FP32,
                         output_rounding=cb.OutputRounding.FINAL_STORAGE, extents=[8, 8])
    assert status_of(cb.Plan, lib, two_d) == cb.Status.NOT_SUPPORTED
    zeta = cb.Transform(op=cb.Operator.SUBSET_ZETA, storage=cb.DataType.UINT32, extents=[8])
    assert status_of(cb.Plan, lib, zeta) == cb.Status.NOT_SUPPORTED
    assert "rank" in lib.last_error() or "lowering" in lib.last_error() or lib.last_error()


def test_explicit_algorithm_must_match(lib):
    ok = cb.PlanOptions(mapping="fwht-fp32-resident-r16")
    with cb.Plan(lib, fwht(), options=ok) as plan:
        assert plan.selection_source() == cb.SelectionSource.EXPLICIT
    bad = cb.PlanOptions(mapping="no-such-kernel")
    assert status_of(cb.Plan, lib, fwht(), bad) == cb.Status.NOT_SUPPORTED


def test_descriptor_json_round_trip(lib):
    t = cb.Transform(op=cb.Operator.NTT, storage=cb.DataType.UINT32, compute=cb.ComputeType.UINT32,
                     extents=[65536], batch=64, modulus=1073479681, word_bits=32,
                     ring=cb.NttRing.NEGACYCLIC, inverse=True)
    with cb.Descriptor(lib, t) as d:
        text = d.json()
        with cb.Descriptor.from_json(lib, text) as again:
            assert json.loads(again.json()) == json.loads(text)
        caps = json.loads(d.capabilities_json())
        assert caps["eligible"] is True and caps["log_n"] == 16
    with pytest.raises(cb.Error) as info:
        cb.Descriptor.from_json(lib, '{"schema": "cubutterfly-semantic-v1", "shape": [8], "bogus": 1}')
    assert info.value.status == cb.Status.INVALID_VALUE


def test_placement_and_workspace_contract(lib):
    with cb.Plan(lib, fwht(n=8, batch=1)) as plan:
        # Out-of-place plans reject aliased pointers before touching the device.
        assert status_of(plan.execute, 0x1000, 0x1000) == cb.Status.INVALID_VALUE
        assert status_of(plan.execute, 0, 0x2000) == cb.Status.INVALID_VALUE
        assert status_of(plan.set_workspace, 0x1008, 64) == cb.Status.INVALID_VALUE  # misaligned
    with cb.Plan(lib, fwht(n=8, batch=1, in_place=True)) as plan:
        assert status_of(plan.execute, 0x1000, 0x2000) == cb.Status.INVALID_VALUE


def test_exceptions_never_escape_null_arguments(lib):
    f = lib._functions
    assert f["CreatePlan"](None, None, None) == cb.Status.INVALID_VALUE
    assert f["Execute"](None, None, None, None) == cb.Status.INVALID_VALUE
    assert f["SetShape"](None, 1, None, 1) == cb.Status.INVALID_VALUE
    size = ct.c_size_t(0)
    assert f["PlanGetWorkspaceSize"](None, ct.byref(size)) == cb.Status.INVALID_VALUE
    assert lib.last_error()


def test_string_query_two_call_protocol(lib):
    with cb.Plan(lib, fwht(n=16, batch=1)) as plan:
        size = ct.c_size_t(0)
        lib._call("PlanGetAlgorithmName", plan.native_handle, None, ct.byref(size))
        assert size.value == len("fwht-fp32-resident-r16") + 1
        small = ct.create_string_buffer(4)
        short = ct.c_size_t(4)
        status = lib._functions["PlanGetAlgorithmName"](plan.native_handle, small, ct.byref(short))
        assert status == cb.Status.INVALID_VALUE and short.value == size.value
