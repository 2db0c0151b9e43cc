"""C-ABI checks that need no GPU: the library loads and exports every symbol
the headers declare, descriptors built through the individual setters equal
the same descriptors built from JSON, and the validation / status / error
contract behaves as the reference's (tests/test_c_api.c, src/c_api.cpp:121-163,
3252-3500)."""
import ctypes as ct
import json
import re
from pathlib import Path

import pytest

import cubutterfly_amd as cb
from cubutterfly_amd import native as abi

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    names = set()
    for header in (ROOT / "include").rglob("*.h"):
        names.update(re.findall(r"\b(cubutterfly\w+)\s*\(", header.read_text()))
    return names


def test_every_declared_symbol_is_exported(lib):
    names = declared_symbols()
    assert len(names) >= 50
    assert not [n for n in sorted(names) if not lib.exported(n)]
    # The binding parsed every declaration it binds.
    assert names == set(abi.FUNCTIONS)


def test_enums_parsed_from_the_headers():
    # Values the reference ABI fixes (include/cubutterfly/cubutterfly.h:35-170).
    assert cb.Status.NOT_SUPPORTED == 3 and cb.Status.INTERNAL_ERROR == 7
    assert cb.DataType.COMPLEX_FP32 == 6 and cb.DataType.UINT64 == 9
    assert cb.Operator.FWHT == 2 and cb.NttLayout.BIT_REVERSED == 2
    assert cb.OutputRounding.FINAL_STORAGE == 1 and cb.ArithmeticPolicy.ALLOW_FP16_MMA == 1
    assert cb.SelectionSource.UNMEASURED_FALLBACK == 5 and cb.NttRing.NEGACYCLIC == 1


def test_version_and_status_strings(lib):
    assert lib.version() == (0, 9, 3)
    assert lib.status_text(cb.Status.SUCCESS) == "success"
    assert lib.status_text(cb.Status.NOT_SUPPORTED) == "not supported"
    assert lib.status_text(99) == "unknown status"


def fwht(n=4096, batch=4096, **kw):
    return cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [n], batch, compute=cb.ComputeType.FP32, **kw)


def test_fwht_plan_sizes_and_introspection(lib):
    with cb.Plan(lib, fwht()) as plan:
        assert plan.input_size() == plan.output_size() == 4096 * 4096 * 4
        assert plan.workspace_size() == 0
        assert plan.algorithm_name() == "fwht-fp32-resident-r16"
        mapping = plan.mapping()
        assert mapping["log_n"] == 12 and mapping["tiles"] == 4096 and 1 <= mapping["grid"] <= 4096
        assert plan.selection_source() == cb.SelectionSource.STATIC_MODEL
        d = plan.descriptor()
        assert d["shape"] == [4096] and d["batch"] == 4096 and d["operator"] == int(cb.Operator.FWHT)


def test_fp16_final_storage_plan(lib):
    t = cb.describe(cb.Operator.FWHT, cb.DataType.FP16, [128], 524288, compute=cb.ComputeType.FP32,
                    output_scale=128 ** -0.5, output_rounding=cb.OutputRounding.FINAL_STORAGE)
    with cb.Plan(lib, t) as plan:
        assert plan.input_size() == 524288 * 128 * 2
        assert plan.algorithm_name() == "fwht-fp16-fp32-resident-r16"


def test_fp16_4096_point_rows_default_to_32_registers(lib):
    # C5a's shape: one 2^12-point row per workgroup of 128 threads x 32 registers.
    t = cb.describe(cb.Operator.FWHT, cb.DataType.FP16, [4096], 16384, compute=cb.ComputeType.FP32,
                    output_scale=1 / 64, output_rounding=cb.OutputRounding.FINAL_STORAGE)
    with cb.Plan(lib, t) as plan:
        assert plan.algorithm_name() == "fwht-fp16-fp32-resident-r32"
        mapping = plan.mapping()
        assert mapping["threads_per_block"] == 128 and mapping["registers_per_thread"] == 32
        assert mapping["tiles"] == mapping["grid"] == 16384 and mapping["phases"] == 3


def status_of(fn, *args, **kwargs):
    try:
        fn(*args, **kwargs)
    except cb.AbiError as e:
        return e.status
    return 0


def test_invalid_descriptors_are_rejected(lib):
    # Non-power-of-two FWHT extent: INVALID_VALUE (semantic rule).
    assert status_of(cb.Plan, lib, fwht(n=100)) == cb.Status.INVALID_VALUE
    # Output epilogue on FP32 storage: INVALID_VALUE (src/butterfly.cu:573-576).
    assert status_of(cb.Plan, lib, fwht(output_scale=0.5)) == cb.Status.INVALID_VALUE
    # NTT needs integer storage.
    assert status_of(cb.Plan, lib, cb.describe(cb.Operator.NTT, cb.DataType.FP32, [8])) == cb.Status.INVALID_VALUE
    # Word bits must match storage.
    t = cb.describe(cb.Operator.NTT, cb.DataType.UINT32, [8], compute=cb.ComputeType.UINT32, modulus=998244353,
                    word_bits=64)
    assert status_of(cb.Plan, lib, t) == cb.Status.INVALID_VALUE
    assert status_of(cb.Plan, lib, fwht(batch=0)) == cb.Status.INVALID_VALUE
    with pytest.raises(KeyError):
        fwht(in_place=True)  # not a descriptor JSON field: placement is


def test_unsupported_lowerings_report_not_supported(lib):
    two_d = cb.describe(cb.Operator.FWHT, cb.DataType.FP16, [8, 8], compute=cb.ComputeType.FP32,
                        output_rounding=cb.OutputRounding.FINAL_STORAGE)
    assert status_of(cb.Plan, lib, two_d) == cb.Status.NOT_SUPPORTED
    zeta = cb.describe(cb.Operator.SUBSET_ZETA, cb.DataType.UINT32, [8])
    assert status_of(cb.Plan, lib, zeta) == cb.Status.NOT_SUPPORTED
    assert lib.last_error()


def test_explicit_algorithm_must_match(lib):
    with cb.Plan(lib, fwht(), algorithm="fwht-fp32-resident-r16") as plan:
        assert plan.selection_source() == cb.SelectionSource.EXPLICIT
    assert status_of(cb.Plan, lib, fwht(), algorithm="no-such-kernel") == cb.Status.NOT_SUPPORTED


def test_descriptor_json_round_trip(lib):
    t = cb.describe(cb.Operator.NTT, cb.DataType.UINT32, [65536], 64, compute=cb.ComputeType.UINT32,
                    modulus=1073479681, word_bits=32, ntt_ring=cb.NttRing.NEGACYCLIC, inverse=True)
    with cb.DescriptorHandle(lib, t) as d:
        printed = d.json()
        with cb.DescriptorHandle(lib, printed) as again:
            assert again.json() == printed
        caps = d.capabilities()
        assert caps["eligible"] is True and caps["log_n"] == 16
    with pytest.raises(cb.AbiError) as info:
        cb.DescriptorHandle(lib, '{"schema": "cubutterfly-semantic-v1", "shape": [8], "bogus": 1}')
    assert info.value.status == cb.Status.INVALID_VALUE


def built_with_setters(lib, d):
    """The same descriptor as the JSON dict `d`, made through the individual
    cubutterflySet* entry points a C caller uses."""
    h = ct.c_void_p()
    lib("CreateDescriptor", ct.byref(h))
    sizes = lambda v: (ct.c_size_t * len(v))(*v) if v else None
    lib("SetOperator", h, d["operator"])
    lib("SetDataType", h, d["storage"], d.get("compute", 0))
    lib("SetShape", h, len(d["shape"]), sizes(d["shape"]), d["batch"])
    lib("SetDirection", h, d.get("inverse", 0), int(d.get("normalize_inverse", True)))
    lib("SetPlacement", h, d.get("placement", 0))
    lib("SetOutputScale", h, d.get("output_scale", 1.0))
    lib("SetOutputRounding", h, d.get("output_rounding", 0))
    lib("SetStrides", h, sizes(d.get("input_strides")), d.get("input_batch_stride", 0),
        sizes(d.get("output_strides")), d.get("output_batch_stride", 0))
    if "input_orders" in d:
        orders = lambda v: (ct.c_int * len(v))(*v)
        lib("SetLogicalOrders", h, orders(d["input_orders"]), orders(d["output_orders"]))
    if d["operator"] == cb.Operator.NTT:
        lib("SetModulus", h, d["modulus"], d["word_bits"])
        lib("SetNttRing", h, d.get("ntt_ring", 0), d.get("ntt_psi", 0))
    return h


SETTER_CASES = [
    fwht(),
    cb.describe(cb.Operator.FWHT, cb.DataType.FP16, [4096], 16384, compute=cb.ComputeType.FP32,
                output_scale=1 / 64, output_rounding=cb.OutputRounding.FINAL_STORAGE),
    cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [1 << 14], 1024, compute=cb.ComputeType.FP32),
    cb.describe(cb.Operator.FFT, cb.DataType.COMPLEX_FP32, [64], 3, inverse=True, normalize_inverse=False,
                placement=cb.Placement.IN_PLACE, input_strides=[2], input_batch_stride=200, output_strides=[2],
                output_batch_stride=200),
    cb.describe(cb.Operator.NTT, cb.DataType.UINT32, [1 << 16], 64, compute=cb.ComputeType.UINT32,
                modulus=1073479681, word_bits=32, ntt_ring=cb.NttRing.NEGACYCLIC, inverse=True),
    cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [16], 2, input_orders=[cb.LogicalOrder.BIT_REVERSED],
                output_orders=[cb.LogicalOrder.NATURAL]),
]


@pytest.mark.parametrize("case", range(len(SETTER_CASES)))
def test_setters_and_json_build_the_same_descriptor(lib, case):
    d = SETTER_CASES[case]
    h = built_with_setters(lib, d)
    try:
        from_setters = json.loads(lib.text("DescriptorGetJson", h))
    finally:
        lib("DestroyDescriptor", h)
    with cb.DescriptorHandle(lib, d) as from_json:
        assert from_json.json() == from_setters


def test_placement_and_workspace_contract(lib):
    with cb.Plan(lib, fwht(n=8, batch=1)) as plan:
        # Out-of-place plans reject aliased pointers before touching the device.
        assert status_of(plan.execute, 0x1000, 0x1000) == cb.Status.INVALID_VALUE
        assert status_of(plan.execute, 0, 0x2000) == cb.Status.INVALID_VALUE
        assert status_of(plan.set_workspace, 0x1008, 64) == cb.Status.INVALID_VALUE  # misaligned
    with cb.Plan(lib, fwht(n=8, batch=1, placement=cb.Placement.IN_PLACE)) as plan:
        assert status_of(plan.execute, 0x1000, 0x2000) == cb.Status.INVALID_VALUE


def test_exceptions_never_escape_null_arguments(lib):
    assert lib.fn("CreatePlan")(None, None, None) == cb.Status.INVALID_VALUE
    assert lib.fn("Execute")(None, None, None, None) == cb.Status.INVALID_VALUE
    assert lib.fn("SetShape")(None, 1, None, 1) == cb.Status.INVALID_VALUE
    size = ct.c_size_t(0)
    assert lib.fn("PlanGetWorkspaceSize")(None, ct.byref(size)) == cb.Status.INVALID_VALUE
    assert lib.last_error()


def test_string_query_two_call_protocol(lib):
    with cb.Plan(lib, fwht(n=16, batch=1)) as plan:
        size = ct.c_size_t(0)
        lib("PlanGetAlgorithmName", plan.handle, None, ct.byref(size))
        assert size.value == len("fwht-fp32-resident-r16") + 1
        small = ct.create_string_buffer(4)
        short = ct.c_size_t(4)
        status = lib.fn("PlanGetAlgorithmName")(plan.handle, small, ct.byref(short))
        assert status == cb.Status.INVALID_VALUE and short.value == size.value


def test_abi_error_names_the_entry_point(lib):
    with pytest.raises(cb.AbiError) as info:
        cb.Plan(lib, fwht(n=100))
    e = info.value
    assert e.function == "cubutterflyDescriptorSetJson" and e.status == cb.Status.INVALID_VALUE
    assert str(e).startswith("cubutterflyDescriptorSetJson -> invalid value") and e.detail


LOG_CALLBACK = ct.CFUNCTYPE(None, ct.c_int, ct.c_char_p, ct.c_char_p, ct.c_void_p)


def plan_events(lib, desc, callback_on=True):
    """(level, event, message) of every log callback during one CreatePlan."""
    events = []
    callback = LOG_CALLBACK(lambda level, event, message, user: events.append(
        (abi.enums["LogLevel"](level), event.decode(), message.decode())))
    handle = ct.c_void_p()
    lib("Create", ct.byref(handle))
    try:
        lib("SetLogCallback", handle, ct.cast(callback, ct.c_void_p) if callback_on else None, None)
        with cb.DescriptorHandle(lib, desc) as d:
            plan = ct.c_void_p()
            lib("CreatePlan", handle, d.handle, ct.byref(plan))
            lib("DestroyPlan", plan)
    finally:
        lib("Destroy", handle)
    return events


def test_log_callback_reports_selection_and_profile_miss(lib):
    # The reference's events (src/c_api.cpp:4526-4529, 4782; docs/c_api.md:
    # 193-198): every plan reports `algorithm-selection`; a DEFAULT plan on
    # the static model, with no measured or cached mapping, warns
    # `workload-profile-miss` with the fallback and the MEASURE advice.
    LogLevel = abi.enums["LogLevel"]
    desc = fwht(n=1024, batch=4)
    events = plan_events(lib, desc)
    names = [e[1] for e in events]
    assert "algorithm-selection" in names
    miss = [e for e in events if e[1] == "workload-profile-miss"]
    assert len(miss) == 1 and miss[0][0] == LogLevel.WARNING
    with cb.Plan(lib, desc) as plan:
        chosen = plan.algorithm_name()
    assert f"using {chosen};" in miss[0][2] and "MEASURE" in miss[0][2]
    info = next(e for e in events if e[1] == "algorithm-selection")
    assert info[0] == LogLevel.INFO and info[2].endswith(f"algorithm={chosen}")
    # An explicitly named lowering is no profile miss.
    explicit = dict(desc, algorithm_policy=int(cb.AlgorithmPolicy.EXPLICIT), explicit_algorithm=chosen)
    assert [e[1] for e in plan_events(lib, explicit)] == ["algorithm-selection"]
    # A null callback turns the events off.
    assert plan_events(lib, desc, callback_on=False) == []


def test_capabilities_follow_the_executable_subset(lib):
    # The capabilities query lowers the descriptor as plan creation does:
    # long FP16 and bit-reversed FWHTs are eligible, FP16 at rank 2 is not.
    fp16 = dict(compute=cb.ComputeType.FP32, output_rounding=cb.OutputRounding.FINAL_STORAGE)
    eligible = [
        cb.describe(cb.Operator.FWHT, cb.DataType.FP16, [1 << 16], 4, **fp16),
        cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [1 << 18], 2, compute=cb.ComputeType.FP32,
                    input_orders=[cb.LogicalOrder.BIT_REVERSED], output_orders=[cb.LogicalOrder.NATURAL]),
    ]
    for t in eligible:
        with cb.DescriptorHandle(lib, t) as d:
            assert d.capabilities()["eligible"] is True, t
    with cb.DescriptorHandle(lib, cb.describe(cb.Operator.FWHT, cb.DataType.FP16, [64, 64], 1, **fp16)) as d:
        caps = d.capabilities()
    assert caps["eligible"] is False and "rank one" in caps["reason"]


def test_concurrent_plan_creation_matches_serial(lib):
    # Plans created from several host threads at once (one handle each; ctypes
    # releases the GIL inside the calls) choose the same lowerings as a serial
    # run: the kernel registries fill once and are read-only afterwards, and
    # error strings are per thread.
    from concurrent.futures import ThreadPoolExecutor
    # FWHT plans need no device at creation (FFT and NTT plans upload their
    # twiddle tables; their concurrent creation is a GPU test).
    descs = [
        fwht(n=4096, batch=64),
        fwht(n=1 << 20, batch=2),
        cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [64, 1 << 14], 2, compute=cb.ComputeType.FP32),
        cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [4096], 8, compute=cb.ComputeType.FP32, input_strides=[3]),
        cb.describe(cb.Operator.FWHT, cb.DataType.FP16, [1 << 15], 2, compute=cb.ComputeType.FP32,
                    output_rounding=cb.OutputRounding.FINAL_STORAGE),
    ]

    def name_of(desc):
        with cb.Plan(lib, desc) as plan:
            return plan.algorithm_name()

    bad = [cb.describe(cb.Operator.FWHT, cb.DataType.FP32, [12], 1, compute=cb.ComputeType.FP32),
           cb.describe(cb.Operator.FWHT, cb.DataType.FP16, [64, 64], 1, compute=cb.ComputeType.FP32,
                       output_rounding=cb.OutputRounding.FINAL_STORAGE)]

    def refused(i):
        try:
            cb.Plan(lib, bad[i % 2])
        except cb.AbiError as e:
            return i % 2, e.status, e.detail
        return None

    serial = [name_of(d) for d in descs]
    with ThreadPoolExecutor(max_workers=8) as pool:
        for _ in range(4):
            assert list(pool.map(name_of, descs * 4)) == serial * 4
        errors = list(pool.map(refused, range(64)))
    # Each thread reads its own error text, whichever refusal ran beside it.
    expected = {0: (cb.Status.INVALID_VALUE, "power of two"), 1: (cb.Status.NOT_SUPPORTED, "rank one")}
    for e in errors:
        assert e is not None and e[1] == expected[e[0]][0] and expected[e[0]][1] in e[2], e
