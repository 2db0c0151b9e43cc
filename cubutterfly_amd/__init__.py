"""Python view of libcubutterfly (the MI355X butterfly library) for tests and
the benchmark.

A transform is a plain dict in the library's own descriptor JSON schema
(`cubutterfly-semantic-v1`, the text cubutterflyDescriptorGetJson prints),
made by `describe()`. `Plan` hands that JSON to cubutterflyDescriptorSetJson,
so the library alone validates a request; this module adds no rules of its
own and reports the library's status and text (`AbiError`). The enums are
generated from the C headers (`native.py`).

Importing loads nothing; `Native()` loads the built library and fails when it
is missing. Device buffers are ints or objects with data_ptr() (torch
tensors); streams are hipStream_t values.
"""
import ctypes as ct
import json

from .native import AbiError, LibraryMissing, Native, device_address, enums

Status = enums["Status"]
Operator = enums["Operator"]
DataType = enums["DataType"]
ComputeType = enums["ComputeType"]
Placement = enums["Placement"]
LogicalOrder = enums["LogicalOrder"]
NttLayout = enums["NttLayout"]
NttRing = enums["NttRing"]
OutputRounding = enums["OutputRounding"]
ArithmeticPolicy = enums["ArithmeticPolicy"]
AlgorithmPolicy = enums["AlgorithmPolicy"]
SelectionSource = enums["SelectionSource"]
LengthMode = enums["LengthMode"]
ExecutionMode = enums["ExecutionMode"]
FftTransformType = enums["FftTransformType"]

SCHEMA = "cubutterfly-semantic-v1"


def _ints(values):
    return [int(v) for v in values]


# Optional descriptor fields: JSON key -> how the Python value is written.
_FIELDS = {
    "inverse": lambda v: int(bool(v)), "normalize_inverse": bool, "placement": int,
    "fft_type": int, "fft_output_scale": float, "length_mode": int, "execution_mode": int,
    "input_strides": _ints, "output_strides": _ints, "input_batch_stride": int, "output_batch_stride": int,
    "input_orders": _ints, "output_orders": _ints, "ntt_input_layout": int, "ntt_output_layout": int,
    "modulus": int, "word_bits": int, "output_scale": float, "output_rounding": int,
    "arithmetic_policy": int, "ntt_ring": int, "ntt_psi": int,
}


def describe(operator, storage, shape, batch=1, compute=ComputeType.NATIVE, **fields):
    """A descriptor dict: operator, storage type, per-axis extents (outermost
    first), batch, compute domain (NATIVE: the storage's own), plus any
    optional JSON field by its JSON name (`inverse`, `placement`, `modulus`,
    `ntt_ring`, ...). Unset optional fields keep the library's defaults."""
    unknown = sorted(set(fields) - set(_FIELDS))
    if unknown:
        raise KeyError(f"not descriptor JSON fields: {unknown}")
    desc = {"schema": SCHEMA, "operator": int(operator), "storage": int(storage), "shape": _ints(shape),
            "batch": int(batch), "compute": int(compute)}
    desc.update((key, _FIELDS[key](value)) for key, value in fields.items())
    return desc


def _json_text(desc):
    return desc if isinstance(desc, str) else json.dumps(desc)


class DescriptorHandle:
    """A library descriptor object built from JSON text (for the JSON and
    capabilities queries); closed on exit."""

    def __init__(self, native, desc):
        self.native, self.handle = native, ct.c_void_p()
        native("CreateDescriptor", ct.byref(self.handle))
        try:
            native("DescriptorSetJson", self.handle, _json_text(desc).encode())
        except BaseException:
            self.close()
            raise

    def json(self):
        return json.loads(self.native.text("DescriptorGetJson", self.handle))

    def capabilities(self):
        return json.loads(self.native.text("DescriptorGetCapabilities", self.handle))

    def close(self):
        if self.handle.value:
            handle, self.handle = self.handle, ct.c_void_p()
            self.native("DestroyDescriptor", handle)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class Plan:
    """A plan and the library handle it runs through.

    `policy` is an AlgorithmPolicy; `algorithm` (a lowering name) implies
    EXPLICIT. `stream` binds the handle's stream, `cache_path` its selection
    cache. execute() is asynchronous on that stream; the buffers and the
    bound workspace must outlive the queued work.
    """

    def __init__(self, native, desc, *, policy=None, algorithm=None, stream=None, cache_path=None):
        self.native = native
        self.context, self.handle = ct.c_void_p(), ct.c_void_p()
        self.workspace = None
        if algorithm is not None or policy is not None:
            desc = json.loads(desc) if isinstance(desc, str) else dict(desc)
            desc["algorithm_policy"] = int(AlgorithmPolicy.EXPLICIT if algorithm is not None else policy)
            desc["explicit_algorithm"] = algorithm or ""
        try:
            native("Create", ct.byref(self.context))
            if stream is not None:
                native("SetStream", self.context, device_address(stream))
            if cache_path is not None:
                native("SetCachePath", self.context, str(cache_path).encode())
            with DescriptorHandle(native, desc) as d:
                native("CreatePlan", self.context, d.handle, ct.byref(self.handle))
        except BaseException:
            self.close()
            raise

    def _bytes(self, query):
        size = ct.c_size_t(0)
        self.native(query, self.handle, ct.byref(size))
        return size.value

    def workspace_size(self):
        return self._bytes("PlanGetWorkspaceSize")

    def input_size(self):
        return self._bytes("PlanGetInputSize")

    def output_size(self):
        return self._bytes("PlanGetOutputSize")

    def set_workspace(self, buffer, nbytes):
        self.native("PlanSetWorkspace", self.handle, device_address(buffer), nbytes)
        self.workspace = buffer  # keep it alive as long as the plan uses it

    def execute(self, x, y):
        self.native("Execute", self.context, self.handle, device_address(x), device_address(y))

    def execute_steady(self, x, y):
        self.native("ExecuteSteady", self.context, self.handle, device_address(x), device_address(y))

    def algorithm_name(self):
        return self.native.text("PlanGetAlgorithmName", self.handle)

    def selection_reason(self):
        return self.native.text("PlanGetSelectionReason", self.handle)

    def selection_source(self):
        value = ct.c_int()
        self.native("PlanGetSelectionSource", self.handle, ct.byref(value))
        return SelectionSource(value.value)

    def mapping(self):
        return json.loads(self.native.text("PlanGetMappingJson", self.handle))

    def descriptor(self):
        return json.loads(self.native.text("PlanGetDescriptorJson", self.handle))

    def physical_extents(self):
        rank = len(self.descriptor()["shape"])
        out = (ct.c_size_t * rank)()
        self.native("PlanGetPhysicalExtents", self.handle, out, rank)
        return list(out)

    def close(self):
        try:
            if self.handle.value:
                handle, self.handle = self.handle, ct.c_void_p()
                self.native("DestroyPlan", handle)
        finally:
            if self.context.value:
                context, self.context = self.context, ct.c_void_p()
                self.native("Destroy", context)
            self.workspace = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
