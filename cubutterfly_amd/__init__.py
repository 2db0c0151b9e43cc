"""Python frontend over libcubutterfly's C ABI (include/cubutterfly/cubutterfly.h).

Mirrors the reference's ctypes frontend (python/cubutterfly/__init__.py:33-460):
the same enums, Transform/PlanOptions dataclasses and Library/Descriptor/Plan
classes with the same argument meaning and error behaviour (a failing call
raises Error carrying the status code and the library's detail string).
Importing this module loads nothing; Library() loads the in-tree
libcubutterfly.so (or CUBUTTERFLY_LIBRARY) and raises if it is not built --
there is no CPU fallback. Device pointers may be ints, ctypes pointers or any
object with data_ptr() (torch tensors); streams are hipStream_t handles.
"""
import ctypes as ct
import json
import operator
import os
from dataclasses import dataclass, field
from enum import IntEnum
from pathlib import Path

_HERE = Path(__file__).resolve().parent
DEFAULT_LIBRARY = _HERE / "libcubutterfly.so"
DEFAULT_MODULUS = 1152921504606584833


class Operator(IntEnum):
    FFT = 0
    NTT = 1
    FWHT = 2
    SUBSET_ZETA = 3
    SUPERSET_ZETA = 4
    STRUCTURED_2X2 = 5


class DataType(IntEnum):
    FP16 = 0
    BF16 = 1
    FP32 = 2
    FP64 = 3
    COMPLEX_FP16 = 4
    COMPLEX_BF16 = 5
    COMPLEX_FP32 = 6
    COMPLEX_FP64 = 7
    UINT32 = 8
    UINT64 = 9


class ComputeType(IntEnum):
    NATIVE = 0
    FP32 = 1
    FP64 = 2
    UINT32 = 3
    UINT64 = 4


class Status(IntEnum):
    SUCCESS = 0
    INVALID_VALUE = 1
    INVALID_TYPE = 2
    NOT_SUPPORTED = 3
    ALLOC_FAILED = 4
    CUDA_ERROR = 5
    BACKEND_ERROR = 6
    INTERNAL_ERROR = 7


class LogicalOrder(IntEnum):
    NATURAL = 0
    BIT_REVERSED = 1


class NttLayout(IntEnum):
    NATURAL = 0
    APPT_STATIC = 1
    BIT_REVERSED = 2


class ExecutionMode(IntEnum):
    AUTO = 0
    XD = 1
    COMPOSITE = 2


class AlgorithmPolicy(IntEnum):
    DEFAULT = 0
    MEASURE = 1
    EXPLICIT = 2


class FftType(IntEnum):
    C2C = 0
    R2C = 1
    C2R = 2


class LengthMode(IntEnum):
    STANDARD = 0
    ZERO_EXTENDED_EMBEDDING = 1


class ArithmeticPolicy(IntEnum):
    STRICT = 0
    ALLOW_FP16_MMA = 1


class OutputRounding(IntEnum):
    STAGE_STORAGE = 0
    FINAL_STORAGE = 1


class SelectionSource(IntEnum):
    MEASURED_TABLE = 0
    USER_CACHE = 1
    RUNTIME_MEASURED = 2
    STATIC_MODEL = 3
    EXPLICIT = 4
    UNMEASURED_FALLBACK = 5


class NttRing(IntEnum):
    """Extension (include/cubutterfly/cubutterfly_mi355x.h)."""
    CYCLIC = 0
    NEGACYCLIC = 1


@dataclass
class Transform:
    op: int = Operator.FFT
    storage: int = DataType.COMPLEX_FP32
    compute: int = ComputeType.NATIVE
    extents: list = field(default_factory=lambda: [256])
    batch: int = 1
    inverse: bool = False
    normalize_inverse: bool = True
    in_place: bool = False
    fft_type: int = FftType.C2C
    fft_output_scale: float = 1.0
    output_scale: float = 1.0
    output_rounding: int = OutputRounding.STAGE_STORAGE
    arithmetic_policy: int = ArithmeticPolicy.STRICT
    length_mode: int = LengthMode.STANDARD
    input_strides: list = field(default_factory=list)
    output_strides: list = field(default_factory=list)
    input_batch_stride: int = 0
    output_batch_stride: int = 0
    modulus: int = DEFAULT_MODULUS
    word_bits: int = 64
    input_orders: list = field(default_factory=list)
    output_orders: list = field(default_factory=list)
    input_order: int = NttLayout.NATURAL
    output_order: int = NttLayout.NATURAL
    execution_mode: int = ExecutionMode.AUTO
    ring: int = NttRing.CYCLIC
    psi: int = 0


@dataclass
class PlanOptions:
    policy: int = AlgorithmPolicy.DEFAULT
    mapping: str = ""
    execution_mode: int = ExecutionMode.AUTO


class Error(RuntimeError):
    def __init__(self, message, status=None):
        super().__init__(message)
        self.status = status


_P, _N, _I = ct.c_void_p, ct.c_size_t, ct.c_int

# name -> argtypes; every function returns a status int unless noted.
_SIGNATURES = {
    "GetVersion": [ct.POINTER(_I)] * 3,
    "Create": [ct.POINTER(_P)], "Destroy": [_P], "SetStream": [_P, _P], "GetStream": [_P, ct.POINTER(_P)],
    "SetCachePath": [_P, ct.c_char_p],
    "CreateDescriptor": [ct.POINTER(_P)], "DestroyDescriptor": [_P],
    "SetOperator": [_P, _I], "SetDataType": [_P, _I, _I],
    "SetShape": [_P, ct.c_uint32, ct.POINTER(_N), _N], "SetExecutionMode": [_P, _I],
    "SetFftTransformType": [_P, _I], "SetFftOutputScale": [_P, ct.c_double],
    "SetOutputScale": [_P, ct.c_double], "SetArithmeticPolicy": [_P, _I], "SetOutputRounding": [_P, _I],
    "SetStrides": [_P, ct.POINTER(_N), _N, ct.POINTER(_N), _N],
    "SetLogicalOrders": [_P, ct.POINTER(_I), ct.POINTER(_I)],
    "SetDirection": [_P, _I, _I], "SetPlacement": [_P, _I], "SetLengthMode": [_P, _I],
    "SetAlgorithmPolicy": [_P, _I, ct.c_char_p], "SetModulus": [_P, ct.c_uint64, ct.c_uint32],
    "SetNttLayouts": [_P, _I, _I], "SetNttRing": [_P, _I, ct.c_uint64],
    "DescriptorValidate": [_P], "DescriptorSetJson": [_P, ct.c_char_p],
    "CreatePlan": [_P, _P, ct.POINTER(_P)], "DestroyPlan": [_P],
    "PlanSetWorkspace": [_P, _P, _N], "Execute": [_P, _P, _P, _P], "ExecuteSteady": [_P, _P, _P, _P],
    "PlanGetSelectionSource": [_P, ct.POINTER(_I)],
    "PlanGetPhysicalExtents": [_P, ct.POINTER(_N), ct.c_uint32],
}
for _name in ("DescriptorGetJson", "DescriptorGetCapabilities", "PlanGetMappingJson",
              "PlanGetDescriptorJson", "PlanGetAlgorithmName", "PlanGetSelectionReason"):
    _SIGNATURES[_name] = [_P, _P, ct.POINTER(_N)]
for _name in ("PlanGetWorkspaceSize", "PlanGetInputSize", "PlanGetOutputSize"):
    _SIGNATURES[_name] = [_P, ct.POINTER(_N)]


class Library:
    """Loaded libcubutterfly with every ABI function bound once."""

    def __init__(self, path=None):
        path = Path(path or os.environ.get("CUBUTTERFLY_LIBRARY") or DEFAULT_LIBRARY)
        if not path.exists():
            raise Error(f"libcubutterfly is not built at {path}; run python -m cubutterfly_amd.build")
        self.path = path
        self._dll = ct.CDLL(os.fspath(path))
        self._functions = {}
        for name, argtypes in _SIGNATURES.items():
            function = getattr(self._dll, "cubutterfly" + name)
            function.argtypes = argtypes
            function.restype = _I
            self._functions[name] = function
        for name in ("GetStatusString", "GetLastErrorString"):
            function = getattr(self._dll, "cubutterfly" + name)
            function.argtypes = [_I] if name == "GetStatusString" else []
            function.restype = ct.c_char_p
            self._functions[name] = function

    def status_string(self, status):
        return self._functions["GetStatusString"](int(status)).decode("utf-8", "replace")

    def last_error(self):
        return (self._functions["GetLastErrorString"]() or b"").decode("utf-8", "replace")

    def _call(self, name, *args):
        status = self._functions[name](*args)
        if status:
            detail = self.last_error()
            raise Error(self.status_string(status) + (": " + detail if detail else ""), status)

    def _query(self, name, handle):
        size = ct.c_size_t()
        self._call(name, handle, None, ct.byref(size))
        buffer = ct.create_string_buffer(size.value)
        self._call(name, handle, buffer, ct.byref(size))
        return buffer.value.decode("utf-8")

    def version(self):
        parts = [ct.c_int() for _ in range(3)]
        self._call("GetVersion", *[ct.byref(p) for p in parts])
        return tuple(p.value for p in parts)


def _array(kind, values):
    return (kind * len(values))(*values) if values else None


def _integer(value, name, kind):
    if isinstance(value, bool):
        raise TypeError(f"{name} must be an integer, not bool")
    try:
        result = operator.index(value)
    except TypeError as exc:
        raise TypeError(f"{name} must be an integer") from exc
    bits = ct.sizeof(kind) * 8
    maximum = (1 << (bits - 1)) - 1 if kind is ct.c_int else (1 << bits) - 1
    if not 0 <= result <= maximum:
        raise ValueError(f"{name} is outside the {kind.__name__} ABI range")
    return result


def pointer(value):
    """Device pointer of an int, ctypes pointer or object with data_ptr()."""
    if hasattr(value, "data_ptr"):
        value = value.data_ptr()
    return value if isinstance(value, ct.c_void_p) else ct.c_void_p(value)


class Descriptor:
    def __init__(self, library, transform, options=None):
        self.library = library
        self._handle = ct.c_void_p()
        library._call("CreateDescriptor", ct.byref(self._handle))
        try:
            self._configure(transform, options or PlanOptions())
        except BaseException:
            self.close()
            raise

    def _configure(self, t, options):
        for name in ("inverse", "normalize_inverse", "in_place"):
            if not isinstance(getattr(t, name), bool):
                raise TypeError(f"{name} must be bool")
        rank = len(t.extents)
        _integer(rank, "rank", ct.c_uint32)
        for values in (t.input_strides, t.output_strides, t.input_orders, t.output_orders):
            if values and len(values) != rank:
                raise ValueError("one entry is required per axis")
        legacy = t.input_order != NttLayout.NATURAL or t.output_order != NttLayout.NATURAL
        if legacy and t.op != Operator.NTT:
            raise ValueError("legacy NTT layouts require an NTT operator")
        if t.op != Operator.NTT and (t.modulus != DEFAULT_MODULUS or t.word_bits != 64):
            raise ValueError("modulus and word_bits require an NTT operator")
        if legacy and (t.input_orders or t.output_orders):
            raise ValueError("legacy NTT layouts and logical orders are ambiguous")
        call = lambda name, *args: self.library._call(name, self._handle, *args)
        extents = [_integer(v, "extents", ct.c_size_t) for v in t.extents]
        call("SetOperator", _integer(t.op, "op", ct.c_int))
        call("SetDataType", _integer(t.storage, "storage", ct.c_int), _integer(t.compute, "compute", ct.c_int))
        call("SetShape", rank, _array(ct.c_size_t, extents), _integer(t.batch, "batch", ct.c_size_t))
        call("SetExecutionMode", _integer(options.execution_mode or t.execution_mode, "execution_mode", ct.c_int))
        call("SetFftTransformType", _integer(t.fft_type, "fft_type", ct.c_int))
        call("SetFftOutputScale", float(t.fft_output_scale))
        call("SetOutputScale", float(t.output_scale))
        call("SetOutputRounding", _integer(t.output_rounding, "output_rounding", ct.c_int))
        call("SetArithmeticPolicy", _integer(t.arithmetic_policy, "arithmetic_policy", ct.c_int))
        call("SetStrides", _array(ct.c_size_t, [_integer(v, "input_strides", ct.c_size_t) for v in t.input_strides]),
             _integer(t.input_batch_stride, "input_batch_stride", ct.c_size_t),
             _array(ct.c_size_t, [_integer(v, "output_strides", ct.c_size_t) for v in t.output_strides]),
             _integer(t.output_batch_stride, "output_batch_stride", ct.c_size_t))
        call("SetDirection", int(t.inverse), int(t.normalize_inverse))
        call("SetPlacement", int(t.in_place))
        call("SetLengthMode", _integer(t.length_mode, "length_mode", ct.c_int))
        policy = AlgorithmPolicy.EXPLICIT if options.mapping else _integer(options.policy, "policy", ct.c_int)
        call("SetAlgorithmPolicy", policy, options.mapping.encode("utf-8") if options.mapping else None)
        if t.op == Operator.NTT:
            call("SetModulus", _integer(t.modulus, "modulus", ct.c_uint64), _integer(t.word_bits, "word_bits", ct.c_uint32))
            call("SetNttLayouts", _integer(t.input_order, "input_order", ct.c_int),
                 _integer(t.output_order, "output_order", ct.c_int))
            call("SetNttRing", _integer(t.ring, "ring", ct.c_int), _integer(t.psi, "psi", ct.c_uint64))
        if not legacy:
            call("SetLogicalOrders", _array(ct.c_int, [_integer(v, "input_orders", ct.c_int) for v in t.input_orders]),
                 _array(ct.c_int, [_integer(v, "output_orders", ct.c_int) for v in t.output_orders]))

    @classmethod
    def from_json(cls, library, text):
        result = cls.__new__(cls)
        result.library, result._handle = library, ct.c_void_p()
        library._call("CreateDescriptor", ct.byref(result._handle))
        try:
            library._call("DescriptorSetJson", result._handle, text.encode("utf-8"))
        except BaseException:
            result.close()
            raise
        return result

    @property
    def native_handle(self):
        if not self._handle.value:
            raise Error("descriptor is closed")
        return self._handle

    def validate(self):
        self.library._call("DescriptorValidate", self.native_handle)

    def json(self):
        return self.library._query("DescriptorGetJson", self.native_handle)

    def capabilities_json(self):
        return self.library._query("DescriptorGetCapabilities", self.native_handle)

    def close(self):
        if self._handle.value:
            handle, self._handle = self._handle, ct.c_void_p()
            self.library._call("DestroyDescriptor", handle)

    def __enter__(self):
        return self

    def __exit__(self, *args):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Plan:
    """Plan with its own handle (context) and a caller-bound workspace.

    execute() is asynchronous on the plan's stream; input, output and
    workspace must stay alive until the work completes. `cache_path` names
    the selection cache: DEFAULT plans replay its records, MEASURE plans
    append the candidate they measured fastest.
    """

    def __init__(self, library, transform, options=None, stream=None, cache_path=None):
        self.library = library
        self._context, self._handle = ct.c_void_p(), ct.c_void_p()
        self._workspace = None
        try:
            library._call("Create", ct.byref(self._context))
            if stream is not None:
                library._call("SetStream", self._context, pointer(stream))
            if cache_path is not None:
                library._call("SetCachePath", self._context, os.fsencode(cache_path))
            if isinstance(transform, Descriptor):
                if options is not None:
                    raise ValueError("selection options must be set when constructing the Descriptor")
                library._call("CreatePlan", self._context, transform.native_handle, ct.byref(self._handle))
            else:
                with Descriptor(library, transform, options) as descriptor:
                    library._call("CreatePlan", self._context, descriptor.native_handle, ct.byref(self._handle))
        except BaseException:
            self.close()
            raise

    @property
    def native_handle(self):
        if not self._handle.value:
            raise Error("plan is closed")
        return self._handle

    def _size(self, name):
        size = ct.c_size_t()
        self.library._call(name, self.native_handle, ct.byref(size))
        return size.value

    def workspace_size(self):
        return self._size("PlanGetWorkspaceSize")

    def input_size(self):
        return self._size("PlanGetInputSize")

    def output_size(self):
        return self._size("PlanGetOutputSize")

    def set_workspace(self, workspace, nbytes):
        self.library._call("PlanSetWorkspace", self.native_handle, pointer(workspace), nbytes)
        self._workspace = workspace

    def execute(self, input, output):
        self.library._call("Execute", self._context, self.native_handle, pointer(input), pointer(output))

    def execute_steady(self, input, output):
        self.library._call("ExecuteSteady", self._context, self.native_handle, pointer(input), pointer(output))

    def physical_extents(self):
        """Executed extent of every axis, outermost first."""
        rank = len(json.loads(self.descriptor_json())["shape"])
        extents = (ct.c_size_t * rank)()
        self.library._call("PlanGetPhysicalExtents", self.native_handle, extents, rank)
        return list(extents)

    def selection_source(self):
        value = ct.c_int()
        self.library._call("PlanGetSelectionSource", self.native_handle, ct.byref(value))
        return SelectionSource(value.value)

    def mapping_json(self):
        return self.library._query("PlanGetMappingJson", self.native_handle)

    def descriptor_json(self):
        return self.library._query("PlanGetDescriptorJson", self.native_handle)

    def algorithm_name(self):
        return self.library._query("PlanGetAlgorithmName", self.native_handle)

    def selection_reason(self):
        return self.library._query("PlanGetSelectionReason", self.native_handle)

    def close(self):
        try:
            if self._handle.value:
                handle, self._handle = self._handle, ct.c_void_p()
                self.library._call("DestroyPlan", handle)
        finally:
            if self._context.value:
                context, self._context = self._context, ct.c_void_p()
                self.library._call("Destroy", context)
            self._workspace = None

    __enter__ = Descriptor.__enter__
    __exit__ = Descriptor.__exit__
    __del__ = Descriptor.__del__
