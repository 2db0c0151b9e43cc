"""ctypes binding of libcubutterfly, generated from the library's own headers.

The C headers under include/ are the single source of truth: at import, this
module reads every `typedef enum` (turned into an IntEnum named after the C
type, members without their shared prefix) and every exported function
declaration (turned into argtypes / restype), so the Python view of the ABI
cannot drift from the C one. Pointers of any kind travel as void*; the
caller passes ints, ctypes objects, byref() or anything with data_ptr().

Loading is explicit (`Native()`): the in-tree libcubutterfly.so, or the file
named by CUBUTTERFLY_LIBRARY. A missing library is an error; there is no
fallback implementation behind this binding.
"""
import ctypes as ct
import os
import re
from enum import IntEnum
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
INCLUDE = PACKAGE.parent / "include"
HEADERS = (INCLUDE / "cubutterfly" / "cubutterfly.h", INCLUDE / "cubutterfly" / "cubutterfly_mi355x.h",
           INCLUDE / "cuntt" / "rns_c_api.h")
LIBRARY = PACKAGE / "libcubutterfly.so"

_SCALARS = {"int": ct.c_int, "unsigned": ct.c_uint, "size_t": ct.c_size_t, "uint32_t": ct.c_uint32,
            "uint64_t": ct.c_uint64, "double": ct.c_double, "float": ct.c_float, "void": None}


def _strip_comments(text):
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def _enum_members(body):
    members, value = [], -1
    for item in filter(None, (part.strip() for part in body.split(","))):
        name, _, expr = item.partition("=")
        value = int(expr.strip(), 0) if expr.strip() else value + 1
        members.append((name.strip(), value))
    # Drop the underscore-separated prefix all members share (keep >= 1 token).
    split = [name.split("_") for name, _ in members]
    shared = 0
    while all(len(s) > shared + 1 for s in split) and len({s[shared] for s in split}) == 1:
        shared += 1
    return [("_".join(s[shared:]), v) for s, (_, v) in zip(split, members)]


def parse_headers(paths=HEADERS):
    """Returns (enums, handles, functions): enum name -> [(member, value)],
    the set of opaque pointer typedefs, and function name -> (return C type,
    [argument C types])."""
    text = "\n".join(_strip_comments(Path(p).read_text()) for p in paths)
    enums = {m.group(2): _enum_members(m.group(1))
             for m in re.finditer(r"typedef\s+enum\s+\w*\s*\{(.*?)\}\s*(\w+)\s*;", text, flags=re.S)}
    handles = set(re.findall(r"typedef\s+struct\s+\w+\s*\*\s*(\w+)\s*;", text))
    handles.update(re.findall(r"typedef\s+[\w\s]+\(\s*\*\s*(\w+)\s*\)", text))  # function pointers
    functions = {}
    for m in re.finditer(r"CUBUTTERFLY(?:_RNS_)?API\s+([\w\s\*]+?)\b(cubutterfly\w+)\s*\((.*?)\)\s*;", text, flags=re.S):
        args = [a.strip() for a in m.group(3).split(",")]
        args = [] if args == ["void"] else args
        # Drop each argument's name: the last identifier when a type precedes it.
        types = [re.sub(r"\b\w+\s*$", "", a).strip() if re.search(r"[\w\*]\s+\w+\s*$", a) else a for a in args]
        functions[m.group(2)] = (m.group(1).strip(), types)
    return enums, handles, functions


def _ctype(c_type, enums, handles, returning):
    bare = re.sub(r"\bconst\b", "", c_type).strip()
    if "*" in bare:
        if returning and re.fullmatch(r"char\s*\*", bare):
            return ct.c_char_p
        return ct.c_void_p
    if bare in enums:
        return ct.c_int
    if bare in handles or bare == "hipStream_t":
        return ct.c_void_p
    if bare not in _SCALARS:
        raise TypeError(f"header type {c_type!r} has no ctypes mapping")
    return _SCALARS[bare]


ENUMS, _HANDLES, FUNCTIONS = parse_headers()


def _enum_class(c_name):
    base = re.sub(r"_t$", "", c_name)
    base = base[len("cubutterfly"):] if base.startswith("cubutterfly") else base
    return IntEnum(base, ENUMS[c_name])


# One IntEnum per C enum, e.g. cubutterflyDataType_t -> DataType.FP32.
enums = {re.sub(r"^cubutterfly|_t$", "", name): _enum_class(name) for name in ENUMS}
Status = enums["Status"]


class AbiError(RuntimeError):
    """A cubutterfly* call returned a failure status. `status` is the C status
    value, `function` the entry point, `detail` the library's error text."""

    def __init__(self, function, status, detail, status_text=None):
        self.function, self.status, self.detail = function, int(status), detail
        label = status_text or str(int(status))
        super().__init__(f"{function} -> {label}" + (f": {detail}" if detail else ""))


class LibraryMissing(RuntimeError):
    pass


def device_address(value):
    """Raw address of a device buffer: an int, a ctypes pointer / c_void_p, or
    any object with data_ptr() (a torch tensor)."""
    if value is None:
        return None
    if hasattr(value, "data_ptr"):
        return value.data_ptr()
    if isinstance(value, ct.c_void_p):
        return value.value
    return value


class Native:
    """libcubutterfly with every header-declared function bound.

    `native("CreatePlan", ...)` calls cubutterflyCreatePlan and raises AbiError
    on a nonzero status (RNS entry points report 1 = invalid, 2 = runtime, with
    cubutterflyRnsLastError's text); `native.fn("CreatePlan")` is the bound
    ctypes function itself for tests of raw status codes.
    """

    def __init__(self, path=None):
        path = Path(path or os.environ.get("CUBUTTERFLY_LIBRARY") or LIBRARY)
        if not path.is_file():
            raise LibraryMissing(f"{path} does not exist: build it with `python -m cubutterfly_amd.build`")
        self.path = path
        self.dll = ct.CDLL(os.fspath(path))
        self._bound = {}
        for name, (ret, args) in FUNCTIONS.items():
            function = getattr(self.dll, name)
            function.restype = _ctype(ret, ENUMS, _HANDLES, True)
            function.argtypes = [_ctype(a, ENUMS, _HANDLES, False) for a in args]
            self._bound[name] = function

    @staticmethod
    def _full(name):
        return name if name.startswith("cubutterfly") else "cubutterfly" + name

    def fn(self, name):
        return self._bound[self._full(name)]

    def exported(self, name):
        return hasattr(self.dll, self._full(name))

    def __call__(self, name, *args):
        full = self._full(name)
        status = self._bound[full](*args)
        if status:
            if full.startswith("cubutterflyRns"):
                raise AbiError(full, status, self.rns_error(), {1: "invalid", 2: "runtime"}.get(status))
            raise AbiError(full, status, self.last_error(), self.status_text(status))

    def status_text(self, status):
        return self._bound["cubutterflyGetStatusString"](int(status)).decode()

    def last_error(self):
        return (self._bound["cubutterflyGetLastErrorString"]() or b"").decode(errors="replace")

    def rns_error(self):
        return (self._bound["cubutterflyRnsLastError"]() or b"").decode(errors="replace")

    def text(self, name, handle):
        """A string query of the (handle, buffer, size_t* bytes) form: size
        first, then the bytes."""
        size = ct.c_size_t(0)
        self(name, handle, None, ct.byref(size))
        out = ct.create_string_buffer(size.value)
        self(name, handle, out, ct.byref(size))
        return out.value.decode()

    def version(self):
        parts = (ct.c_int(), ct.c_int(), ct.c_int())
        self("GetVersion", *(ct.byref(p) for p in parts))
        return tuple(p.value for p in parts)
