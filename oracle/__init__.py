"""ctypes wrapper over the CPU oracle (oracle/liboracle.so) -- TEST INFRASTRUCTURE ONLY.

The oracle restates cuButterfly's CPU reference algorithms (see oracle.h for the
file:line each follows). Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import this module; the product library never does.
"""
import ctypes as ct
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB = None


def library_path():
    return _HERE / "liboracle.so"


def build():
    """Compile liboracle.so with the committed Makefile (gcc only)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", str(_HERE), "-B", "liboracle.so"], check=True)


def _lib():
    global _LIB
    if _LIB is None:
        path = library_path()
        if not path.exists():
            raise RuntimeError(f"oracle library {path} is not built; run make -C oracle")
        lib = ct.CDLL(str(path))
        u64, u32, i, f = ct.c_uint64, ct.c_uint32, ct.c_int, ct.c_float
        p = ct.c_void_p
        sig = {
            "cbo_fwht_f32": (i, [p, u64, i, i]),
            "cbo_fwht_f32_batch": (i, [p, u64, u64, i, i, i]),
            "cbo_f32_to_f16_rne": (ct.c_uint16, [f]),
            "cbo_f16_to_f32": (f, [ct.c_uint16]),
            "cbo_fwht_f16_final_batch": (i, [p, p, u64, u64, f, i, i, i]),
            "cbo_fft_c64": (i, [p, u64, i, i]),
            "cbo_fft_c64_batch": (i, [p, u64, u64, i, i, i]),
            "cbo_mod_mul": (u64, [u64, u64, u64]),
            "cbo_mod_pow": (u64, [u64, u64, u64]),
            "cbo_is_prime": (i, [u64]),
            "cbo_find_primitive_root": (u64, [u32, u64]),
            "cbo_find_psi": (u64, [u32, u64, u64]),
            "cbo_ntt_cyclic": (i, [p, u64, u64, i]),
            "cbo_ntt_cyclic_batch": (i, [p, u64, u64, u64, i, i]),
            "cbo_ntt_negacyclic_batch": (i, [p, p, u64, u64, u64, i, i]),
            "cbo_rns_reference": (i, [p, p, u32, u64, u64, i, i, i, i]),
            "cbo_rns_batch": (i, [p, p, u32, p, p, u64, i, i, i, i, i]),
        }
        for name, (restype, argtypes) in sig.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = restype, argtypes
        _LIB = lib
    return _LIB


def default_threads():
    return max(1, min(16, os.cpu_count() or 1))


def _ptr(array):
    return array.ctypes.data_as(ct.c_void_p)


def _check(status, what):
    if status != 0:
        raise ValueError(f"oracle {what} rejected its arguments (status {status})")


def fwht_f32(x, inverse=False, normalize=False, threads=1):
    """Row-wise FWHT of a float32 array [..., n] (reference_fwht<float>)."""
    a = np.array(x, dtype=np.float32, copy=True, order="C")
    n = a.shape[-1]
    _check(_lib().cbo_fwht_f32_batch(_ptr(a), n, a.size // n, int(inverse), int(normalize), threads),
           "fwht_f32")
    return a


def f32_to_f16_bits(x):
    lib = _lib()
    flat = np.asarray(x, dtype=np.float32).ravel()
    return np.array([lib.cbo_f32_to_f16_rne(float(v)) for v in flat], dtype=np.uint16)


def fwht_f16_final(x_f16, scale, inverse=False, normalize=False, threads=1):
    """FP16 storage, FP32 compute, single RNE narrowing after x (float)scale."""
    a = np.ascontiguousarray(x_f16, dtype=np.float16)
    n = a.shape[-1]
    out = np.empty_like(a)
    _check(_lib().cbo_fwht_f16_final_batch(_ptr(a.view(np.uint16)), _ptr(out.view(np.uint16)), n,
                                            a.size // n, float(np.float32(scale)), int(inverse),
                                            int(normalize), threads), "fwht_f16_final")
    return out


def fft_c64(x, inverse=False, normalize=False, threads=1):
    """Row-wise complex64 FFT [..., n] (reference_fft(std::vector<Complex32>&))."""
    a = np.array(x, dtype=np.complex64, copy=True, order="C")
    n = a.shape[-1]
    _check(_lib().cbo_fft_c64_batch(_ptr(a), n, a.size // n, int(inverse), int(normalize), threads),
           "fft_c64")
    return a


def mod_pow(b, e, q):
    return int(_lib().cbo_mod_pow(b, e, q))


def is_prime(q):
    return bool(_lib().cbo_is_prime(q))


def find_primitive_root(log_n, q):
    return int(_lib().cbo_find_primitive_root(log_n, q))


def find_psi(log_n, q, root):
    return int(_lib().cbo_find_psi(log_n, q, root))


def ntt_cyclic(x, q, inverse=False, threads=1):
    a = np.array(x, dtype=np.uint64, copy=True, order="C")
    n = a.shape[-1]
    _check(_lib().cbo_ntt_cyclic_batch(_ptr(a), n, a.size // n, q, int(inverse), threads), "ntt_cyclic")
    return a


def ntt_negacyclic(x, q, inverse=False, threads=1):
    a = np.ascontiguousarray(x, dtype=np.uint64)
    n = a.shape[-1]
    out = np.empty_like(a)
    _check(_lib().cbo_ntt_negacyclic_batch(_ptr(a), _ptr(out), n, a.size // n, q, int(inverse), threads),
           "ntt_negacyclic")
    return out


def rns(x, moduli, roots, negacyclic=True, inverse=False, input_bit_reversed=False,
        output_bit_reversed=False, threads=1):
    """x: uint64 [count, n]; polynomial p uses (moduli[p], roots[p])."""
    a = np.ascontiguousarray(x, dtype=np.uint64)
    count, n = a.shape
    log_n = n.bit_length() - 1
    q = np.ascontiguousarray(moduli, dtype=np.uint64)
    r = np.ascontiguousarray(roots, dtype=np.uint64)
    assert q.size == count and r.size == count
    out = np.empty_like(a)
    _check(_lib().cbo_rns_batch(_ptr(a), _ptr(out), log_n, _ptr(q), _ptr(r), count, int(negacyclic),
                                int(inverse), int(input_bit_reversed), int(output_bit_reversed), threads),
           "rns")
    return out
