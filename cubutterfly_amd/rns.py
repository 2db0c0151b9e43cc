"""Prepared multi-limb (RNS) word64 NTT plans, through include/cuntt/rns_c_api.h.

`request()` builds the plan request (the RNS JSON schema v1: log_n, direction,
ring, orders, domains {modulus, root}, polynomials {domain, input_offset,
output_offset}); `RnsPlan` creates, prepares and executes it. Every rule
(schema, primes, roots, overlap, placement, prepare-once, capture) is checked
by the library, whose status and text come back as `AbiError`.
"""
import ctypes as ct
import json

from .native import AbiError, device_address

# Cache policy of cubutterflyRnsPrepare by name.
CACHE_POLICIES = {"prefer": 0, "require": 1, "refresh": 2}


def request(log_n, domains, *, inverse=False, ring="negacyclic", input_order=None, output_order=None,
            polynomials=None):
    """`domains`: (modulus, forward root) pairs. Without `polynomials`, limb d
    is the dense row d (word offset d * 2^log_n on both sides). Orders default
    to natural -> bit-reversed forward and bit-reversed -> natural inverse."""
    n = 1 << log_n
    if polynomials is None:
        polynomials = [{"domain": d, "input_offset": d * n, "output_offset": d * n} for d in range(len(domains))]
    forward_orders = ("natural", "bit_reversed")
    default_in, default_out = forward_orders[::-1] if inverse else forward_orders
    return {"schema_version": 1, "log_n": log_n, "inverse": bool(inverse), "ring": ring,
            "input_order": input_order or default_in, "output_order": output_order or default_out,
            "domains": [{"modulus": int(q), "root": int(r)} for q, r in domains],
            "polynomials": polynomials}


class RnsPlan:
    def __init__(self, native, req):
        self.native, self.handle = native, ct.c_void_p()
        text = req if isinstance(req, str) else json.dumps(req)
        native("RnsCreate", text.encode(), ct.byref(self.handle))

    def prepare(self, stream=None, *, in_place=False, cache_dir=None, cache="prefer", repetitions=5):
        """Time and fix the lowering for one placement; once per plan, outside
        graph capture. `cache` is prefer / require / refresh of the record in
        `cache_dir`."""
        if cache not in CACHE_POLICIES:
            raise ValueError(f"cache must be one of {sorted(CACHE_POLICIES)}")
        directory = b"" if cache_dir is None else str(cache_dir).encode()
        self.native("RnsPrepare", self.handle, int(bool(in_place)), directory, CACHE_POLICIES[cache],
                    int(repetitions), device_address(stream))
        return self

    def execute(self, x, y, stream=None):
        self.native("RnsExecute", self.handle, device_address(x), device_address(y), device_address(stream))

    def info(self):
        return json.loads(self.native.text("RnsInfoJson", self.handle))

    def close(self):
        if self.handle.value:
            handle, self.handle = self.handle, ct.c_void_p()
            self.native("RnsDestroy", handle)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


__all__ = ["AbiError", "CACHE_POLICIES", "RnsPlan", "request"]
