"""RNS C ABI checks that need no GPU: strict config parsing and validation
(reference src/rns_tuning.cpp:124-150, src/rns_ntt.cu:259-300) reject bad
requests with status 1 before any device work."""
import json

import pytest

import cubutterfly_amd as cb
from cubutterfly_amd import rns, workloads
import oracle

Q = 1152921504606584833


def good(log_n=12):
    psi = oracle.find_primitive_root(log_n + 1, Q)
    return rns.request(log_n, [(Q, psi)])


@pytest.fixture(scope="module")
def lib():
    return cb.Native()


def rejected(lib, cfg):
    with pytest.raises(cb.AbiError) as info:
        rns.RnsPlan(lib, cfg)
    assert info.value.status == 1, str(info.value)
    return str(info.value)


def test_unknown_fields_are_rejected(lib):
    cfg = good()
    cfg["extra"] = 1
    assert "does not define: extra" in rejected(lib, cfg)
    cfg = good()
    cfg["domains"][0]["bogus"] = 3
    assert "does not define: bogus" in rejected(lib, cfg)


def test_schema_and_enums(lib):
    cfg = good()
    cfg["schema_version"] = 2
    assert "schema_version" in rejected(lib, cfg)
    cfg = good()
    cfg["ring"] = "twisted"
    assert "ring must be" in rejected(lib, cfg)
    cfg = good()
    cfg["output_order"] = "reversed"
    rejected(lib, cfg)
    cfg = good()
    cfg["log_n"] = -1
    rejected(lib, cfg)
    import ctypes as ct
    handle = ct.c_void_p()
    with pytest.raises(cb.AbiError) as info:  # truncated JSON straight to the native parser
        lib("RnsCreate", b'{"schema_version": 1, "log_n": 12', ct.byref(handle))
    assert info.value.status == 1 and not handle.value


def test_domain_validation(lib):
    for log_n in (11, 21):
        rejected(lib, rns.request(log_n, [(Q, 3)]))
    rejected(lib, rns.request(12, [(Q + 2, 3)]))            # not prime
    rejected(lib, rns.request(12, [(Q, 1)]))                # root of order 1
    w = oracle.find_primitive_root(12, Q)
    rejected(lib, rns.request(12, [(Q, w)]))                # order n: a cyclic root for a negacyclic ring
    rejected(lib, rns.request(12, [(Q, 0)]))
    cfg = good()
    cfg["polynomials"][0]["domain"] = 1
    rejected(lib, cfg)


def test_overlapping_outputs(lib):
    cfg = good()
    n = 1 << 12
    cfg["polynomials"] = [{"domain": 0, "input_offset": 0, "output_offset": 0},
                          {"domain": 0, "input_offset": n, "output_offset": n - 1}]
    assert "overlapping" in rejected(lib, cfg)


def test_moduli_generator_matches_survey():
    q = workloads.c4_moduli()
    assert len(q) == 32 and q[0] == Q and q[-1] == 1152921504538951681
    assert all((v - 1) % (1 << 17) == 0 and v < 1 << 60 for v in q)


@pytest.mark.parametrize("q", [1152921504606584833, 1073479681, 576460756061519873, 998244353])
def test_root_helpers_follow_the_reference_rule(q):
    from cubutterfly_amd import ntt_roots
    for log_n in (4, 12, 16):
        if (q - 1) % (2 << log_n):
            continue
        w = ntt_roots.primitive_root(log_n, q)
        assert w == oracle.find_primitive_root(log_n, q)
        assert ntt_roots.psi_for_root(log_n, q, w) == oracle.find_psi(log_n, q, w)
