"""CPU checks of the product library: it loads, exports every symbol include/rabbit_amd.h declares,
and the calls that need no GPU behave (status codes, host-side helpers)."""
import ctypes as C

import numpy as np


def test_library_exports_every_declared_symbol(rbt_lib):
    from rabbit_amd import abi
    declared = abi.header_symbols()
    assert len(declared) >= 30
    missing = [s for s in declared if not hasattr(rbt_lib, s)]
    assert not missing, missing
    assert set(declared) == set(abi.SIGNATURES), "ctypes signatures out of sync with the header"


def test_version_names_the_target(rbt_lib):
    assert b"gfx950" in rbt_lib.rbt_version()


def test_null_context_is_an_error_not_a_crash(rbt_lib):
    assert rbt_lib.rbt_sync(None) == -1
    assert rbt_lib.rbt_matmul(None, None, None, None, 1, 1, 1) == -1
    assert rbt_lib.rbt_pool_get(None, 0, 0) is None or not rbt_lib.rbt_pool_get(None, 0, 0)
    out = C.c_void_p()
    assert rbt_lib.rbt_init(None, 0) == -1


def test_unique_experts_host_helper(rbt_lib):
    ids = np.array([[5, 2, 9], [2, 7, 5], [1, 9, 3]], np.int32)
    out = np.zeros(9, np.int32)
    n = rbt_lib.rbt_unique_experts(ids.ctypes.data, 3, 3, out.ctypes.data)
    assert list(out[:n]) == [5, 2, 9, 7, 1, 3]  # glm52/moe.rs:333-344


def test_qt_resident_bytes(rbt_lib):
    from rabbit_amd.abi import RbtQT
    q = RbtQT(10, 100, 2, None, None, 0)
    assert rbt_lib.rbt_qt_resident_bytes(C.byref(q)) == 10 * 50 + 10 * 4
    q = RbtQT(10, 100, 1, None, None, 25)
    assert rbt_lib.rbt_qt_resident_bytes(C.byref(q)) == 10 * 50 + 10 * 4 * 4
    q = RbtQT(10, 100, 0, None, None, 0)
    assert rbt_lib.rbt_qt_resident_bytes(C.byref(q)) == 10 * 100 * 4
