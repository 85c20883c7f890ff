"""The C-ABI library loads on a host without a GPU and exports every symbol
include/memvanta_hip.h declares (no compute calls here)."""
import ctypes

from memvanta_amd import capi


def test_library_exports_every_declared_symbol():
    lib = capi.load_library()
    names = capi.header_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_bindings_cover_the_header():
    assert set(capi.header_functions()) == set(capi._SIGS)


def test_version_and_error_channel():
    lib = capi.load_library()
    assert lib.mvh_version() >= 1
    assert lib.mvh_context_destroy(None) == 0
    # a null out-pointer is rejected with a message, no device needed
    assert lib.mvh_tensor_info(None, None, None, None, None, None) == 1
    assert b"null tensor" in lib.mvh_last_error()
    n = ctypes.c_size_t()
    assert lib.mvh_kv_bytes_allocated(None, ctypes.byref(n)) == 1
