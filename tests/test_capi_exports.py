"""The C-ABI library loads on a host without a GPU and exports every symbol
include/memvanta_hip.h declares (no compute calls here)."""
import ctypes

import pytest

from conftest import golden
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


def test_kv_type_names_match_reference():
    """parse_kv_cache_type / kv_cache_type_name (src/llama_model.cpp:16-17)
    against the compiled reference's answers; host-only calls."""
    g = golden("kv_types.npz")
    assert [capi.kv_type_name(t) for t in range(3)] == g["names"].tolist()
    assert capi.kv_type_name(7) == "?"
    assert [capi.kv_parse_type(s) for s in ("f32", "f16", "q8", "q8_0")] == g["parsed"].tolist()
    with pytest.raises(capi.MvhError, match="unknown KV cache type: bf16"):
        capi.kv_parse_type("bf16")


def test_profile_kind_names_match_reference():
    """kernel_profile_kind_name (src/gguf_kernels.cpp:222) for every kind and
    out-of-range values, against the compiled reference's strings; the
    registry's enable / reset / snapshot run without a device."""
    g = golden("profile.npz")
    assert [capi.profile_kind_name(int(k)) for k in g["kind_codes"]] == g["kind_names"].tolist()
    assert capi.PROFILE_KINDS == tuple(g["kind_names"][1:10].tolist())
    capi.profile_enable(False)
    capi.profile_reset()
    assert capi.profile_snapshot() == []


def test_header_compiles_as_c_and_links(tmp_path):
    """A plain C program (what a cgo / C++ shim sees) compiles against the
    header alone and links against the library; no call touches a device."""
    import os
    import subprocess

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    src = tmp_path / "use_abi.c"
    src.write_text(r'''
#include <stdio.h>
#include "memvanta_hip.h"
int main(void) {
    size_t bytes = 0;
    if (mvh_version() < 1) return 1;
    if (mvh_kv_bytes_allocated(NULL, &bytes) != MVH_E_INVALID) return 2;
    if (!mvh_last_error()[0]) return 3;
    int t = -1;
    if (mvh_kv_parse_type("q8_0", &t) != MVH_OK || t != MVH_KV_Q8) return 4;
    if (mvh_kv_type_name(MVH_KV_F32)[1] != '3') return 5;
    size_t n = 7;
    mvh_profile_reset();
    if (mvh_profile_snapshot(NULL, 0, &n) != MVH_OK || n != 0) return 6;
    if (mvh_profile_kind_name(MVH_PROF_FFN_DOWN)[4] != 'd') return 7;
    puts("ok");
    return 0;
}
''')
    exe = tmp_path / "use_abi"
    lib_dir = os.path.join(root, "memvanta_amd")
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.join(root, "include"), str(src), "-o", str(exe),
                    "-L", lib_dir, "-lmemvanta_hip", "-Wl,-rpath," + lib_dir], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    assert out.strip() == "ok"
