"""Builds the reference-side integration check -- TEST INFRASTRUCTURE ONLY.

Extracts the shim that the integration guide prints (the ```cpp block headed
``// src/gguf_kernels_hip.cpp``) into _ref/gguf_kernels_hip.cpp, then compiles
shim_check.cpp, which includes it, against the reference checkout's headers
and links it with the reference compiled from its sources (_ref/libmvref.so,
oracle/Makefile) and libmemvanta_hip.so: _ref/shim_check.  Needs the
reference checkout (for its headers) and both libraries; the result, like
libmvref.so, is a git-ignored build product.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
REF = os.environ.get("MEMVANTA_REF", "/root/reference")
SHIM_TAG = "```cpp\n// src/gguf_kernels_hip.cpp"


def extract_shim(md_path: str = os.path.join(ROOT, "INTEGRATION.md")) -> str:
    text = open(md_path).read()
    start = text.index(SHIM_TAG) + len("```cpp\n")
    end = text.index("```", start)
    return text[start:end]


def build(ref: str = REF, out_dir: str = os.path.join(HERE, "_ref")) -> str:
    """Compile and link _ref/shim_check (or out_dir/shim_check); returns its path."""
    os.makedirs(out_dir, exist_ok=True)
    shim = os.path.join(out_dir, "gguf_kernels_hip.cpp")
    with open(shim, "w") as f:
        f.write(extract_shim())
    exe = os.path.join(out_dir, "shim_check")
    mvref = os.path.join(HERE, "_ref", "libmvref.so")
    hip = os.path.join(ROOT, "memvanta_amd", "libmemvanta_hip.so")
    for p in (mvref, hip):
        if not os.path.exists(p):
            raise FileNotFoundError(p)
    cmd = ["g++", "-std=c++20", "-O2", "-Wall", "-Wextra", "-Werror", "-fopenmp",
           f"-I{os.path.join(ref, 'include')}", f"-I{os.path.join(ROOT, 'include')}", f"-I{out_dir}",
           os.path.join(HERE, "shim_check.cpp"), "-o", exe, mvref, hip,
           "-Wl,-rpath,$ORIGIN", "-Wl,-rpath,$ORIGIN/../../memvanta_amd", "-Wl,--no-undefined", "-lpthread"]
    subprocess.run(cmd, check=True)
    return exe


if __name__ == "__main__":
    print(build(*(sys.argv[1:2] or [REF])))
