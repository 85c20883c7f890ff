"""The reference-side shim of the integration guide, compiled as printed there.

CPU: the shim text is extracted from the integration guide, compiled against the
reference checkout's own headers (include/memvanta/gguf_kernels.hpp) with
compile-time checks that each shim function has the signature of the
reference function it replaces, and linked with libmemvanta_hip.so and the
reference compiled from its sources (every symbol resolved).  Skipped where
the reference checkout or the libraries are absent.

GPU: oracle/_ref/shim_check (built by __graft_entry__.build() where the
reference checkout exists) opens a GGUF with the reference's GgufFile and runs
every tensor through the reference's CPU functions and through the shim, and
the profiler through both; results must agree as the parity tests require.
"""
import json
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT
from memvanta_amd import synth

REF_INCLUDE = "/root/reference/include/memvanta/gguf_kernels.hpp"
MVREF = os.path.join(ROOT, "oracle", "_ref", "libmvref.so")
HIPLIB = os.path.join(ROOT, "memvanta_amd", "libmemvanta_hip.so")
SHIM_CHECK = os.path.join(ROOT, "oracle", "_ref", "shim_check")


def test_shim_text_matches_reference_signatures_and_links(tmp_path):
    if not os.path.exists(REF_INCLUDE):
        pytest.skip("reference checkout absent")
    if not (os.path.exists(MVREF) and os.path.exists(HIPLIB)):
        pytest.skip("libmvref.so / libmemvanta_hip.so not built")
    from oracle import shim_build

    shim = shim_build.extract_shim()
    for fn in ("tensor_read_row_f32", "tensor_matvec", "tensor_matmul_batch", "tensor_matmul_batch_v06",
               "kernel_profile_snapshot"):
        assert f" {fn}(" in shim
    exe = shim_build.build(out_dir=str(tmp_path))
    assert os.path.exists(exe)
    syms = subprocess.run(["nm", "-DC", "--undefined-only", exe], capture_output=True, text=True, check=True).stdout
    for sym in ("mvh_matvec", "mvh_matmul_batch_v06", "mvh_read_row_f32", "mvh_tensor_upload",
                "mvh_profile_snapshot", "memvanta::GgufFile::tensor_data"):
        assert sym in syms, f"{sym} not bound by the shim"


# (name, type, K, N): every type of the tensor_matvec dispatch, K with and
# without a multiple of 256 (the row-group GEMV and the fallbacks), an
# embedding-like table for read_row
SHIM_TENSORS = [("blk.0.attn_q.weight", synth.Q4_0, 4096, 96), ("blk.1.ffn_up.weight", synth.Q8_0, 1024, 80),
                ("blk.2.ffn_down.weight", synth.Q6_K, 2048, 64), ("token_embd.weight", synth.Q4_0, 288, 50),
                ("blk.3.attn_output.weight", synth.F32, 300, 40), ("output.weight", synth.F16, 256, 33)]
NEAR_EXACT = {synth.Q6_K, synth.F16}  # double sums added as trees: within 2 ulp


@pytest.mark.gpu
def test_shim_check_reference_vs_hip(tmp_path):
    if not os.path.exists(SHIM_CHECK):
        pytest.skip("oracle/_ref/shim_check not built (needs the reference checkout at build time)")
    rng = np.random.default_rng(2718)
    path = str(tmp_path / "shim.gguf")
    w = synth.GgufWriter()
    w.add_str("general.architecture", "matrices")
    for name, ty, k, n in SHIM_TENSORS:
        x = rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)
        data = synth.quantize(ty, x) if ty not in (synth.F32, synth.F16) else (
            x.astype(np.float16).view(np.uint8) if ty == synth.F16 else x.view(np.uint8))
        data = np.ascontiguousarray(data)
        w.add_tensor(name, (k, n), ty, data.nbytes, lambda d=data: iter([d.tobytes()]))
    w.write(path)
    print(f"shim_check on {path}", flush=True)
    p = subprocess.run([SHIM_CHECK, path, *[t[0] for t in SHIM_TENSORS]], capture_output=True, text=True,
                       timeout=120)
    assert p.returncode == 0, p.stderr
    lines = [json.loads(line) for line in p.stdout.splitlines() if line.startswith("{")]
    types = {t[0]: t[1] for t in SHIM_TENSORS}
    seen = set()
    for r in lines:
        if r["op"] == "profile":
            continue
        seen.add((r["tensor"], r["op"]))
        if "reference_error" in r:
            assert r["reference_error"] and r["reference_error"] == r["hip_error"], r
            continue
        if types[r["tensor"]] in NEAR_EXACT:
            assert r["max_ulp"] <= 2, r
        else:
            assert r["mismatch"] == 0, r
    assert len(seen) == 6 * len(SHIM_TENSORS)
    wrong = [r for r in lines if r["op"] == "read_row_wrong_cols"]
    assert all(r["reference_error"] == f"tensor row shape mismatch: {r['tensor']}" for r in wrong)
    prof = {side: [(r["tensor"], r["layer"], r["kind"], r["calls"], r["batch"]) for r in lines
                   if r["op"] == "profile" and r["side"] == side] for side in ("hip", "reference")}
    assert prof["hip"] == prof["reference"] and len(prof["hip"]) == len(SHIM_TENSORS)
