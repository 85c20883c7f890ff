"""GPU parity of MemVanta's native block formats (src/quant.cpp,
src/quant_kernels.cpp) through the C ABI: the quantizers byte for byte,
matvec_q4_q8 / matmul_q4_0_batch / matvec_q4_0 / matvec_q8_0 bit for bit
against the compiled reference's golden vectors and against the oracle at the
7B decode shapes (every one of them is an in-order fp32 chain the kernels
reproduce exactly)."""
import importlib.util
import os

import numpy as np
import pytest

from conftest import ROOT, assert_bitexact, golden
from memvanta_amd import capi, synth

pytestmark = pytest.mark.gpu

_spec = importlib.util.spec_from_file_location("make_golden", os.path.join(ROOT, "tests", "golden", "make_golden.py"))
mg = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(mg)

NQ4, NQ8 = capi.MVH_TYPE_NATIVE_Q4_0, capi.MVH_TYPE_NATIVE_Q8_0
SHAPES_7B = [(4096, 4096), (4096, 11008), (11008, 4096), (4096, 32000)]  # (K, N)


def _upload(ctx, blocks, ty, rows, cols, name="native"):
    return ctx.upload(name, ty, cols, rows, np.ascontiguousarray(blocks, np.uint8).reshape(-1))


def test_quantizers_golden(ctx):
    """quantize_q8_0 / quantize_q4_0: round half to even, zero blocks (d = 0,
    zero bytes), a scale whose reciprocal overflows (the low clamp)."""
    g = golden("native.npz")
    assert np.array_equal(ctx.quantize_native(g["probe_x"], 36), g["probe_q8"])
    assert np.array_equal(ctx.quantize_native(g["probe_x"], 20), g["probe_q4"])


@pytest.mark.parametrize("n", [32, 4096, 11008, 1 << 20])
def test_quantizers_vs_numpy(ctx, n):
    rng = np.random.default_rng(n)
    x = synth.activations(rng, 1, n)[0] * np.float32(3)
    x[:32] = 0.0
    if n > 64:
        x[32:64] = np.float32(1e-38)
    assert np.array_equal(ctx.quantize_native(x, 36).reshape(-1), synth.quantize_q8_0_native(x).reshape(-1))
    assert np.array_equal(ctx.quantize_native(x, 20).reshape(-1), synth.quantize_q4_0_native(x).reshape(-1))


def test_golden_vectors(ctx):
    g = golden("native.npz")
    for i, (rows, cols, B) in enumerate(mg.NATIVE_MATS):
        key = f"r{rows}_c{cols}"
        W = mg.native_weights(i, rows, cols)
        A4, A8 = synth.quantize_q4_0_native(W), synth.quantize_q8_0_native(W)
        t4, t8 = _upload(ctx, A4, NQ4, rows, cols), _upload(ctx, A8, NQ8, rows, cols)
        assert np.array_equal(ctx.quantize_native(g[f"{key}__x"], 36), g[f"{key}__xq"])
        assert_bitexact(ctx.matvec_q4_q8(t4, g[f"{key}__xq"]), g[f"{key}__q4q8"], f"{key} matvec_q4_q8")
        assert_bitexact(ctx.matmul_q4_0_batch(t4, g[f"{key}__X"]), g[f"{key}__batch"], f"{key} matmul_q4_0_batch")
        assert_bitexact(ctx.matvec_native(t4, g[f"{key}__x"]), g[f"{key}__mv_q4_0"], f"{key} matvec_q4_0")
        assert_bitexact(ctx.matvec_native(t8, g[f"{key}__x"]), g[f"{key}__mv_q8_0"], f"{key} matvec_q8_0")
        t4.free()
        t8.free()


@pytest.mark.parametrize("k,n", SHAPES_7B + [(288, 768), (800, 300), (5632, 2048), (16384, 9), (256, 3)])
def test_matvec_q4_q8_vs_oracle(ctx, oracle, k, n):
    """matvec_q4_q8 at the decode GEMV config's shapes (persistent kernel) and
    at K % 256 != 0 (one wave per row)."""
    rng = np.random.default_rng(k * 3 + n)
    A = synth.quantize_q4_0_native(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    t = _upload(ctx, A, NQ4, n, k)
    x = synth.activations(rng, 1, k)[0]
    xq = ctx.quantize_native(x, 36)
    assert np.array_equal(xq, synth.quantize_q8_0_native(x))
    assert_bitexact(ctx.matvec_q4_q8(t, xq), oracle.nq_matvec_q4_q8(A, xq, n, k), f"matvec_q4_q8 {k}->{n}")
    t.free()


@pytest.mark.parametrize("k,n,b", [(4096, 4096, 1), (4096, 256, 3), (4096, 512, 32), (11008, 64, 5), (288, 100, 7),
                                   (2048, 96, 2)])
def test_matmul_q4_0_batch_vs_oracle(ctx, oracle, k, n, b):
    rng = np.random.default_rng(k + 17 * n + b)
    A = synth.quantize_q4_0_native(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    t = _upload(ctx, A, NQ4, n, k)
    X = synth.activations(rng, b, k)
    assert_bitexact(ctx.matmul_q4_0_batch(t, X), oracle.nq_matmul_q4_0_batch(A, X, n, k), f"batch {k}->{n} x{b}")
    t.free()


@pytest.mark.parametrize("k,n", [(4096, 4096), (11008, 64), (288, 33), (8192, 40)])
def test_matvec_q4_0_q8_0_vs_oracle(ctx, oracle, k, n):
    rng = np.random.default_rng(k + n)
    W = rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)
    x = synth.activations(rng, 1, k)[0]
    for bs, ty in ((20, NQ4), (36, NQ8)):
        A = synth.quantize_q4_0_native(W) if bs == 20 else synth.quantize_q8_0_native(W)
        t = _upload(ctx, A, ty, n, k)
        assert_bitexact(ctx.matvec_native(t, x), oracle.nq_matvec(A, x, n, k, bs), f"matvec {bs} {k}->{n}")
        t.free()


def test_device_pointers(ctx, oracle):
    """MVH_DEVICE: quantize into device blocks, then matvec_q4_q8 from them."""
    import torch

    k, n = 4096, 1000
    rng = np.random.default_rng(2)
    A = synth.quantize_q4_0_native(rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    t = _upload(ctx, A, NQ4, n, k)
    x = synth.activations(rng, 1, k)[0]
    xd = torch.from_numpy(x).to("cuda:0")
    qd = torch.empty((k // 32, 36), dtype=torch.uint8, device="cuda:0")
    yd = torch.empty(n, dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    ctx.quantize_native(xd, 36, out=qd)
    ctx.matvec_q4_q8(t, qd, y=yd)
    ctx.synchronize()
    assert np.array_equal(qd.cpu().numpy(), synth.quantize_q8_0_native(x))
    assert_bitexact(yd.cpu().numpy(), oracle.nq_matvec_q4_q8(A, synth.quantize_q8_0_native(x), n, k))
    t.free()


def test_errors(ctx):
    # 2 rows of 48 columns: 96 elements are 3 whole blocks, but a row is not
    t = ctx.upload("odd", NQ4, 48, 2, np.zeros(60, np.uint8))
    with pytest.raises(capi.MvhError, match="q4_q8 cols must be multiple of 32"):
        ctx.matvec_q4_q8(t, np.zeros(36, np.uint8))
    with pytest.raises(capi.MvhError, match="q4_0 cols must be multiple of 32"):
        ctx.matmul_q4_0_batch(t, np.zeros((1, 48), np.float32))
    t.free()
    with pytest.raises(capi.MvhError, match="q8_0 length must be multiple of 32"):
        ctx.quantize_native(np.zeros(48, np.float32), 36)
    with pytest.raises(capi.MvhError, match="q4_0 length must be multiple of 32"):
        ctx.quantize_native(np.zeros(40, np.float32), 20)
    g = ctx.upload("blk.0.attn_q.weight", synth.Q4_0, 64, 2, np.zeros(72, np.uint8))
    with pytest.raises(capi.MvhError, match="needs a native Q4_0 tensor"):
        ctx.matvec_q4_q8(g, np.zeros(72, np.uint8))
    g.free()
    t8 = ctx.upload("n8", NQ8, 64, 1, np.zeros(72, np.uint8))
    with pytest.raises(capi.MvhError, match="unsupported matvec tensor type native Q8_0"):
        ctx.matvec(t8, np.zeros(64, np.float32))
    t8.free()
