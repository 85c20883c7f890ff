"""GPU parity: every kernel through the C ABI against the oracle on the same
seeded inputs.  Integer/byte results and the fp32 chains that reproduce the
reference's operation order are compared bit for bit; the two places that
add a double sum in a different order (Q6_K rows, the attention softmax
denominator) are compared within 2 ulp and must be bit-identical on at least
99.9% of the outputs."""
import importlib.util
import os

import numpy as np
import pytest

from conftest import ROOT, assert_bitexact, bits, golden
from memvanta_amd import capi, synth

_spec = importlib.util.spec_from_file_location("make_golden", os.path.join(ROOT, "tests", "golden", "make_golden.py"))
mg = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(mg)

pytestmark = pytest.mark.gpu

SHAPES_7B = [(4096, 4096), (4096, 11008), (11008, 4096), (4096, 32000)]  # (K, N)


def _w(rng, ty, rows, cols):
    return synth.quantize(ty, rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02))


def ulp_diff(a, b):
    a = bits(a).astype(np.int64)
    b = bits(b).astype(np.int64)
    a = np.where(a & 0x80000000, 0x80000000 - a, a)
    b = np.where(b & 0x80000000, 0x80000000 - b, b)
    return np.abs(a - b)


# ---------------------------------------------------------------- conversions

def test_fp16_to_fp32_all_65536(ctx, oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = ctx.fp16_to_fp32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(bits(got)[~nan], bits(want)[~nan])
    assert np.isnan(got[nan]).all()
    # the oracle's conversion agrees on a spread of patterns incl. subnormals
    probe = np.array([0, 1, 2, 0x3ff, 0x400, 0x3c00, 0x7bff, 0x7c00, 0x8001, 0xfbff], np.uint16)
    assert np.array_equal(bits(oracle.fp16_to_fp32(probe)), bits(ctx.fp16_to_fp32(probe)))


def test_fp32_to_fp16_reference_rounding(ctx, oracle):
    rng = np.random.default_rng(3)
    # 2^26 patterns strided over all 2^32, 2^24 random ones, and every
    # exponent with mantissas at the rounding/carry boundaries
    strided = (np.arange(1 << 26, dtype=np.uint64) * 64).astype(np.uint32)
    rand = rng.integers(0, 1 << 32, size=1 << 24, dtype=np.uint64).astype(np.uint32)
    e = np.arange(512, dtype=np.uint32) << 23
    m = np.concatenate([np.array([0, 1, 0xfff, 0x1000, 0x1001, 0x1fff, 0x2000, 0x7fefff, 0x7ff000, 0x7fffff], np.uint32),
                        rng.integers(0, 1 << 23, size=2000, dtype=np.uint64).astype(np.uint32)])
    edge = (e[:, None] | m[None, :]).ravel()
    pats = np.concatenate([strided, rand, edge])
    got = ctx.fp32_to_fp16(pats.view(np.float32))
    want = oracle.fp32_to_fp16(pats.view(np.float32))
    bad = np.flatnonzero(got != want)
    assert bad.size == 0, f"{bad.size} mismatches, first pattern 0x{pats[bad[0]]:08x}"
    # known answers of the non-RNE routine (ties away, OR-ed carry)
    kv = np.array([1.00048828125, 1.9999, 0.12499999, 65504.0, 70000.0, 1e-6, -1.9999], np.float32)
    assert list(ctx.fp32_to_fp16(kv)) == [0x3c01, 0x3c00, 0x2c00, 0x7bff, 0x7c00, 0x0011, 0xbc00]


# ---------------------------------------------------------------- quantizer

@pytest.mark.parametrize("m,k", [(1, 4096), (1, 11008), (32, 4096), (7, 288), (512, 2048)])
def test_quantize_q8_bitexact(ctx, oracle, m, k):
    rng = np.random.default_rng(m * 1000 + k)
    x = synth.activations(rng, m, k)
    x[0, :32] = 0.0                                   # all-zero block -> d = 1, q = 0
    x[0, 32:64] = np.float32(0.0)
    x[0, 40] = 127.0                                  # d = 1, inv = 1
    x[0, 41], x[0, 42], x[0, 43] = 2.5, -2.5, 126.5   # ties round away from zero
    if k > 96:
        x[0, 64:96] = np.float32(1e-30)               # tiny but non-zero block
    q, d = ctx.quantize_q8(x)
    q_ref, d_ref = oracle.quantize_q8(x)
    assert np.array_equal(q, q_ref)
    assert_bitexact(d, d_ref, "q8 scales")
    assert q[0, 41] == 3 and q[0, 42] == -3 and q[0, 43] == 127 and d[0, 0] == 1.0


def test_quantize_q8_overflow_edge(ctx, oracle):
    """Scales whose reciprocal overflows or that underflow to 0: the device
    converts the non-finite quotients as the reference's x86 lround does (-127),
    in the quantizer and in the GEMV that quantizes its own input."""
    g = golden("quant_edge.npz")
    x = g["x"]
    q, d = ctx.quantize_q8(x)
    q_ref, d_ref = oracle.quantize_q8(x)
    assert np.array_equal(q, q_ref)
    assert_bitexact(d, d_ref, "edge scales")
    w = np.ascontiguousarray(mg.probe_matrix(256))
    t = ctx.upload("probe", synth.Q4_0, 256, 256, w)
    for i in range(x.shape[0]):
        assert_bitexact(ctx.matvec(t, x[i]), g["y"][i], f"edge probe {i}")
    t.free()


# ---------------------------------------------------------------- decode GEMV

@pytest.mark.parametrize("k,n", SHAPES_7B + [(288, 768), (768, 288), (2048, 2048), (5632, 2048)])
def test_gemv_q4_0_bitexact(ctx, oracle, k, n):
    rng = np.random.default_rng(k + n)
    w = _w(rng, synth.Q4_0, n, k)
    t = ctx.upload("blk.0.attn_q.weight", synth.Q4_0, k, n, w)
    for rep in range(2):
        x = synth.activations(rng, 1, k)[0]
        assert_bitexact(ctx.matvec(t, x), oracle.matvec(w, synth.Q4_0, n, k, x), f"Q4_0 {k}->{n}")
    t.free()


# (K, N) over the row-group GEMV's pass shapes (passes of 16 units of 8
# blocks; K / 256 units per row): 4096 -> 1 whole pass; 11008 -> 3 passes, the
# last of 11 units; 5632 -> 2 passes (6 in the last); 2048 -> 1 pass of 8
# units; 8192 -> 2; 16384 -> 4; 256 -> a single unit; N not a multiple of the
# 4-row tile, N < 4, and grids larger than the resident wave count.
Q8_INPUT_SHAPES = [(4096, 4096), (11008, 4096), (5632, 2048), (2048, 1003), (16384, 37),
                   (8192, 4099), (256, 130), (4096, 3), (4096, 22016), (4096, 32000), (11008, 12288)]


@pytest.mark.parametrize("k,n", Q8_INPUT_SHAPES)
def test_gemv_q4_0_prequantized_bitexact(ctx, oracle, k, n):
    """The model's decode path: Q4_0 x an already quantized Q8 activation
    (mvh_matvec_q8), against the oracle's tensor_matvec on the fp32 input."""
    rng = np.random.default_rng(5 * k + n)
    w = _w(rng, synth.Q4_0, n, k)
    t = ctx.upload("blk.0.ffn_up.weight", synth.Q4_0, k, n, w)
    x = synth.activations(rng, 1, k)[0]
    q, d = oracle.quantize_q8(x)
    assert_bitexact(ctx.matvec_q8(t, q, d), oracle.matvec(w, synth.Q4_0, n, k, x), f"Q4_0 x Q8 {k}->{n}")
    t.free()


# one token at K = 2048 / 4096 runs the row-group kernel (16 rows per
# workgroup; ragged last workgroups at 37 and 1001 rows), other K the
# persistent or per-token kernels
@pytest.mark.parametrize("k,n", [(288, 32000), (2048, 2048), (2048, 256), (5632, 2048), (4096, 4096), (288, 768),
                                 (4096, 37), (256, 130), (8192, 33), (11008, 64), (16384, 5), (2048, 11264),
                                 (2048, 2560), (2048, 1001)])
def test_gemv_q8_0_bitexact(ctx, oracle, k, n):
    rng = np.random.default_rng(7 * k + n)
    w = _w(rng, synth.Q8_0, n, k)
    t = ctx.upload("output.weight", synth.Q8_0, k, n, w)
    x = synth.activations(rng, 1, k)[0]
    assert_bitexact(ctx.matvec(t, x), oracle.matvec(w, synth.Q8_0, n, k, x), f"Q8_0 {k}->{n}")
    t.free()


@pytest.mark.parametrize("k,n", [(4096, 37), (256, 130), (8192, 33), (11008, 64), (16384, 5), (2048, 2048),
                                 (1024, 96)])
def test_q4_0_f32act_one_token_bitexact(ctx, oracle, k, n):
    """dot_q4_0_fp32 for one token (tensor_matmul_batch with batch 1): the
    persistent fp32-activation GEMV for K % 256 == 0 up to K = 8192 (4-block
    units: 2 per row at K = 256, 64 at K = 8192; row counts that leave the
    last tile partial), the two-phase kernel beyond (K = 11008, 16384)."""
    rng = np.random.default_rng(11 * k + n)
    w = _w(rng, synth.Q4_0, n, k)
    t = ctx.upload("blk.0.attn_q.weight", synth.Q4_0, k, n, w)
    x = synth.activations(rng, 1, k)
    assert_bitexact(ctx.matmul_batch(t, x), oracle.matmul_batch(w, synth.Q4_0, n, k, x), f"Q4_0 f32act {k}->{n}")
    t.free()


# row counts that leave the last workgroup's waves partly or wholly idle, odd
# and even super-block counts per row; one and two rows per lane (two from
# 16384 rows at K <= 4096 and from 8192 rows beyond), with ragged last
# workgroups in both
@pytest.mark.parametrize("k,n", [(4096, 32000), (2048, 32000), (5632, 2048), (256, 64), (6144, 1000), (8192, 37),
                                 (11008, 64), (4096, 16390), (6144, 8203), (256, 16383)])
def test_gemv_q6_k(ctx, oracle, k, n):
    rng = np.random.default_rng(3 * k + n)
    w = _w(rng, synth.Q6_K, n, k)
    t = ctx.upload("output.weight", synth.Q6_K, k, n, w)
    x = synth.activations(rng, 1, k)[0]
    got = ctx.matvec(t, x)
    want = oracle.matvec(w, synth.Q6_K, n, k, x)
    u = ulp_diff(got, want)
    assert u.max() <= 2, u.max()
    assert (u == 0).mean() >= 0.999, (u == 0).mean()
    t.free()


@pytest.mark.parametrize("k,n", [(4096, 16400), (2048, 300), (5632, 300)])
def test_gemv_q6_k_nonfinite(ctx, oracle, k, n):
    """An infinite or NaN activation: the rows' double sums give inf, -inf or
    NaN (a zero weight times inf) exactly where the oracle's do, on both the
    one- and the two-rows-per-lane paths."""
    rng = np.random.default_rng(k + n)
    w = _w(rng, synth.Q6_K, n, k)
    t = ctx.upload("output.weight", synth.Q6_K, k, n, w)
    for bad in (np.inf, -np.inf, np.nan):
        x = synth.activations(rng, 1, k)[0]
        x[k // 3] = bad
        got = ctx.matvec(t, x)
        want = oracle.matvec(w, synth.Q6_K, n, k, x)
        assert np.array_equal(np.isnan(got), np.isnan(want))
        fin = ~np.isnan(want)
        assert np.array_equal(got[fin], want[fin])
    t.free()


@pytest.mark.parametrize("k,n,batch", [(5632, 2048, 32), (2048, 300, 37), (11008, 17, 16), (256, 64, 20),
                                       (6144, 1, 48)])
def test_q6_k_token_groups(ctx, oracle, k, n, batch):
    """tensor_matmul_batch of Q6_K weights (dot_q6_k_fp32 per token) with whole
    16-token groups on the batch kernel and the rest per token: the
    TinyLlama-1.1B ffn_down shape, rows off the 16-row tile down to one row,
    odd super-block counts, one super-block per row; every token within 2 ulp
    of the oracle, nearly all bit-identical."""
    rng = np.random.default_rng(5 * k + n + batch)
    w = _w(rng, synth.Q6_K, n, k)
    t = ctx.upload("blk.0.ffn_down.weight", synth.Q6_K, k, n, w)
    x = synth.activations(rng, batch, k)
    got = ctx.matmul_batch(t, x)
    want = oracle.matmul_batch(w, synth.Q6_K, n, k, x, threads=16)
    u = ulp_diff(got, want)
    assert u.max() <= 2, u.max()
    assert (u == 0).mean() >= 0.999, (u == 0).mean()
    assert_bitexact(ctx.matmul_batch_v06(t, x, capi.MVH_ACT_Q8), got, "v06 of Q6_K is the same per-token dot")
    t.free()


def test_matvec_errors_match_reference_text(ctx):
    w = np.zeros(210, np.uint8)
    t = ctx.upload("blk.3.ffn_down.weight", synth.Q6_K, 128, 2, w)
    with pytest.raises(capi.MvhError, match="Q6_K matrix row not block aligned: blk.3.ffn_down.weight"):
        ctx.matvec(t, np.zeros(128, np.float32))
    with pytest.raises(capi.MvhError, match="does not match"):
        ctx.upload("bad", synth.Q4_0, 64, 2, np.zeros(10, np.uint8))


# ---------------------------------------------------------------- batched prefill

@pytest.mark.parametrize("ty", [synth.Q4_0, synth.Q8_0])
@pytest.mark.parametrize("name", ["blk.0.attn_q.weight", "blk.0.ffn_up.weight"])
@pytest.mark.parametrize("batch", [2, 5, 11, 32])
def test_matmul_v06_ref_mode_bitexact(ctx, oracle, ty, name, batch):
    rng = np.random.default_rng(batch * 31 + ty)
    k, n = 1024, 96
    w = _w(rng, ty, n, k)
    t = ctx.upload(name, ty, k, n, w)
    x = synth.activations(rng, batch, k)
    got = ctx.matmul_batch_v06(t, x, capi.MVH_ACT_REF)
    want = oracle.matmul_batch_v06(w, ty, n, k, x, is_ffn="ffn" in name, force_q8=False)
    assert_bitexact(got, want, f"v06 ref {name} B={batch}")
    t.free()


@pytest.mark.parametrize("ty", [synth.Q4_0, synth.Q8_0])
@pytest.mark.parametrize("name,batch,k,n", [("blk.0.attn_q.weight", 32, 4096, 300), ("blk.0.attn_q.weight", 12, 4096, 33),
                                            ("blk.0.ffn_up.weight", 24, 11008, 40), ("blk.0.attn_q.weight", 27, 768, 64),
                                            ("blk.0.ffn_up.weight", 8, 2048, 1), ("blk.0.ffn_up.weight", 40, 4096, 7),
                                            ("blk.0.attn_q.weight", 16, 256, 45)])
def test_matmul_v06_ref_mode_lanes_bitexact(ctx, oracle, ty, name, batch, k, n):
    """Default prefill numerics (batch4 / batch8 accumulators) at 7B-scale K:
    for Q4_0 whole 16-token groups run two rows per lane, then whole 8-token
    groups on the lane-spread kernel, the rest of the blocked tokens per
    token, the unblocked tail with dot_*_fp32; row counts off the 32-row tile
    (down to a single partial tile), a one-unit row (K = 256)."""
    rng = np.random.default_rng(batch * 13 + k + n + ty)
    w = _w(rng, ty, n, k)
    t = ctx.upload(name, ty, k, n, w)
    x = synth.activations(rng, batch, k)
    got = ctx.matmul_batch_v06(t, x, capi.MVH_ACT_REF)
    want = oracle.matmul_batch_v06(w, ty, n, k, x, is_ffn="ffn" in name, force_q8=False)
    assert_bitexact(got, want, f"v06 ref {name} B={batch} K={k} N={n}")
    t.free()


def test_matmul_v06_ref_mode_special_scales(ctx, oracle):
    """Default prefill numerics on the two-row Q4_0 kernel with block scales
    that are +0, -0, f16 subnormals, negative, +-inf and NaN, and activations
    holding zeros, -0 and float denormals: bit-identical to the oracle (NaN
    exactly where it has NaN).  Rows 0..31 mix every special scale (the
    reference's subtract-and-multiply path), rows 32..63 only signed zeros,
    rows 64..95 only subnormal and negative scales (the fma path)."""
    rng = np.random.default_rng(77)
    k, n, batch = 2048, 96, 32
    nb = k // 32
    w = _w(rng, synth.Q4_0, n, k).reshape(n, nb, 18).copy()
    sets = [(range(0, 32), [0x0000, 0x8000, 0x0001, 0x83FF, 0x7C00, 0xFC00, 0x7E00, 0xBC00]),
            (range(32, 64), [0x0000, 0x8000]), (range(64, 96), [0x0001, 0x03FF, 0x8001, 0xC500, 0x8400])]
    for rows, vals in sets:
        for r in rows:
            for b in rng.choice(nb, size=6, replace=False):
                v = int(rng.choice(vals))
                w[r, b, 0], w[r, b, 1] = v & 0xFF, v >> 8
    w = w.reshape(-1)
    t = ctx.upload("blk.0.attn_q.weight", synth.Q4_0, k, n, w)
    x = synth.activations(rng, batch, k)
    x[:, ::97] = 0.0
    x[:, 5::101] = -0.0
    x[:, 7::89] = np.float32(1e-40) * np.sign(x[:, 7::89] + np.float32(0.5))
    got = ctx.matmul_batch_v06(t, x, capi.MVH_ACT_REF)
    want = oracle.matmul_batch_v06(w, synth.Q4_0, n, k, x, is_ffn=False, force_q8=False)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    assert np.array_equal(bits(got[fin]), bits(want[fin]))
    t.free()


@pytest.mark.parametrize("ty", [synth.Q4_0, synth.Q8_0])
@pytest.mark.parametrize("batch,k,n", [(2, 1024, 96), (32, 4096, 512), (7, 288, 768)])
def test_matmul_v06_q8_mode_bitexact(ctx, oracle, ty, batch, k, n):
    rng = np.random.default_rng(batch + k + n + ty)
    w = _w(rng, ty, n, k)
    t = ctx.upload("blk.0.attn_k.weight", ty, k, n, w)
    x = synth.activations(rng, batch, k)
    got = ctx.matmul_batch_v06(t, x, capi.MVH_ACT_Q8)
    want = oracle.matmul_batch_v06(w, ty, n, k, x, is_ffn=False, force_q8=True)
    assert_bitexact(got, want, f"v06 q8 B={batch}")
    t.free()


@pytest.mark.parametrize("ty", [synth.Q4_0, synth.Q8_0])
@pytest.mark.parametrize("batch,k,n", [(32, 2048, 2048), (32, 2048, 256), (37, 4096, 300), (16, 256, 45),
                                       (48, 5632, 33), (17, 11008, 1)])
def test_blocksum_rows_bitexact(ctx, oracle, ty, batch, k, n):
    """dot_q4_0_fp32 / dot_q8_0_fp32 numerics on whole 16-token groups of the
    staged two-row kernel (K % 256 == 0), the rest of the tokens per token:
    tensor_matmul_batch for both types and tensor_matmul_batch_v06 with
    MEMVANTA_FORCE_Q8_ACT for Q8_0; the TinyLlama-1.1B attention shapes, rows
    off the 32-row tile down to one row, one-unit rows, ragged batches."""
    rng = np.random.default_rng(batch * 7 + k + n + ty)
    w = _w(rng, ty, n, k)
    t = ctx.upload("blk.0.attn_q.weight", ty, k, n, w)
    x = synth.activations(rng, batch, k)
    want = oracle.matmul_batch(w, ty, n, k, x)
    assert_bitexact(ctx.matmul_batch(t, x), want, f"matmul_batch B={batch} K={k} N={n}")
    if ty == synth.Q8_0:
        want_v06 = oracle.matmul_batch_v06(w, ty, n, k, x, is_ffn=False, force_q8=True)
        assert_bitexact(want_v06, want, "FORCE_Q8 Q8_0 is the per-token dot")
        assert_bitexact(ctx.matmul_batch_v06(t, x, capi.MVH_ACT_Q8), want, f"v06 q8 B={batch} K={k} N={n}")
    t.free()


@pytest.mark.parametrize("batch,k,n", [(32, 4096, 4096), (128, 4096, 1024), (512, 4096, 256), (32, 4096, 11008),
                                        (32, 11008, 4096), (33, 256, 100), (3, 512, 17), (70, 768, 45),
                                        (300, 4096, 1000), (257, 256, 63), (400, 11008, 70)])
def test_prefill_gemm_int8_mfma_bitexact(ctx, oracle, batch, k, n):
    """The int8-MFMA Q4_0 x Q8 GEMM (K % 256 == 0) against the FORCE_Q8 reference
    chain: the GEMM config shapes, plus token and row counts off the 32 x 32 tile
    and, from 256 tokens (the workgroup kernel), off its 64-row x 32-token tile
    (a partial last token group, a partial last row group, one K-chunk)."""
    rng = np.random.default_rng(batch * 7 + k + n)
    w = _w(rng, synth.Q4_0, n, k)
    t = ctx.upload("blk.0.ffn_gate.weight", synth.Q4_0, k, n, w)
    x = synth.activations(rng, batch, k)
    got = ctx.matmul_batch_v06(t, x, capi.MVH_ACT_Q8)
    want = oracle.matmul_batch_v06(w, synth.Q4_0, n, k, x, is_ffn=True, force_q8=True)
    assert_bitexact(got, want, f"mfma gemm M={batch} K={k} N={n}")
    t.free()


@pytest.mark.parametrize("k,n", [(4096, 4096), (4096, 11008), (11008, 4096)])
@pytest.mark.parametrize("m", [128, 512])
def test_prefill_gemm_config_shapes_bitexact(ctx, oracle, k, n, m):
    """The batched-prefill GEMM config at its full sizes (M = 128 / 512 on the
    7B FFN and attention shapes): the 32-token tile instances the bench times,
    against the FORCE_Q8 reference chain of every (row, token)."""
    rng = np.random.default_rng(m + 3 * k + n)
    w = _w(rng, synth.Q4_0, n, k)
    t = ctx.upload("blk.0.ffn_up.weight", synth.Q4_0, k, n, w)
    x = synth.activations(rng, m, k)
    got = ctx.matmul_batch_v06(t, x, capi.MVH_ACT_Q8)
    want = oracle.matmul_batch_v06(w, synth.Q4_0, n, k, x, is_ffn=True, force_q8=True, threads=16)
    assert_bitexact(got, want, f"mfma gemm M={m} K={k} N={n}")
    t.free()


def test_argmax_first_index_of_max(ctx):
    """Greedy sampling = std::max_element (src/llama_model.cpp:60): ties go to
    the first index, at any distance and in any row."""
    rng = np.random.default_rng(31)
    V = 32000
    rows = rng.standard_normal((8, V), dtype=np.float32)
    rows[0, [17, 9000, 31999]] = 50.0           # a tie across three threads
    rows[1, :] = 1.25                            # every element equal -> 0
    rows[2, :] = -np.inf                         # all -inf -> 0
    rows[3, 31999] = 99.0                        # max at the last index
    rows[4, [1023, 1024, 2047]] = 7.0            # ties straddling the 1024-lane stride
    rows[5, [5, 4]] = 9.0                        # adjacent tie
    rows[6, 0] = 12.0                            # max at index 0
    rows[7, [30000, 100]] = np.float32(3.0e38)   # the largest finite values
    got = ctx.argmax(rows)
    assert got.tolist() == [int(np.argmax(r)) for r in rows] == [17, 0, 0, 31999, 1023, 4, 0, 100]
    for n in (1, 2, 63, 1025):
        r = rng.standard_normal(n).astype(np.float32)
        assert int(ctx.argmax(r)[0]) == int(np.argmax(r))
    with pytest.raises(capi.MvhError, match="empty logits"):
        ctx.argmax(np.zeros((1, 0), np.float32))


def test_handles_outlive_their_context(oracle):
    """A tensor or KV cache freed after the context that created it was
    destroyed touches only its own device and memory (freeing once
    dereferenced the destroyed context: a use-after-free at process exit when
    a caller closed the context first); the tensor stays usable from another
    context on the same device."""
    rng = np.random.default_rng(404)
    k, n = 4096, 1003
    w = _w(rng, synth.Q4_0, n, k)
    c1 = capi.Context(0)
    t = c1.upload("blk.0.attn_q.weight", synth.Q4_0, k, n, w)
    kv = c1.kv_cache(2, 256, 128, 512)
    c1.close()
    c2 = capi.Context(0)
    try:
        x = synth.activations(rng, 1, k)[0]
        assert_bitexact(c2.matvec(t, x), oracle.matvec(w, synth.Q4_0, n, k, x), "tensor after its context closed")
        kv.close()
        t.free()
    finally:
        c2.close()


def test_stream_read_probe_arguments(ctx):
    import torch

    buf = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(1 << 20, dtype=torch.int32, device="cuda")
    ctx.stream_read(buf, buf.numel(), sink, sink.numel())
    ctx.synchronize()
    assert int(sink.abs().sum()) == 0  # zeros never produce the sink's trigger value
    with pytest.raises(capi.MvhError, match="multiple of 16"):
        ctx.stream_read(buf, 1000, sink, sink.numel())
    with pytest.raises(capi.MvhError):
        ctx.stream_read(buf, buf.numel(), sink, 16)  # sink smaller than one workgroup's words


@pytest.mark.parametrize("ty,k", [(synth.Q4_0, 288), (synth.Q8_0, 1024), (synth.Q6_K, 512)])
def test_matmul_batch_fallback(ctx, oracle, ty, k):
    rng = np.random.default_rng(k + ty)
    n = 80
    w = _w(rng, ty, n, k)
    t = ctx.upload("blk.1.ffn_down.weight", ty, k, n, w)
    x = synth.activations(rng, 3, k)
    got = ctx.matmul_batch(t, x)
    want = oracle.matmul_batch(w, ty, n, k, x)
    if ty == synth.Q6_K:
        assert ulp_diff(got, want).max() <= 2
    else:
        assert_bitexact(got, want, "matmul_batch")
    # batch 1 through v06 falls back to the same per-token fp32 dot
    assert_bitexact(ctx.matmul_batch_v06(t, x[:1]), got[:1], "v06 B=1")
    t.free()


@pytest.mark.parametrize("ty,k", [(synth.Q4_0, 288), (synth.Q8_0, 4096), (synth.Q6_K, 2048), (synth.F32, 100),
                                  (synth.F16, 300)])
def test_read_row(ctx, oracle, ty, k):
    rng = np.random.default_rng(k)
    n = 50
    w = _w(rng, ty, n, k)
    t = ctx.upload("token_embd.weight", ty, k, n, w)
    for row in (0, 17, n - 1):
        assert_bitexact(ctx.read_row(t, row), oracle.read_row(w, ty, n, k, row), f"row {row}")
    with pytest.raises(capi.MvhError, match="tensor row shape mismatch"):
        ctx.read_row(t, n)
    with pytest.raises(capi.MvhError, match="tensor row shape mismatch: token_embd.weight"):
        ctx.read_row(t, 0, out=np.empty(k + 32, np.float32), cols=k + 32)  # cols != ne0
    t.free()


# ---------------------------------------------------------------- paged KV + attention

KV_TYPES = {"f32": capi.MVH_KV_F32, "f16": capi.MVH_KV_F16, "q8": capi.MVH_KV_Q8}


@pytest.mark.parametrize("tname", sorted(KV_TYPES))
@pytest.mark.parametrize("kv_dim,page", [(288, 128), (256, 16), (4096, 128)])
def test_kv_write_bits_and_pages(ctx, oracle, kv_dim, page, tname):
    """Stored rows (elements and the Q8 row scale) bit-identical to PagedKVCache::write."""
    kt = KV_TYPES[tname]
    rng = np.random.default_rng(kv_dim + page + kt)
    kv = ctx.kv_cache(2, kv_dim, page, 400, kv_type=kt)
    assert kv.type() == kt
    okv = oracle.kv(kv_dim, page, kt)
    n = 300
    k = rng.standard_normal((n, kv_dim), dtype=np.float32) * np.float32(3)
    v = rng.standard_normal((n, kv_dim), dtype=np.float32)
    k[1] = 0.0                                  # Q8: all-zero row, scale 1
    v[2, 5] = np.float32(-1e30)                 # Q8: one huge element, the rest round to 0
    k[3, :4] = np.array([127.0, 0.5, -0.5, 2.5], np.float32)  # Q8: max 127 -> scale 1, ties away from zero
    kv.write(1, 0, k[:37], v[:37])          # a multi-token write
    for p in range(37, n):
        kv.write(1, p, k[p], v[p])
    for p in range(n):
        okv.write(p, k[p], v[p])
    for p in (0, 1, 2, 3, 36, 37, page - 1, page, n - 1):
        for which in (0, 1):
            got, gs = kv.read_row(1, p, which)
            want, ws = okv.row(p, which)
            assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), (p, which)
            assert bits(gs) == bits(ws), (p, which, gs, ws)
    assert kv.bytes_allocated() == okv.bytes_allocated()
    with pytest.raises(capi.MvhError, match="page missing"):
        kv.read_row(0, 0, 0)
    kv.reset()
    assert kv.bytes_allocated() == 0
    with pytest.raises(capi.MvhError, match="context exhausted"):
        kv.write(0, 399, k[:2], v[:2])
    kv.close()


@pytest.mark.parametrize("tname", sorted(KV_TYPES))
@pytest.mark.parametrize("n_head,n_kv,hd,pos", [(6, 6, 48, 0), (6, 6, 48, 200), (32, 4, 64, 511),
                                                (32, 32, 128, 767), (32, 32, 128, 130)])
def test_attn_decode(ctx, oracle, n_head, n_kv, hd, pos, tname):
    kt = KV_TYPES[tname]
    rng = np.random.default_rng(n_head + hd + pos)
    kv_dim = n_kv * hd
    kv = ctx.kv_cache(1, kv_dim, 128, 1024, kv_type=kt)
    okv = oracle.kv(kv_dim, 128, kt)
    k = rng.standard_normal((pos + 1, kv_dim), dtype=np.float32)
    v = rng.standard_normal((pos + 1, kv_dim), dtype=np.float32)
    kv.write(0, 0, k, v)
    for p in range(pos + 1):
        okv.write(p, k[p], v[p])
    q = rng.standard_normal(n_head * hd, dtype=np.float32) * np.float32(2)
    got = kv.attn_decode(0, q, pos, n_head, n_kv, hd)
    want = okv.attn_decode(q, pos, n_head, n_kv, hd)
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel <= 1e-6, rel
    assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()
    print(f"attn exact fraction {(bits(got) == bits(want)).mean():.4f}")
    kv.close()


@pytest.mark.parametrize("tname", sorted(KV_TYPES))
@pytest.mark.parametrize("n_head,n_kv,hd,pos,B", [(32, 4, 128, 100, 45), (32, 32, 128, 0, 32), (6, 6, 48, 37, 5),
                                                  (8, 2, 64, 300, 1)])
def test_attn_batch(ctx, oracle, n_head, n_kv, hd, pos, B, tname):
    """The batched causal attention of forward_batch_impl (src/llama_model.cpp:248): token b of the batch
    equals decode attention at position pos + b over the same cache."""
    kt = KV_TYPES[tname]
    rng = np.random.default_rng(n_head + hd + pos + B)
    kv_dim = n_kv * hd
    kv = ctx.kv_cache(1, kv_dim, 128, 1024, kv_type=kt)
    okv = oracle.kv(kv_dim, 128, kt)
    n = pos + B
    k = rng.standard_normal((n, kv_dim), dtype=np.float32)
    v = rng.standard_normal((n, kv_dim), dtype=np.float32)
    kv.write(0, 0, k, v)
    for p in range(n):
        okv.write(p, k[p], v[p])
    q = rng.standard_normal((B, n_head * hd), dtype=np.float32) * np.float32(2)
    got = kv.attn_batch(0, q, pos, B, n_head, n_kv, hd)
    want = np.stack([okv.attn_decode(q[b], pos + b, n_head, n_kv, hd) for b in range(B)])
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel <= 1e-6, rel
    assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()
    with pytest.raises(capi.MvhError, match="context exhausted"):
        kv.attn_batch(0, q, 1024 - B + 1, B, n_head, n_kv, hd)
    kv.close()


@pytest.mark.parametrize("k", [8, 9, 12, 13, 15, 301, 4096])
def test_gemv_f32_bitexact(ctx, oracle, k):
    """F32 weights: dot_f32_simd per (row, token) -- 8 fma lanes, t0+..+t7, the tail 4-wide unfused then fused --
    bit-exact for every tail length, through matvec and matmul_batch."""
    rng = np.random.default_rng(k)
    n = 70
    w = synth.quantize(synth.F32, rng.standard_normal((n, k), dtype=np.float32))
    t = ctx.upload("blk.0.attn_q.weight", synth.F32, k, n, w)
    x = rng.standard_normal(k, dtype=np.float32)
    assert_bitexact(ctx.matvec(t, x), oracle.matvec(w, synth.F32, n, k, x), f"F32 matvec {k}")
    xb = rng.standard_normal((3, k), dtype=np.float32)
    assert_bitexact(ctx.matmul_batch(t, xb), oracle.matmul_batch(w, synth.F32, n, k, xb), f"F32 batch {k}")
    t.free()


@pytest.mark.parametrize("k,n", [(301, 33), (4096, 4096), (2048, 32000)])
def test_gemv_f16(ctx, oracle, k, n):
    """F16 weights: the double sum of the reference added as per-lane partials and a wave tree."""
    rng = np.random.default_rng(k + n)
    w = synth.quantize(synth.F16, rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    t = ctx.upload("output.weight", synth.F16, k, n, w)
    x = synth.activations(rng, 1, k)[0]
    got = ctx.matvec(t, x)
    want = oracle.matvec(w, synth.F16, n, k, x)
    u = ulp_diff(got, want)
    assert u.max() <= 2, u.max()
    assert (u == 0).mean() >= 0.999, (u == 0).mean()
    xb = synth.activations(rng, 2, k)
    gb = ctx.matmul_batch(t, xb)
    wb = oracle.matmul_batch(w, synth.F16, n, k, xb)
    assert ulp_diff(gb, wb).max() <= 2
    t.free()


_WG_CHILD = r"""
import sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from memvanta_amd import capi, synth
from oracle.pyoracle import Oracle
o, ctx = Oracle(), capi.Context(0)
for batch, k, n in [(3, 512, 17), (33, 256, 100), (40, 4096, 70), (300, 4096, 1000)]:
    rng = np.random.default_rng(batch + k + n)
    w = synth.quantize(synth.Q4_0, rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    t = ctx.upload("blk.0.ffn_gate.weight", synth.Q4_0, k, n, w)
    x = synth.activations(rng, batch, k)
    got = ctx.matmul_batch_v06(t, x, capi.MVH_ACT_Q8)
    want = o.matmul_batch_v06(w, synth.Q4_0, n, k, x, is_ffn=True, force_q8=True)
    bad = int((got.view(np.uint32) != want.view(np.uint32)).sum())
    print(f"M={batch} K={k} N={n} differing={bad}", flush=True)
    assert bad == 0
    t.free()
ctx.close()
print("ok", flush=True)
"""


@pytest.mark.parametrize("wg", ["1", "0"])
def test_prefill_gemm_kernel_override_bitexact(wg):
    """MVH_GEMM_WG (read once per process) forces the workgroup int8-MFMA GEMM
    at every batch size (1) or never (0): both selections against the
    FORCE_Q8 reference chain in a child process that sets it before any GPU
    call -- small and ragged token counts on the workgroup kernel, 300 tokens
    on the wave-private kernel."""
    import os
    import subprocess
    import sys

    from conftest import ROOT

    env = dict(os.environ, MVH_GEMM_WG=wg)
    p = subprocess.run([sys.executable, "-u", "-c", _WG_CHILD, ROOT], env=env, capture_output=True, text=True,
                       timeout=110)
    assert p.returncode == 0 and p.stdout.strip().endswith("ok"), p.stdout + p.stderr
