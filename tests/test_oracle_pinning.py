"""Pins the C restatement (oracle/mv_oracle.c) to MemVanta's own outputs.

* golden vectors written by tests/golden/make_golden.py from the compiled
  reference (bit-exact comparisons);
* the compiled reference itself when oracle/_ref is built here (exhaustive
  fp32_to_fp16 sweep, live model run);
* closed forms and invariants (exact fp16 decode, quantizer special cases,
  fp64 brute-force bounds, thread-count independence, 8- vs 4-token blocking);
* planted mistakes: mutated copies of the oracle must FAIL the golden check,
  which shows the checks above would catch each of those errors.
"""
import hashlib
import os
import shutil
import subprocess
import tempfile

import numpy as np
import pytest

from conftest import ROOT, assert_bitexact, bits, golden
from memvanta_amd import synth

import importlib.util

_spec = importlib.util.spec_from_file_location("make_golden", os.path.join(ROOT, "tests", "golden", "make_golden.py"))
mg = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(mg)


@pytest.fixture(scope="module")
def mats():
    """Weights of make_golden.MATS regenerated from the seed (sha-checked)."""
    g = golden("kernels.npz")
    rng = np.random.default_rng(mg.MAT_SEED)
    out = {}
    for name, rows, cols, ty in mg.MATS:
        w = synth.quantize(ty, rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02))
        key = name.replace(".", "_")
        assert hashlib.sha256(w.tobytes()).hexdigest() == str(g[f"{key}__sha"]), f"weight generator drifted: {name}"
        out[name] = (w, rows, cols, ty, key)
    return out


@pytest.fixture(scope="module")
def tiny_model(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("model") / "tiny.gguf")
    sha = synth.write_model(synth.TINY, path, seed=1234)
    assert sha == str(golden("model_tiny.npz")["model_sha"]), "model generator drifted"
    return path


@pytest.fixture(scope="module")
def gqa_model(tmp_path_factory):
    """The 2-layer TinyLlama-shape mixed model (32 heads over 4 KV heads)."""
    g = golden("model_gqa.npz")
    path = str(tmp_path_factory.mktemp("gqa") / "gqa.gguf")
    sha = synth.write_model(synth.TINYLLAMA_MIXED_2L, path, seed=int(g["seed"]))
    assert sha == str(g["model_sha"]), "model generator drifted"
    return path


def _gqa_check(o, path, tname, mode):
    """Oracle vs the compiled reference's GQA golden run: prefill logits of 40
    tokens (32 + 8 chunks), six greedy steps, the last step's logits, KV bytes."""
    g = golden("model_gqa.npz")
    key = f"{tname}_m{mode}"
    m = o.model(path, ctx=256, force_q8=bool(mode), kv_type=KV_TYPES[tname])
    try:
        assert_bitexact(m.prefill(g["prompt"], 32), g[f"prefill_logits_{key}"], f"GQA prefill logits {key}")
        ids, cur = [], 29
        for _ in range(6):
            lg = m.forward(cur)
            cur = int(np.argmax(lg))
            ids.append(cur)
        assert ids == g[f"decode_ids_{key}"].tolist(), f"GQA greedy ids {key}"
        assert_bitexact(lg, g[f"decode_last_logits_{key}"], f"GQA decode logits {key}")
        assert m.kv_bytes() == int(g[f"kv_bytes_{key}"])
    finally:
        m.close()


# ----------------------------------------------------------------- fp16

def test_fp16_to_fp32_exhaustive(oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.fp16_to_fp32(h)
    want = h.view(np.float16).astype(np.float32)
    ok = ~np.isnan(want)
    assert np.array_equal(bits(got)[ok], bits(want)[ok])
    assert np.isnan(got[~ok]).all()


def test_fp32_to_fp16_golden(oracle):
    g = golden("fp16.npz")
    got = oracle.fp32_to_fp16(g["bits"].view(np.float32))
    assert np.array_equal(got, g["half"])
    # the quirks the golden set covers: ties away from zero, OR-ed carry
    kv = np.array([1.00048828125, 1.9999, 0.12499999, 65504.0, 70000.0, 1e-6, -1.9999], np.float32)
    assert [int(v) for v in oracle.fp32_to_fp16(kv)] == [0x3c01, 0x3c00, 0x2c00, 0x7bff, 0x7c00, 0x0011, 0xbc00]


def test_fp32_to_fp16_exhaustive_vs_reference(oracle, ref):
    step = 1 << 28
    for first in range(0, 1 << 32, step):
        want = ref.fp32_to_fp16_bits(first, step)
        bad = oracle.lib.mvo_fp32_to_fp16_count_mismatch(first, step, want)
        assert bad == 0, f"{bad} mismatches in [0x{first:08x}, +2^28)"


# ----------------------------------------------------------------- quantizer

def test_quantizer_probe_golden(oracle):
    g = golden("kernels.npz")
    w, x, y = g["probe__w"], g["probe__x"], g["probe__y"]
    for i in range(x.shape[0]):
        assert_bitexact(oracle.matvec(w, synth.Q4_0, 256, 256, x[i]), y[i], f"probe {i}")


def test_quantizer_overflow_edge_golden(oracle):
    """Blocks whose scale's reciprocal overflows (or whose scale underflows to
    0): the reference's x86 lround turns the non-finite quotients into -127."""
    g = golden("quant_edge.npz")
    w = mg.probe_matrix(256)
    for i in range(g["x"].shape[0]):
        assert_bitexact(oracle.matvec(w, synth.Q4_0, 256, 256, g["x"][i]), g["y"][i], f"edge probe {i}")
    q, _ = oracle.quantize_q8(g["x"])
    assert (q[0, :32] == -127).all()


def test_quantizer_closed_form(oracle):
    g = golden("kernels.npz")
    x = g["probe__x"]
    q, d = oracle.quantize_q8(x)
    # the probe rows recover d_a * q_e exactly rounded: same q from both sides
    y = g["probe__y"]
    for i in range(x.shape[0]):
        rec = (d[i].repeat(32).astype(np.float64) * q[i]).astype(np.float32)
        assert np.array_equal(bits(rec), bits(y[i]))
    blocks = x.reshape(x.shape[0], -1, 32)
    mx = np.abs(blocks).max(axis=2)
    assert np.array_equal(d[mx > 0], (mx[mx > 0] / np.float32(127)).astype(np.float32))
    assert (d[mx == 0] == 1).all() and (q.reshape(blocks.shape)[mx == 0] == 0).all()
    assert np.abs(q).max() == 127
    # x[2][:8] has block max 127 -> d = 1, and ties round away from zero
    assert list(q[2][:8]) == [3, -3, 1, -1, 127, 127, -127, 2]
    assert q[3][32:64].tolist() == [127] * 32  # 1e-30 block: d = mx/127 still normalises


# ----------------------------------------------------------------- kernels

def test_matvec_golden(oracle, mats):
    g = golden("kernels.npz")
    for name, (w, rows, cols, ty, key) in mats.items():
        assert_bitexact(oracle.matvec(w, ty, rows, cols, g[f"{key}__x"]), g[f"{key}__matvec"], f"matvec {name}")


def test_matmul_batch_golden(oracle, mats):
    g = golden("kernels.npz")
    for name, (w, rows, cols, ty, key) in mats.items():
        assert_bitexact(oracle.matmul_batch(w, ty, rows, cols, g[f"{key}__xb"]), g[f"{key}__batch"], f"batch {name}")


def test_matmul_v06_golden_both_modes(oracle, mats):
    g = golden("kernels.npz")
    n = 0
    for name, (w, rows, cols, ty, key) in mats.items():
        for B in (2, 5, 11, 32):
            if f"{key}__v06_x{B}" not in g:
                continue
            X = g[f"{key}__v06_x{B}"]
            ffn = ".ffn_" in name
            assert_bitexact(oracle.matmul_batch_v06(w, ty, rows, cols, X, ffn, False), g[f"{key}__v06_ref{B}"],
                            f"v06 ref {name} B={B}")
            assert_bitexact(oracle.matmul_batch_v06(w, ty, rows, cols, X, ffn, True), g[f"{key}__v06_q8{B}"],
                            f"v06 q8 {name} B={B}")
            n += 1
    assert n == 12  # three K=1024 tensors x four batch sizes


def test_read_row_golden(oracle, mats):
    g = golden("kernels.npz")
    w, rows, cols, ty, key = mats["token_embd.weight"]
    assert_bitexact(oracle.read_row(w, ty, rows, cols, 5), g[f"{key}__row5"], "read_row")


def test_fp64_bounds(oracle, mats):
    """The fp32 results stay within a few ulp-scale units of the exact dot."""
    g = golden("kernels.npz")
    for name, (w, rows, cols, ty, key) in mats.items():
        x = g[f"{key}__x"]
        W = synth.dequantize(ty, w, rows, cols)
        if ty == synth.Q4_0:  # the activation is quantized first
            q, d = oracle.quantize_q8(x)
            xe = q.astype(np.float64) * np.repeat(d.astype(np.float64), 32)
        else:
            xe = x.astype(np.float64)
        exact = W @ xe
        got = oracle.matvec(w, ty, rows, cols, x).astype(np.float64)
        scale = np.abs(W) @ np.abs(xe)
        assert (np.abs(got - exact) <= 1e-6 * scale + 1e-30).all(), name


def test_thread_count_independence(oracle, mats):
    g = golden("kernels.npz")
    for name, (w, rows, cols, ty, key) in mats.items():
        x = g[f"{key}__x"]
        assert_bitexact(oracle.matvec(w, ty, rows, cols, x, threads=1), oracle.matvec(w, ty, rows, cols, x, threads=7),
                        name)


def test_batch8_equals_two_batch4(oracle, mats):
    """FFN tensors block 8 tokens as two 4-token calls: identical results."""
    g = golden("kernels.npz")
    w, rows, cols, ty, key = mats["blk.0.ffn_up.weight"]
    X = g[f"{key}__v06_x32"]
    assert_bitexact(oracle.matmul_batch_v06(w, ty, rows, cols, X, True), oracle.matmul_batch_v06(w, ty, rows, cols, X, False),
                    "batch8 vs batch4")


def test_kv_golden(oracle):
    g = golden("kv.npz")
    kv = oracle.kv(64, int(g["page"]))
    for p in range(g["k"].shape[0]):
        kv.write(p, g["k"][p], g["v"][p])
    q = g["q"]
    dots = np.array([[kv.dot_key(p, off, q[off:off + 32]) for off in (0, 32)] for p in range(g["k"].shape[0])],
                    np.float32)
    assert_bitexact(dots, g["dots"], "dot_key")
    acc = np.zeros(64, np.float32)
    for p in range(g["k"].shape[0]):
        kv.add_value(p, 0, np.float32(0.37 / (p + 1)), acc)
    assert_bitexact(acc, g["acc"], "add_value")
    assert kv.bytes_allocated() == int(g["bytes"])


KV_TYPES = {"f32": 0, "f16": 1, "q8": 2}


def _kv_types_check(o, tname):
    """Replays kv_types.npz for one cache type through oracle `o`."""
    g = golden("kv_types.npz")
    kv = o.kv(64, int(g[f"{tname}__page"]), KV_TYPES[tname])
    k, v = g[f"{tname}__k"], g[f"{tname}__v"]
    for p in range(k.shape[0]):
        kv.write(p, k[p], v[p])
    lens, offs, qs = g[f"{tname}__lens"], g[f"{tname}__offs"], g[f"{tname}__qs"]
    dots = np.array([[kv.dot_key(p, int(offs[i]), qs[i, :lens[i]]) for i in range(lens.size)]
                     for p in range(k.shape[0])], np.float32)
    assert_bitexact(dots, g[f"{tname}__dots"], f"{tname} dot_key (tails 1..23)")
    onehot = np.zeros_like(g[f"{tname}__onehot"])
    for p in range(k.shape[0]):
        for d in range(64):
            e = np.zeros(8, np.float32)
            e[d % 8] = 1.0
            onehot[p, d] = kv.dot_key(p, d - d % 8, e)
    assert_bitexact(onehot, g[f"{tname}__onehot"], f"{tname} stored values x scale")
    for ln, off in ((64, 0), (29, 3), (7, 40)):
        acc = np.zeros(ln, np.float32)
        for p in range(k.shape[0]):
            kv.add_value(p, off, np.float32(0.37 / (p + 1)) if p % 3 else np.float32(-1.25), acc)
        assert_bitexact(acc, g[f"{tname}__acc{ln}"], f"{tname} add_value")
    assert kv.bytes_allocated() == int(g[f"{tname}__bytes"])
    return kv


@pytest.mark.parametrize("tname", sorted(KV_TYPES))
def test_kv_types_golden(oracle, tname):
    _kv_types_check(oracle, tname)


def test_kv_type_names(oracle):
    g = golden("kv_types.npz")
    assert [oracle.kv_type_name(t) for t in range(3)] == g["names"].tolist()
    assert [oracle.kv_parse_type(s) for s in ("f32", "f16", "q8", "q8_0")] == g["parsed"].tolist()
    with pytest.raises(RuntimeError, match="unknown KV cache type: bf16"):
        oracle.kv_parse_type("bf16")


def test_kv_q8_special_cases(oracle):
    """Closed-form cases of the Q8 row: an all-zero row has scale 1 and
    stores zeros; a row whose max is 127 has scale exactly 1, so x/s = x and
    the stored values are x rounded half away from zero; the max element
    always stores +-127; scales are per token, shared by all heads."""
    kv = oracle.kv(16, 4, KV_TYPES["q8"])
    z = np.zeros(16, np.float32)
    x = np.array([127, -0.5, 0.5, 1.5, -2.5, 2.4999998, 126.5, -126.5] + [0] * 8, np.float32)
    y = np.linspace(-3, 7, 16).astype(np.float32)
    kv.write(0, z, x)
    kv.write(1, y, z)
    q, s = kv.row(0, 0)
    assert s == 1.0 and not q.any()
    q, s = kv.row(0, 1)
    assert s == 1.0 and q[:8].tolist() == [127, -1, 1, 2, -3, 2, 127, -127]
    q, s = kv.row(1, 0)
    assert s == np.float32(7) / np.float32(127) and q[-1] == 127 and np.abs(q).max() == 127
    # dot with a one-hot query returns float(q) * s, rounded once
    e = np.zeros(8, np.float32)
    e[3] = 1
    assert kv.dot_key(1, 8, e) == np.float32(np.float32(q[11]) * s)


def test_kv_types_vs_reference_live(oracle, ref):
    rng = np.random.default_rng(8)
    for t in KV_TYPES.values():
        ko, kr = oracle.kv(48, 5, t), ref.kv(48, 5, t)
        k = rng.standard_normal((23, 48), dtype=np.float32) * np.float32(4)
        v = rng.standard_normal((23, 48), dtype=np.float32)
        for p in range(23):
            ko.write(p, k[p], v[p])
            kr.write(p, k[p], v[p])
        for p in range(23):
            for ln in range(1, 25):
                q = rng.standard_normal(ln, dtype=np.float32)
                off = int(rng.integers(0, 48 - ln + 1))
                assert bits(ko.dot_key(p, off, q)) == bits(kr.dot_key(p, off, q)), (t, p, ln, off)
                ao = rng.standard_normal(ln, dtype=np.float32)
                ar = ao.copy()
                ko.add_value(p, off, np.float32(0.3), ao)
                kr.add_value(p, off, np.float32(0.3), ar)
                assert_bitexact(ao, ar, f"type {t} add_value")
        assert ko.bytes_allocated() == kr.bytes_allocated()


# ----------------------------------------------------------------- model

@pytest.mark.parametrize("mode", [0, 1])
def test_tiny_model_golden(oracle, tiny_model, mode):
    g = golden("model_tiny.npz")
    m = oracle.model(tiny_model, ctx=256, force_q8=bool(mode))
    assert_bitexact(m.prefill(g["prompt"], 32), g[f"prefill_logits_m{mode}"], "prefill logits")
    ids, cur = [], 17
    for _ in range(12):
        lg = m.forward(cur)
        cur = int(np.argmax(lg))
        ids.append(cur)
    assert ids == g[f"decode_ids_m{mode}"].tolist()
    assert_bitexact(lg, g[f"decode_last_logits_m{mode}"], "decode logits")
    assert m.kv_bytes() == int(g[f"kv_bytes_m{mode}"])
    m.reset()
    assert_bitexact(m.prefill(g["prompt33"], 32), g[f"prefill33_logits_m{mode}"], "prefill 32+1")


@pytest.mark.parametrize("tname", ["f32", "q8"])
@pytest.mark.parametrize("mode", [0, 1])
def test_tiny_model_kv_types_golden(oracle, tiny_model, tname, mode):
    g = golden("model_tiny.npz")
    m = oracle.model(tiny_model, ctx=256, force_q8=bool(mode), kv_type=KV_TYPES[tname])
    assert_bitexact(m.prefill(g["prompt"], 32), g[f"kv{tname}_prefill_logits_m{mode}"], "prefill logits")
    ids, cur = [], 17
    for _ in range(12):
        lg = m.forward(cur)
        cur = int(np.argmax(lg))
        ids.append(cur)
    assert ids == g[f"kv{tname}_decode_ids_m{mode}"].tolist()
    assert_bitexact(lg, g[f"kv{tname}_decode_last_logits_m{mode}"], "decode logits")
    assert m.kv_bytes() == int(g[f"kv{tname}_kv_bytes_m{mode}"])


@pytest.mark.parametrize("tname", ["f16", "q8"])
@pytest.mark.parametrize("mode", [0, 1])
def test_gqa_model_golden(oracle, gqa_model, tname, mode):
    """32 query heads over 4 KV heads: head h reads KV head h / 8, which only a
    grouped-query model tells apart from h % 4 (the tiny model has group 1)."""
    _gqa_check(oracle, gqa_model, tname, mode)


def test_tiny_model_vs_reference_live(oracle, ref, tiny_model):
    mo = oracle.model(tiny_model, ctx=256)
    mr = ref.model(tiny_model, ctx=256)
    t = synth.prompt_tokens(77, 70)
    assert_bitexact(mo.prefill(t, 32), mr.prefill(t, 32), "live prefill")
    for tok in (3, 31999, 0):
        assert_bitexact(mo.forward(tok), mr.forward(tok), "live decode")


def test_model_errors(oracle, tiny_model):
    m = oracle.model(tiny_model, ctx=4)
    with pytest.raises(RuntimeError, match="token id out of range"):
        m.forward(32000)
    m.prefill(np.array([1, 2, 3, 4], np.int32), 2, logits=False)
    with pytest.raises(RuntimeError, match="context exhausted"):
        m.forward(1)


# ----------------------------------------------------------------- native block formats

def _native_check(o):
    """Oracle vs the compiled reference's native-format golden vectors
    (quantize_q8_0 / quantize_q4_0 probes, matvec_q4_q8, matmul_q4_0_batch,
    matvec_q4_0, matvec_q8_0 at K = 32, 288, 4096, 11008)."""
    g = golden("native.npz")
    assert np.array_equal(o.nq_quantize(g["probe_x"], 36), g["probe_q8"]), "quantize_q8_0 probes"
    assert np.array_equal(o.nq_quantize(g["probe_x"], 20), g["probe_q4"]), "quantize_q4_0 probes"
    for i, (rows, cols, B) in enumerate(mg.NATIVE_MATS):
        key = f"r{rows}_c{cols}"
        W = mg.native_weights(i, rows, cols)
        assert hashlib.sha256(W.tobytes()).hexdigest() == str(g[f"{key}__w_sha"]), "weight generator drifted"
        A4, A8 = o.nq_quantize(W, 20), o.nq_quantize(W, 36)
        assert hashlib.sha256(A4.tobytes()).hexdigest() == str(g[f"{key}__a4_sha"]), f"{key} quantize_q4_0"
        assert hashlib.sha256(A8.tobytes()).hexdigest() == str(g[f"{key}__a8_sha"]), f"{key} quantize_q8_0"
        assert np.array_equal(o.nq_quantize(g[f"{key}__x"], 36), g[f"{key}__xq"]), f"{key} activation quantize_q8_0"
        assert_bitexact(o.nq_matvec_q4_q8(A4, g[f"{key}__xq"], rows, cols), g[f"{key}__q4q8"], f"{key} matvec_q4_q8")
        assert_bitexact(o.nq_matmul_q4_0_batch(A4, g[f"{key}__X"], rows, cols), g[f"{key}__batch"],
                        f"{key} matmul_q4_0_batch")
        assert_bitexact(o.nq_matvec(A4, g[f"{key}__x"], rows, cols, 20), g[f"{key}__mv_q4_0"], f"{key} matvec_q4_0")
        assert_bitexact(o.nq_matvec(A8, g[f"{key}__x"], rows, cols, 36), g[f"{key}__mv_q8_0"], f"{key} matvec_q8_0")


def test_native_golden(oracle):
    _native_check(oracle)


def test_native_numpy_quantizers_golden():
    """memvanta_amd.synth's numpy quantizers (the GPU tests' input generator)
    write the reference's bytes."""
    g = golden("native.npz")
    assert np.array_equal(synth.quantize_q8_0_native(g["probe_x"]).reshape(-1, 36), g["probe_q8"])
    assert np.array_equal(synth.quantize_q4_0_native(g["probe_x"]).reshape(-1, 20), g["probe_q4"])
    for i, (rows, cols, B) in enumerate(mg.NATIVE_MATS):
        key = f"r{rows}_c{cols}"
        W = mg.native_weights(i, rows, cols)
        assert hashlib.sha256(synth.quantize_q4_0_native(W).tobytes()).hexdigest() == str(g[f"{key}__a4_sha"])
        assert hashlib.sha256(synth.quantize_q8_0_native(W).tobytes()).hexdigest() == str(g[f"{key}__a8_sha"])


def test_native_closed_forms(oracle):
    """Block decode against its definition: a Q4_0 block of nibbles (q+8) with
    d = 1 against a one-hot Q8 activation returns q (element 2i low nibble,
    2i+1 high); the fp64 brute-force dot bounds every matvec; the ties of the
    quantizers go to even."""
    qs = np.arange(32) % 16 - 8
    blk = np.zeros(20, np.uint8)
    blk[:4] = np.frombuffer(np.float32(1.0).tobytes(), np.uint8)
    blk[4:] = (qs[0::2] + 8) | ((qs[1::2] + 8) << 4)
    for e in range(32):
        xb = np.zeros(36, np.uint8)
        xb[:4] = np.frombuffer(np.float32(1.0).tobytes(), np.uint8)
        xb[4 + e] = 1
        assert oracle.nq_matvec_q4_q8(blk, xb, 1, 32)[0] == qs[e]
    t = np.zeros(32, np.float32)
    t[0] = 127.0
    t[1:5] = [0.5, 1.5, 2.5, -2.5]
    q = oracle.nq_quantize(t, 36)[0, 4:9].view(np.int8)
    assert q.tolist() == [127, 0, 2, 2, -2]
    rng = np.random.default_rng(3)
    rows, cols = 16, 1024
    W = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.02)
    A4 = oracle.nq_quantize(W, 20)
    x = rng.standard_normal(cols, dtype=np.float32)
    xq = oracle.nq_quantize(x, 36)
    wd = A4.reshape(rows, -1, 20)
    dw = wd[..., :4].copy().view(np.float32)[..., 0].astype(np.float64)
    nib = np.stack([wd[..., 4:] & 15, wd[..., 4:] >> 4], -1).reshape(rows, -1, 32).astype(np.float64) - 8
    xd = xq[:, :4].copy().view(np.float32)[:, 0].astype(np.float64)
    xv = xq[:, 4:].view(np.int8).astype(np.float64)
    exact = np.einsum("rbk,bk,rb,b->r", nib, xv, dw, xd)
    got = oracle.nq_matvec_q4_q8(A4, xq, rows, cols)
    assert np.all(np.abs(got - exact) <= 1e-4 * np.abs(exact).max())


def test_native_errors(oracle):
    with pytest.raises(RuntimeError, match="q4_q8 cols must be multiple of 32"):
        oracle.nq_matvec_q4_q8(np.zeros(40, np.uint8), np.zeros(72, np.uint8), 1, 48)
    with pytest.raises(RuntimeError, match="q4_0 cols must be multiple of 32"):
        oracle.nq_matmul_q4_0_batch(np.zeros(40, np.uint8), np.zeros(48, np.float32), 1, 48)
    with pytest.raises(RuntimeError, match="q8_0 length must be multiple of 32"):
        oracle.nq_quantize(np.zeros(48, np.float32), 36)


def test_native_vs_reference_live(oracle, ref):
    rng = np.random.default_rng(8)
    for rows, cols in ((5, 64), (33, 2048)):
        W = rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(0.05)
        x = synth.activations(rng, 1, cols)[0]
        A4 = ref.nq_quantize(W, 20)
        xq = ref.nq_quantize(x, 36)
        assert np.array_equal(oracle.nq_quantize(W, 20), A4)
        assert np.array_equal(oracle.nq_quantize(x, 36), xq)
        assert_bitexact(oracle.nq_matvec_q4_q8(A4, xq, rows, cols), ref.nq_matvec_q4_q8(A4, xq, rows, cols))
        X = synth.activations(rng, 4, cols)
        assert_bitexact(oracle.nq_matmul_q4_0_batch(A4, X, rows, cols), ref.nq_matmul_q4_0_batch(A4, X, rows, cols))


# ----------------------------------------------------------------- planted mistakes

MUTATIONS = {
    "rope_unfused": ("b[i] = fmaf(x0, c, -(x1 * s));", "b[i] = x0 * c - x1 * s;"),
    "q4q8_unfused": ("sum = fmaf(p, (float)dot_q4_q8_block(blk, aq + 32 * b), sum);",
                     "sum = sum + p * (float)dot_q4_q8_block(blk, aq + 32 * b);"),
    "quant_round_even": ("long r = lroundf(z[k] * inv);", "long r = lrintf(z[k] * inv);"),
    "fp16_carry_added": ("return (uint16_t)(sign | ((uint32_t)exp << 10) | ((mant + 0x1000u) >> 13));",
                         "return (uint16_t)(sign | (((uint32_t)exp << 10) + ((mant + 0x1000u) >> 13)));"),
    "q8_lane_order": ("for (int j = 0; j < 8; ++j) t[j] = fmaf((float)qs[k + j], x[b * 32 + k + j], t[j]);",
                      "for (int j = 0; j < 8; ++j) t[j] = fmaf((float)qs[k + j], x[b * 32 + k + j], t[(j + k / 8) & 7]);"),
    "kv_q8_multiply_by_inverse": ("long r = lroundf(x[d] / s);", "long r = lroundf(x[d] * (1.0f / s));"),
    "kv_q8_scale_per_element": ("float w = kv->type == MVO_KV_Q8 ? alpha * sc : alpha;",
                                "float w = alpha;\n    if (kv->type == MVO_KV_Q8) alpha = sc;"),
    "f32_tail_all_fused": ("for (int j = 0; j < 4; ++j) s = s + a[i + j] * b[i + j];",
                           "for (int j = 0; j < 4; ++j) s = fmaf(a[i + j], b[i + j], s);"),
    # the KV head of query head h: h / group, not h % n_head_kv (equal when
    # group = 1), once in the decode attention and once in the prefill loop
    "gqa_head_map_decode": ("size_t kb = (h / group) * hd, qb = h * hd;",
                            "size_t kb = (h % n_head_kv) * hd, qb = h * hd;"),
    "gqa_head_map_prefill": ("kb = (h / group) * hd, qb = h * hd, upto = start + b;",
                             "kb = (h % m->n_head_kv) * hd, qb = h * hd, upto = start + b;"),
    # the score scale: a division by sqrtf(hd), not a product with its reciprocal
    # (src/llama_model.cpp:248,256), in the decode and in the prefill attention
    "attn_scale_reciprocal_decode": ("float sf = mvo_kv_dot_key(kv, t, kb, q + qb, hd) / sq;",
                                     "float sf = mvo_kv_dot_key(kv, t, kb, q + qb, hd) * (1.0f / sq);"),
    "attn_scale_reciprocal_prefill": ("float sf = mvo_kv_dot_key(m->kv[li], t, kb, Q + b * D + qb, hd) / sq;",
                                      "float sf = mvo_kv_dot_key(m->kv[li], t, kb, Q + b * D + qb, hd) * (1.0f / sq);"),
    # native blocks: the weight scale must multiply isum before the fused add of x.d
    "nq_q4q8_unfused": ("        sum = fmaf(p, nq_d(xb), sum);", "        sum = sum + p * nq_d(xb);"),
    "nq_q4q8_scale_order": ("float p = (float)isum * nq_d(wa);\n        sum = fmaf(p, nq_d(xb), sum);",
                            "float p = nq_d(wa) * nq_d(xb);\n        sum = fmaf(p, (float)isum, sum);"),
    "nq_quant_round_away": ("int q = (int)nearbyintf(p[i] * id);\n            q = q < -127",
                            "int q = (int)lroundf(p[i] * id);\n            q = q < -127"),
    "nq_nibble_gguf_order": ("q[k] = ((k & 1) ? (packed >> 4) : (packed & 0x0f)) - 8;",
                             "q[k] = (k < 16 ? (wa[4 + k] & 15) : (wa[4 + k - 16] >> 4)) - 8; (void)packed;"),
    "nq_zero_block_unit_scale": ("float d = amax == 0.0f ? 0.0f : amax / 7.0f;",
                                 "float d = amax == 0.0f ? 1.0f : amax / 7.0f;"),
    "batch4_unrounded_scale": ("float q = (float)qi * d;\n                    size_t off = b * 32 + h * 16 + k + j;",
                               "float q = (float)qi;\n                    size_t off = b * 32 + h * 16 + k + j;"),
}


def _mutant(tmp, name):
    src = open(os.path.join(ROOT, "oracle", "mv_oracle.c")).read()
    a, b = MUTATIONS[name]
    assert a in src, f"mutation anchor missing: {name}"
    d = os.path.join(tmp, name)
    os.makedirs(d)
    shutil.copy(os.path.join(ROOT, "oracle", "mv_oracle.h"), d)
    with open(os.path.join(d, "mv_oracle.c"), "w") as f:
        f.write(src.replace(a, b))
    so = os.path.join(d, "lib.so")
    subprocess.run(["gcc", "-std=gnu11", "-O2", "-mavx2", "-mfma", "-mf16c", "-ffp-contract=off", "-fopenmp", "-fPIC",
                    "-shared", "-o", so, os.path.join(d, "mv_oracle.c"), "-lm"], check=True)
    from oracle.pyoracle import Oracle

    return Oracle(so)


def _golden_ok(o, mats, tiny_model, gqa_model):
    g = golden("kernels.npz")
    try:
        for name, (w, rows, cols, ty, key) in mats.items():
            assert_bitexact(o.matvec(w, ty, rows, cols, g[f"{key}__x"]), g[f"{key}__matvec"])
            for B in (5, 32):
                if f"{key}__v06_x{B}" in g:
                    X = g[f"{key}__v06_x{B}"]
                    assert_bitexact(o.matmul_batch_v06(w, ty, rows, cols, X, ".ffn_" in name, False),
                                    g[f"{key}__v06_ref{B}"])
        for i in range(g["probe__x"].shape[0]):
            assert_bitexact(o.matvec(g["probe__w"], synth.Q4_0, 256, 256, g["probe__x"][i]), g["probe__y"][i])
        f16 = golden("fp16.npz")
        assert np.array_equal(o.fp32_to_fp16(f16["bits"].view(np.float32)), f16["half"])
        gm = golden("model_tiny.npz")
        m = o.model(tiny_model, ctx=256)
        try:
            assert_bitexact(m.prefill(gm["prompt"], 32), gm["prefill_logits_m0"])
            # the decode sites too (head_dim 48: sqrtf(48) is not a power of two, unlike the GQA model's 64)
            ids, cur = [], 17
            for _ in range(12):
                lg = m.forward(cur)
                cur = int(np.argmax(lg))
                ids.append(cur)
            assert ids == gm["decode_ids_m0"].tolist()
            assert_bitexact(lg, gm["decode_last_logits_m0"])
        finally:
            m.close()
        for tname in KV_TYPES:
            _kv_types_check(o, tname)
        _gqa_check(o, gqa_model, "f16", 0)
        _native_check(o)
    except AssertionError:
        return False
    return True


def test_unmutated_oracle_passes_golden_checks(oracle, mats, tiny_model, gqa_model):
    """The control of the planted-mistake tests: the checks accept the oracle as built."""
    assert _golden_ok(oracle, mats, tiny_model, gqa_model)


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_planted_mistake_is_caught(name, mats, tiny_model, gqa_model):
    with tempfile.TemporaryDirectory() as tmp:
        assert not _golden_ok(_mutant(tmp, name), mats, tiny_model, gqa_model), f"golden checks miss mutation {name}"
