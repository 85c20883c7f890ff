"""End-to-end parity of the device-resident LlamaModel (mvh_model_*).

The tiny config is compared with the compiled reference's own logits and
greedy ids (golden vectors); the GQA / Q8_0 / Q6_K config and a 7B-shape layer
are compared with the oracle run live on the host.  Greedy ids must be
identical; logits within 1e-3 relative L2 (the bit-identical fraction is
asserted too: every step reproduces the reference's operation order, only the
double sums of RMSNorm and the softmax denominator are added as trees)."""
import numpy as np
import pytest

from conftest import bits, golden
from memvanta_amd import capi, synth

pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / np.linalg.norm(b.astype(np.float64)))


def close(got, want, what, exact_frac=0.999):
    r = rel_l2(got, want)
    assert r <= 1e-3, f"{what}: rel L2 {r}"
    frac = float((bits(got) == bits(want)).mean())
    assert frac >= exact_frac, f"{what}: only {frac:.4f} of logits bit-identical (rel L2 {r:.2e})"


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("m") / "tiny.gguf")
    assert synth.write_model(synth.TINY, path, seed=1234) == str(golden("model_tiny.npz")["model_sha"])
    return path


@pytest.mark.parametrize("mode", [0, 1])
def test_tiny_prefill_decode_vs_reference_golden(tiny, mode):
    g = golden("model_tiny.npz")
    m = capi.Model(tiny, ctx=256, act_mode=mode, max_batch=32)
    close(m.prefill(g["prompt"], 32), g[f"prefill_logits_m{mode}"], "prefill")
    ids, cur = [], 17
    for _ in range(12):
        lg = m.forward(cur)
        cur = int(np.argmax(lg))
        ids.append(cur)
    assert ids == g[f"decode_ids_m{mode}"].tolist()
    close(lg, g[f"decode_last_logits_m{mode}"], "decode")
    assert m.kv_bytes() == int(g[f"kv_bytes_m{mode}"])
    m.reset()
    assert m.kv_bytes() == 0
    close(m.prefill(g["prompt33"], 32), g[f"prefill33_logits_m{mode}"], "prefill 32+1")
    m.close()


def test_tiny_graph_greedy_equals_stepwise(tiny):
    g = golden("model_tiny.npz")
    m = capi.Model(tiny, ctx=256, max_batch=32)
    m.prefill(g["prompt"], 32, logits=False)
    ids, last = m.generate_greedy(17, 12, logits=True)
    assert ids.tolist() == g["decode_ids_m1"].tolist()
    close(last, g["decode_last_logits_m1"], "graph decode")
    assert m.position == 40 + 12
    # a second run from the same state replays the same captured graph
    m.reset()
    m.prefill(g["prompt"], 32, logits=False)
    assert m.generate_greedy(17, 12).tolist() == g["decode_ids_m1"].tolist()
    m.close()


def test_model_errors(tiny):
    m = capi.Model(tiny, ctx=8, max_batch=4)
    with pytest.raises(capi.MvhError, match="token id out of range"):
        m.forward(32000)
    with pytest.raises(capi.MvhError, match="larger than"):
        m.prefill(np.arange(8, dtype=np.int32), 8)
    m.prefill(np.arange(8, dtype=np.int32), 4, logits=False)
    with pytest.raises(capi.MvhError, match="context exhausted"):
        m.forward(1)
    m.close()


@pytest.mark.parametrize("n_prompt,chunk", [(150, 32), (230, 16), (77, 5), (24, 1)])
@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("kv", [capi.MVH_KV_F16, capi.MVH_KV_Q8, capi.MVH_KV_F32])
def test_pipelined_prefill_equals_chunk_by_chunk(tiny, mode, kv, n_prompt, chunk):
    """The chunks of one prefill call take three streams in turn (chunk c + 1
    computes layer l beside chunk c's layer l + 1, its attention of layer l
    ordered after the KV writes of layer l of every earlier chunk).  Logits,
    KV bytes and the greedy ids that follow must be bit-identical to one call
    per chunk, where nothing runs beside a chunk.  150 / 32: four full chunks
    and a ragged 22, the lanes wrap once; 230 / 16: fifteen chunks, the
    lanes wrap four times; 77 / 5: chunks that are not whole 16-token GEMM
    slabs; 24 / 1: one-token chunks (the per-token matmul path)."""
    prompt = synth.prompt_tokens(9, n_prompt)
    runs = []
    for split in (False, True):
        m = capi.Model(tiny, ctx=256, act_mode=mode, max_batch=32, kv_type=kv)
        if split:
            for i in range(0, len(prompt), chunk):
                lg = m.prefill(prompt[i:i + chunk], chunk, logits=i + chunk >= len(prompt))
        else:
            lg = m.prefill(prompt, chunk)
        runs.append((lg.copy(), m.kv_bytes(), m.position, m.generate_greedy(17, 6).tolist()))
        m.close()
    (a, kb_a, pos_a, ids_a), (b, kb_b, pos_b, ids_b) = runs
    assert (bits(a) == bits(b)).all()
    assert (kb_a, pos_a, ids_a) == (kb_b, pos_b, ids_b)


@pytest.mark.parametrize("chunk", [32, 16])
def test_pipelined_prefill_equals_chunk_by_chunk_hd128(tmp_path, chunk):
    """As above on a one-layer 7B-shape model (head_dim 128: the chunked
    scores/softmax + value kernels and the int8-MFMA GEMM in every chunk)."""
    cfg = synth.dataclasses.replace(synth.LLAMA7B_1L, name="openllama-7b-v2-q4_0-1layer-pipe", ctx=256)
    path = str(tmp_path / "m.gguf")
    synth.write_model(cfg, path, seed=41)
    prompt = synth.prompt_tokens(12, 120)
    runs = []
    for split in (False, True):
        m = capi.Model(path, ctx=256, act_mode=1, max_batch=32)
        if split:
            for i in range(0, len(prompt), chunk):
                lg = m.prefill(prompt[i:i + chunk], chunk, logits=i + chunk >= len(prompt))
        else:
            lg = m.prefill(prompt, chunk)
        runs.append((lg.copy(), m.kv_bytes(), m.generate_greedy(3, 4).tolist()))
        m.close()
    (a, kb_a, ids_a), (b, kb_b, ids_b) = runs
    assert (bits(a) == bits(b)).all()
    assert (kb_a, ids_a) == (kb_b, ids_b)


@pytest.mark.parametrize("mode", [0, 1])
def test_whole_prompt_batch_equals_chunks_of_32(tmp_path, mode):
    """One prefill batch for the whole prompt (every GEMM at M = 256: the
    workgroup int8-MFMA kernel in FORCE_Q8 mode, 16-token groups two rows per
    lane in the default numerics) against chunks of 32 on a one-layer 7B-shape
    model: chunk boundaries on multiples of 8 tokens leave every output's
    arithmetic unchanged, so logits, KV bytes and the ids that follow are
    bit-identical."""
    cfg = synth.dataclasses.replace(synth.LLAMA7B_1L, name="openllama-7b-v2-q4_0-1layer-whole", ctx=320)
    path = str(tmp_path / "m.gguf")
    synth.write_model(cfg, path, seed=43)
    prompt = synth.prompt_tokens(14, 256)
    runs = []
    for batch in (32, 256):
        m = capi.Model(path, ctx=320, act_mode=mode, max_batch=256)
        lg = m.prefill(prompt, batch)
        runs.append((lg.copy(), m.kv_bytes(), m.generate_greedy(5, 4).tolist()))
        m.close()
    (a, kb_a, ids_a), (b, kb_b, ids_b) = runs
    assert (bits(a) == bits(b)).all()
    assert (kb_a, ids_a) == (kb_b, ids_b)


@pytest.mark.parametrize("kind", ["token", "context"])
def test_pipelined_prefill_error_completes_earlier_chunks(tiny, kind):
    """An error raised in the third chunk while the first two still run on
    their streams (a bad token id, or the context running out): the call
    drains every stream before it raises, the two chunks before it complete
    (as in a chunk-by-chunk run), the position stops after them, and decoding
    from there on lane 0 equals decoding after a prefill of just those two
    chunks."""
    prompt = synth.prompt_tokens(4, 96)
    bad = prompt.copy()
    ctx = 256
    if kind == "token":
        bad[70] = 32000
    else:
        ctx = 80  # chunk 3 (positions 64..95) does not fit
    m = capi.Model(tiny, ctx=ctx, max_batch=32)
    with pytest.raises(capi.MvhError, match="token id out of range" if kind == "token" else "context exhausted"):
        m.prefill(bad, 32)
    assert m.position == 64
    got = m.forward(5)
    ref = capi.Model(tiny, ctx=ctx, max_batch=32)
    ref.prefill(prompt[:64], 32, logits=False)
    want = ref.forward(5)
    assert (bits(got) == bits(want)).all()
    m.close()
    ref.close()


@pytest.mark.parametrize("cfg_name", ["tinyllama-1.1b-mixed-2layer", "openllama-7b-v2-q4_0-1layer"])
@pytest.mark.parametrize("mode", [0, 1])
def test_large_shapes_vs_oracle(tmp_path, oracle, cfg_name, mode):
    cfg = synth.CONFIGS[cfg_name]
    path = str(tmp_path / "m.gguf")
    synth.write_model(cfg, path, seed=31)
    prompt = synth.prompt_tokens(8, 37)
    mo = oracle.model(path, ctx=256, force_q8=bool(mode))
    m = capi.Model(path, ctx=256, act_mode=mode, max_batch=32)
    close(m.prefill(prompt, 32), mo.prefill(prompt, 32), f"{cfg_name} prefill")
    cur = 5
    for _ in range(4):
        want = mo.forward(cur)
        got = m.forward(cur)
        close(got, want, f"{cfg_name} decode")
        assert int(np.argmax(got)) == int(np.argmax(want))
        cur = int(np.argmax(want))
    assert m.kv_bytes() == mo.kv_bytes()
    m.close()


@pytest.mark.parametrize("cfg_name,n_prompt", [("tiny-long", 600), ("openllama-7b-v2-q4_0-1layer-long", 530)])
def test_long_context_vs_oracle(tmp_path, oracle, cfg_name, n_prompt):
    """Positions past 512: the decode attention stages V in rounds of 512 rows."""
    base = synth.TINY if cfg_name.startswith("tiny") else synth.LLAMA7B_1L
    cfg = synth.dataclasses.replace(base, name=cfg_name, ctx=1024, layers=min(base.layers, 2))
    path = str(tmp_path / "m.gguf")
    synth.write_model(cfg, path, seed=17)
    prompt = synth.prompt_tokens(3, n_prompt)
    mo = oracle.model(path, ctx=1024, force_q8=True)
    m = capi.Model(path, ctx=1024, act_mode=1, max_batch=32)
    close(m.prefill(prompt, 32), mo.prefill(prompt, 32), f"{cfg_name} prefill")
    cur = 9
    for _ in range(3):
        want = mo.forward(cur)
        got = m.forward(cur)
        close(got, want, f"{cfg_name} decode")
        cur = int(np.argmax(want))
        assert int(np.argmax(got)) == cur
    m.close()


@pytest.mark.parametrize("max_batch,chunk", [(48, 45), (48, 17)])
def test_prefill_ragged_chunks_vs_oracle(tmp_path, oracle, max_batch, chunk):
    """Prefill chunks that are not multiples of the 16-token GEMM slabs or of the
    32-token attention groups (partial slabs and groups, two groups per chunk)."""
    cfg = synth.dataclasses.replace(synth.LLAMA7B_1L, name="openllama-7b-v2-q4_0-1layer-ragged", ctx=256)
    path = str(tmp_path / "m.gguf")
    synth.write_model(cfg, path, seed=23)
    prompt = synth.prompt_tokens(5, 100)
    mo = oracle.model(path, ctx=256, force_q8=True)
    m = capi.Model(path, ctx=256, act_mode=1, max_batch=max_batch)
    close(m.prefill(prompt, chunk), mo.prefill(prompt, chunk), f"prefill chunks of {chunk}")
    want = mo.forward(11)
    got = m.forward(11)
    close(got, want, "decode after ragged prefill")
    assert int(np.argmax(got)) == int(np.argmax(want))
    m.close()


KV_TYPES = {"f32": capi.MVH_KV_F32, "q8": capi.MVH_KV_Q8}


@pytest.mark.parametrize("cfg_name,mode", [("openllama-7b-v2-q4_0", 1), ("tinyllama-1.1b-mixed", 0),
                                           ("tinyllama-1.1b-mixed", 1)])
def test_full_depth_greedy_vs_oracle(tmp_path, oracle, cfg_name, mode):
    """Whole models at their full depth (the 32-layer OpenLLaMA-7B-v2 shape,
    the 22-layer TinyLlama-1.1B mixed shape) against the oracle: an 8-token
    prompt prefilled in one chunk, then 8 greedy decode steps on the device
    (the captured-graph loop) and on the host restatement.  Greedy ids must be
    identical; every step's logits within 1e-3 relative L2."""
    cfg = synth.CONFIGS[cfg_name]
    path = str(tmp_path / "m.gguf")
    synth.write_model(cfg, path, seed=41, device="cuda", digest=False)
    prompt = synth.prompt_tokens(13, 8)
    mo = oracle.model(path, ctx=256, force_q8=bool(mode), threads=16)
    m = capi.Model(path, ctx=256, act_mode=mode, max_batch=32)
    want = mo.prefill(prompt, 32)
    close(m.prefill(prompt, 32), want, f"{cfg_name} prefill")
    ids_ref, cur = [], int(np.argmax(want))
    for _ in range(8):
        ids_ref.append(cur)
        lg = mo.forward(cur)
        got = m.forward(cur)
        close(got, lg, f"{cfg_name} decode")
        cur = int(np.argmax(lg))
    ids_ref.append(cur)
    # the device loop from the same state: reset, prefill, generate
    m.reset()
    m.prefill(prompt, 32, logits=False)
    assert m.generate_greedy(ids_ref[0], 8).tolist() == ids_ref[1:]
    m.close()
    mo.close()


@pytest.fixture(scope="module")
def gqa(tmp_path_factory):
    """The 2-layer TinyLlama-shape mixed model of the GQA golden (32 heads, 4 KV heads)."""
    g = golden("model_gqa.npz")
    path = str(tmp_path_factory.mktemp("gqa") / "gqa.gguf")
    assert synth.write_model(synth.TINYLLAMA_MIXED_2L, path, seed=int(g["seed"])) == str(g["model_sha"])
    return path


@pytest.mark.parametrize("tname", ["f16", "q8"])
@pytest.mark.parametrize("mode", [0, 1])
def test_gqa_vs_reference_golden(gqa, tname, mode):
    """Grouped-query attention (query head h reads KV head h / 8,
    src/llama_model.cpp:248,256) against the compiled reference's own run:
    prefill logits of 40 tokens (32 + 8 chunks), six greedy ids, the last
    step's logits and KV bytes; then the captured-graph greedy loop."""
    g = golden("model_gqa.npz")
    key = f"{tname}_m{mode}"
    kt = capi.MVH_KV_F16 if tname == "f16" else capi.MVH_KV_Q8
    m = capi.Model(gqa, ctx=256, act_mode=mode, max_batch=32, kv_type=kt)
    close(m.prefill(g["prompt"], 32), g[f"prefill_logits_{key}"], f"GQA {key} prefill")
    ids, cur = [], 29
    for _ in range(6):
        lg = m.forward(cur)
        cur = int(np.argmax(lg))
        ids.append(cur)
    assert ids == g[f"decode_ids_{key}"].tolist()
    close(lg, g[f"decode_last_logits_{key}"], f"GQA {key} decode")
    assert m.kv_bytes() == int(g[f"kv_bytes_{key}"])
    m.reset()
    m.prefill(g["prompt"], 32, logits=False)
    assert m.generate_greedy(29, 6).tolist() == g[f"decode_ids_{key}"].tolist()
    m.close()


@pytest.mark.parametrize("tname", sorted(KV_TYPES))
@pytest.mark.parametrize("mode", [0, 1])
def test_tiny_kv_types_vs_reference_golden(tiny, tname, mode):
    """LlamaModel with kv_type F32 / Q8 (src/llama_model.cpp:16-56) against the
    compiled reference run with the same cache type."""
    g = golden("model_tiny.npz")
    m = capi.Model(tiny, ctx=256, act_mode=mode, max_batch=32, kv_type=KV_TYPES[tname])
    assert m.kv_type() == KV_TYPES[tname]
    close(m.prefill(g["prompt"], 32), g[f"kv{tname}_prefill_logits_m{mode}"], f"kv {tname} prefill")
    ids, cur = [], 17
    for _ in range(12):
        lg = m.forward(cur)
        cur = int(np.argmax(lg))
        ids.append(cur)
    assert ids == g[f"kv{tname}_decode_ids_m{mode}"].tolist()
    close(lg, g[f"kv{tname}_decode_last_logits_m{mode}"], f"kv {tname} decode")
    assert m.kv_bytes() == int(g[f"kv{tname}_kv_bytes_m{mode}"])
    # the captured-graph greedy loop runs the same cache type
    m.reset()
    m.prefill(g["prompt"], 32, logits=False)
    assert m.generate_greedy(17, 12).tolist() == g[f"kv{tname}_decode_ids_m{mode}"].tolist()
    m.close()


@pytest.mark.parametrize("tname", sorted(KV_TYPES))
@pytest.mark.parametrize("cfg_name", ["tinyllama-1.1b-mixed-2layer", "openllama-7b-v2-q4_0-1layer"])
def test_kv_types_large_shapes_vs_oracle(tmp_path, oracle, cfg_name, tname):
    """F32 / Q8 KV pages at the GQA and 7B shapes (prefill through the chunked
    attention kernels, decode through the two-kernel path)."""
    cfg = synth.CONFIGS[cfg_name]
    path = str(tmp_path / "m.gguf")
    synth.write_model(cfg, path, seed=41)
    prompt = synth.prompt_tokens(12, 45)
    kt = KV_TYPES[tname]
    mo = oracle.model(path, ctx=256, force_q8=True, kv_type=kt)
    m = capi.Model(path, ctx=256, act_mode=1, max_batch=32, kv_type=kt)
    close(m.prefill(prompt, 32), mo.prefill(prompt, 32), f"{cfg_name} kv {tname} prefill")
    cur = 7
    for _ in range(3):
        want = mo.forward(cur)
        got = m.forward(cur)
        close(got, want, f"{cfg_name} kv {tname} decode")
        cur = int(np.argmax(want))
        assert int(np.argmax(got)) == cur
    assert m.kv_bytes() == mo.kv_bytes()
    m.close()


@pytest.mark.parametrize("tname", ["f32", "f16", "q8"])
@pytest.mark.parametrize("cfg_name,page", [("tiny", 7), ("openllama-7b-v2-q4_0-1layer", 16)])
def test_page_sizes_vs_oracle(tmp_path, oracle, cfg_name, page, tname):
    """KV pages of 7 and 16 tokens (positions cross many page boundaries in
    one prefill chunk and in the V staging rounds) with every cache type."""
    kt = {"f32": capi.MVH_KV_F32, "f16": capi.MVH_KV_F16, "q8": capi.MVH_KV_Q8}[tname]
    cfg = synth.TINY if cfg_name == "tiny" else synth.CONFIGS[cfg_name]
    path = str(tmp_path / "m.gguf")
    synth.write_model(cfg, path, seed=57)
    prompt = synth.prompt_tokens(21, 70)
    mo = oracle.model(path, ctx=256, page=page, force_q8=True, kv_type=kt)
    m = capi.Model(path, ctx=256, page_tokens=page, act_mode=1, max_batch=32, kv_type=kt)
    close(m.prefill(prompt, 32), mo.prefill(prompt, 32), f"page {page} kv {tname} prefill")
    cur = 3
    for _ in range(3):
        want = mo.forward(cur)
        got = m.forward(cur)
        close(got, want, f"page {page} kv {tname} decode")
        cur = int(np.argmax(want))
        assert int(np.argmax(got)) == cur
    assert m.kv_bytes() == mo.kv_bytes()
    m.close()


@pytest.mark.parametrize("mode", [0, 1])
def test_f16_f32_weights_vs_oracle(tmp_path, oracle, mode):
    """A model with F16 attention/FFN matrices, an F16 embedding and an F32 output head (tensor_matvec's and
    tensor_matmul_batch's F16 / F32 branches; v06 falls back to tensor_matmul_batch for them)."""
    cfg = synth.dataclasses.replace(synth.TINY, name="tiny-f16-f32", wtype=synth.F16, embd_type=synth.F16,
                                    out_type=synth.F32, layers=2)
    path = str(tmp_path / "m.gguf")
    synth.write_model(cfg, path, seed=61)
    prompt = synth.prompt_tokens(4, 41)
    mo = oracle.model(path, ctx=256, force_q8=bool(mode))
    m = capi.Model(path, ctx=256, act_mode=mode, max_batch=32)
    close(m.prefill(prompt, 32), mo.prefill(prompt, 32), "f16/f32 prefill")
    cur = 19
    for _ in range(4):
        want = mo.forward(cur)
        got = m.forward(cur)
        close(got, want, "f16/f32 decode")
        cur = int(np.argmax(want))
        assert int(np.argmax(got)) == cur
    m.close()


_ATTN_CHILD = r"""
import sys, dataclasses
import numpy as np
sys.path.insert(0, sys.argv[1])
from memvanta_amd import capi, synth
from oracle.pyoracle import Oracle
o = Oracle()
for base, n_prompt in ((synth.LLAMA7B_1L, 300), (synth.TINYLLAMA_MIXED_2L, 270)):
    cfg = dataclasses.replace(base, name=base.name + "-ns", ctx=512)
    path = sys.argv[2] + "/" + cfg.name + ".gguf"
    synth.write_model(cfg, path, seed=29, digest=False)
    prompt = synth.prompt_tokens(6, n_prompt)
    mo = o.model(path, ctx=512, force_q8=True, threads=16)
    m = capi.Model(path, ctx=512, act_mode=1, max_batch=32)
    steps = [("prefill", lambda mm: mm.prefill(prompt, 32))] + [("decode", None)] * 3
    cur = 3
    for i, (what, fn) in enumerate(steps):
        if fn:
            want, got = fn(mo), fn(m)
        else:
            want, got = mo.forward(cur), m.forward(cur)
        rel = float(np.linalg.norm(got.astype(np.float64) - want) / np.linalg.norm(want.astype(np.float64)))
        same = float((got.view(np.uint32) == want.view(np.uint32)).mean())
        print(f"{cfg.name} {what} pos {n_prompt + i - 1}: rel {rel:.2e} bit-identical {same:.4f}", flush=True)
        assert rel <= 1e-3 and same >= 0.999 and int(np.argmax(got)) == int(np.argmax(want))
        cur = int(np.argmax(want))
    m.close()
    mo.close()
print("ok", flush=True)
"""


@pytest.mark.parametrize("override", ["MVH_ATTN_NS=1", "MVH_ATTN_NS=2", "MVH_ATTN_NS=0", "MVH_ATTN_SCORES_TILE=0",
                                      "MVH_L2_WARM=0", "MVH_L2_WARM=1,1,1,1,1"])
def test_attention_variants_vs_oracle(tmp_path, override):
    """The kernels the tuning overrides select, in a child process that sets
    the override before any GPU call: the fused F16 decode attention with 1 or
    2 slices per head (LDS-staged kernel) or 0 (the register-staged one) --
    the default, 4 at head_dim 128 and at 64 without a Q8 output (the GQA
    model's Q8_0 o projection), 2 at 64 otherwise, runs in every other model
    test --, the per-(head, token) prefill scores kernel in place of the
    K-tile one for F16 chunks of 8..32 tokens, and the decode step's L2
    warm-up of the GEMV weights off or at every site in full (the norm,
    attention and SwiGLU launches then carry warm-up workgroups over whole
    tensors).  Head dims 128 (MHA) and 64 (GQA 32/4), prefill chunks of 32
    ending in ragged ones (12 and 14 tokens), decode positions past 256 (a
    second staging round); the prefill's last logits and three decode steps
    against the oracle."""
    import os
    import subprocess
    import sys

    from conftest import ROOT

    key, val = override.split("=")
    env = dict(os.environ, **{key: val})
    p = subprocess.run([sys.executable, "-u", "-c", _ATTN_CHILD, ROOT, str(tmp_path)], env=env, capture_output=True,
                       text=True, timeout=110)
    assert p.returncode == 0 and p.stdout.strip().endswith("ok"), p.stdout + p.stderr
