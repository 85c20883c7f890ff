"""Whole models at their full depth against the reference compiled from its
own sources (golden vectors written by tests/golden/make_golden_deep.py):
the 22-layer TinyLlama-1.1B-shape mixed-quant model (GQA 32/4, Q8_0 attention
and FFN, Q6_K ffn_down and output) and the 32-layer OpenLLaMA-7B-v2-shape
Q4_0 model (Q6_K output), each in both prefill numerics (default and
MEMVANTA_FORCE_Q8_ACT=1): a 128-token seed prefill in chunks of 32 (seeded
uniform ids), then 32 greedy decode steps from token 17 at positions
128..159 (src/llama_model.cpp:240-259; the tg protocol of
benchmarks/real_model_bench.cpp:22).

Greedy ids must be identical at every step; logits within 1e-3 relative L2
with >= 99.9% of them bit-identical (the seed prefill's last token, the
first and the last decode step in full; every step at 1024 fixed vocabulary
entries, where >= 99% must be bit-identical); KV bytes equal; then the
device-resident greedy loop from the same state gives the same ids.  The
model files are byte-identical to the ones the golden run used (sha256)."""
import os

import numpy as np
import pytest

from conftest import bits, golden
from memvanta_amd import capi, synth

pytestmark = pytest.mark.gpu

CASES = {"deep_tinyllama_mixed": synth.TINYLLAMA_MIXED, "deep_openllama_7b": synth.LLAMA7B}


def rel_l2(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(np.asarray(b, np.float64)))


def close(got, want, what, exact_frac=0.999):
    r = rel_l2(got, want)
    assert r <= 1e-3, f"{what}: rel L2 {r}"
    frac = float((bits(got) == bits(want)).mean())
    assert frac >= exact_frac, f"{what}: only {frac:.4f} bit-identical (rel L2 {r:.2e})"


@pytest.fixture(scope="module", params=sorted(CASES))
def deep(request, tmp_path_factory):
    fix = request.param
    g = golden(f"{fix}.npz")
    path = str(tmp_path_factory.mktemp(fix) / "m.gguf")
    print(f"writing {fix}", flush=True)
    assert synth.write_model(CASES[fix], path, seed=int(g["model_seed"]), blocks="random") == str(g["model_sha"])
    yield fix, path, g
    os.unlink(path)


@pytest.mark.parametrize("mode", [0, 1])
def test_full_depth_seed128_decode32_vs_reference_golden(deep, mode):
    fix, path, g = deep
    print(f"{fix} mode {mode}", flush=True)
    first, sub = int(g["first_token"]), g["subset"]
    want_ids = g[f"ids_m{mode}"].tolist()
    m = capi.Model(path, ctx=int(g["ctx"]), act_mode=mode, max_batch=32)
    try:
        close(m.prefill(g["prompt"], 32), g[f"prefill_logits_m{mode}"], f"{fix} m{mode} seed prefill")
        ids, cur = [], first
        for i in range(len(want_ids)):
            lg = m.forward(cur)
            close(lg[sub], g[f"step_subset_m{mode}"][i], f"{fix} m{mode} decode step {i} (subset)", 0.99)
            if i == 0:
                close(lg, g[f"first_logits_m{mode}"], f"{fix} m{mode} first decode step")
            cur = int(np.argmax(lg))
            ids.append(cur)
            assert ids == want_ids[:i + 1], f"{fix} m{mode}: greedy ids differ at step {i}: {ids} vs {want_ids}"
        close(lg, g[f"last_logits_m{mode}"], f"{fix} m{mode} last decode step")
        assert m.kv_bytes() == int(g[f"kv_bytes_m{mode}"])
        m.reset()
        m.prefill(g["prompt"], 32, logits=False)
        assert m.generate_greedy(first, len(want_ids)).tolist() == want_ids
    finally:
        m.close()
