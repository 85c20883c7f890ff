"""Golden vectors of whole models at their full depth, from the reference
compiled from its own sources (oracle/_ref/libmvref.so, built by oracle/Makefile).

For the TinyLlama-1.1B-shape mixed-quant model (22 layers, GQA 32/4, Q8_0
attention / FFN, Q6_K ffn_down and output) and the OpenLLaMA-7B-v2-shape Q4_0
model (32 layers, MHA, Q6_K output), both written by
synth.write_model(..., blocks="random") (valid blocks drawn as bytes: the same
file on every host, in seconds), and for both prefill numerics (the default
and MEMVANTA_FORCE_Q8_ACT=1):

* a 128-token seed prefill in chunks of 32 (seeded uniform ids) with its
  last-token logits;
* 32 greedy decode steps from token 17 (LlamaModel::forward + argmax, as
  benchmarks/real_model_bench.cpp:22 runs them) at positions 128..159: every
  step's id, every step's logits at SUBSET fixed vocabulary entries, and the
  full logits of the first and the last step.

Only these arrays and the model file's sha256 are stored (no reference source
text).  Run from the repository root:

    python tests/golden/make_golden_deep.py [workdir]      # workdir: where the model files go (/dev/shm)
"""
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from memvanta_amd import synth  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
CTX, BATCH, SEED_TOKENS, STEPS, FIRST = 768, 32, 128, 32, 17
SUBSET = 1024
# (fixture, config, model seed, prompt seed)
MODELS = [("deep_tinyllama_mixed", synth.TINYLLAMA_MIXED, 11, 111),
          ("deep_openllama_7b", synth.LLAMA7B, 12, 112)]


def subset_index(vocab: int) -> np.ndarray:
    return np.sort(np.random.default_rng(4242).choice(vocab, SUBSET, replace=False)).astype(np.int32)


def run(ref, path, prompt, force_q8, threads):
    m = ref.model(path, ctx=CTX, threads=threads, force_q8=force_q8)
    try:
        pre = m.prefill(prompt, BATCH, logits=True).copy()
        ids, lgs, cur = [], [], FIRST
        for _ in range(STEPS):
            lg = m.forward(cur).copy()
            cur = int(np.argmax(lg))
            ids.append(cur)
            lgs.append(lg)
        return pre, np.array(ids, np.int32), np.stack(lgs), m.kv_bytes()
    finally:
        m.close()


def main():
    from oracle.pyoracle import Ref, ref_available

    if not ref_available():
        sys.exit("oracle/_ref/libmvref.so is not built (python -m memvanta_amd.build --all)")
    work = sys.argv[1] if len(sys.argv) > 1 else "/dev/shm"
    threads = len(os.sched_getaffinity(0))
    ref = Ref()
    for fix, cfg, mseed, pseed in MODELS:
        path = os.path.join(work, f"{fix}.gguf")
        t0 = time.time()
        sha = synth.write_model(cfg, path, seed=mseed, blocks="random")
        print(f"{fix}: model written ({time.time() - t0:.0f} s)", flush=True)
        prompt = synth.prompt_tokens(pseed, SEED_TOKENS, cfg.vocab)
        sub = subset_index(cfg.vocab)
        out = {"model_sha": np.array(sha), "model_seed": np.array(mseed), "prompt": prompt, "subset": sub,
               "first_token": np.array(FIRST), "ctx": np.array(CTX)}
        for mode in (0, 1):
            t0 = time.time()
            pre, ids, lgs, kvb = run(ref, path, prompt, bool(mode), threads)
            out[f"prefill_logits_m{mode}"] = pre
            out[f"ids_m{mode}"] = ids
            out[f"step_subset_m{mode}"] = lgs[:, sub]
            out[f"first_logits_m{mode}"] = lgs[0]
            out[f"last_logits_m{mode}"] = lgs[-1]
            out[f"kv_bytes_m{mode}"] = np.array(kvb, np.uint64)
            print(f"{fix} mode {mode}: ids {ids[:8].tolist()}... ({time.time() - t0:.0f} s)", flush=True)
        np.savez_compressed(os.path.join(HERE, f"{fix}.npz"), **out)
        os.unlink(path)


if __name__ == "__main__":
    main()
