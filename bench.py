#!/usr/bin/env python3
"""Benchmark of MemVanta's quantized-matmul + paged-F16-attention hot path on one MI355X.

Workload (the headline): an OpenLLaMA-7B-v2-shape random-init model (dim 4096,
FFN 11008, 32 layers, 32 heads (MHA), vocab 32000; attention/FFN/embedding
Q4_0, output Q6_K; weights N(0, 0.02), drawn and quantized on the device),
ctx 768, batch 32, paged F16 KV (128-token pages) -- the protocol of the
reference's real_model_bench (benchmarks/real_model_bench.cpp:20-27):

* tg128: reset, prefill a 128-token seed (untimed), then 128 greedy decode
  tokens from token 17, timed -- the reference's tg rep.  One step = one whole
  tg128 rep; the 128 tokens run as the device-resident greedy loop (captured
  HIP graphs of eight decode steps, argmax on the device) at positions 128..255.
  `value` = 128 * K / (the K reps' decode seconds) (tok/s); `ms_per_step` =
  the mean decode time of one rep.  The per-call API rate (forward() + host
  argmax, as the reference's loop does) is reported beside it.
* pp512: reset, prefill 512 prompt ids in chunks of 32 with last-token
  logits (tensor_matmul_batch_v06 numerics, MEMVANTA_FORCE_Q8_ACT=1 mode), and
  the same with the default prefill numerics (no MEMVANTA_FORCE_Q8_ACT), the
  numerics of the reference's published pp512.
* prompt and seed ids are seeded uniform in [0, vocab) (the 7B config's
  protocol); one more tg128 rep seeded with the reference bench's
  fixed_tokens ((i*1543+17) % vocab) is reported beside it.
* the same tg and pp512 are timed beside it with F32 and Q8 KV pages
  (LlamaModel's kv_type) and reported under config.other_kv_cache_types.

The tiny config (dim 288, 6 layers, pp128/tg32, ctx 256) and the
TinyLlama-1.1B-shape mixed-quant config (Q8_0 attention/FFN, Q6_K ffn_down and
output, GQA 32/4, pp512/tg128, ctx 768) run the same way with seeded uniform
prompt ids and are reported under config.other_models.

`roofline` times the dominant kernel, the Q4_0 x Q8 decode GEMV, alone at the
launches of one 7B decode layer (q|k|v fused [4096->12288], o [4096->4096],
gate|up fused [4096->22016], down [11008->4096]; the isolated-GEMV shapes
[4096->4096], [4096->11008], [11008->4096], [4096->32000] are timed beside),
with HIP events on the backend's stream over graph replays that rotate weight
copies (at least 640 MB between two uses of one copy, more than the 256 MB
Infinity Cache) so every launch streams its weights from HBM; the prefill GEMM
timing rotates copies the same way.  The measured read ceiling is the
library's streaming-read probe over 1 GiB buffers (two, alternated).

`cpu_baseline` runs in a child process that never loads the HIP runtime: the
reference compiled from its sources (oracle/_ref/libmvref.so, kind
"reference"), or the C restatement (kind "port") when that library is absent,
on the same GGUF files, with the reference's OpenMP placement
(OMP_PROC_BIND=close, OMP_PLACES=cores): the 128-token seed prefill (default
numerics, the numerics of the published figures; the reference's FORCE_Q8
prefill is about 3x slower on the CPU) and the decode positions of the GPU
run, its greedy ids compared with those of the GPU after the same
default-numerics prefill, a FORCE_Q8 prefill sample, the isolated
tensor_matvec / tensor_matmul_batch_v06 at the GEMV / GEMM config shapes on
the same weight bytes, a 4-thread sample (the published figures' thread
count), the other two models' seed prefill + decode with their ids compared,
and lscpu.
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "tg128 tok/s + achieved HBM GB/s (7B-shape Q4_0); pp512 prefill tok/s"
HBM_PEAK_GBS = 8000.0
CTX, BATCH, PAGE, SEED_TOKENS, PROMPT_TOKENS, FIRST_TOKEN = 768, 32, 128, 128, 512, 17
TG_TOKENS = 128          # decode tokens of one tg rep (tg128)
PROMPT_SEED_7B = 2026    # seed of the 7B model's uniform prompt / seed ids
# per-layer decode GEMV launches of the 7B shape (K, N, launches per layer)
DECODE_GEMVS = [(4096, 12288, 1), (4096, 4096, 1), (4096, 22016, 1), (11008, 4096, 1)]
GEMV_CONFIG = [(4096, 4096), (4096, 11008), (11008, 4096), (4096, 32000)]  # the isolated-GEMV config (K, N)
ISOLATED_GEMVS = GEMV_CONFIG + [(4096, 12288), (4096, 22016)]
PREFILL_GEMMS = [(4096, 4096), (4096, 11008), (11008, 4096)]  # (K, N) of the GEMM config
PREFILL_M = [32, 128, 512]
INT8_PEAK_TOPS = 5000.0  # dense int8 MFMA, MI355X
# names the config matrices carry in the GGUF the CPU leg reads (the name picks
# the reference's FFN / attention accumulator layout in default numerics)
MATRIX_NAMES = {(4096, 4096): "blk.0.attn_q.weight", (4096, 11008): "blk.0.ffn_up.weight",
                (11008, 4096): "blk.0.ffn_down.weight", (4096, 32000): "output.weight"}
MATRIX_SEED, ACT_SEED = 1234, 99
REF_TG128_TOKS = 1.52  # published reference tg128, OpenLLaMA-7B-v2 Q4_0, 4-thread Xeon 8573C, ctx 768
REF_PP512_TOKS = 3.15  # published reference pp512, same run (default prefill numerics)
# the other model configs: (name, synth config, ctx, pp tokens, seed tokens, tg tokens, prompt seed)
# and the CPU leg's (seed tokens, decode tokens) for it
OTHER_MODELS = [("tiny pp128/tg32", "tiny-llama-288", 256, 128, 128, 32, 2024, (128, 32)),
                ("TinyLlama-1.1B-shape mixed quant pp512/tg128", "tinyllama-1.1b-mixed", 768, 512, 128, 128, 2025,
                 (8, 6))]
CPU_TG_TOKENS_7B, CPU_PP_FORCE_Q8_TOKENS, CPU_SEED_4_THREADS, CPU_TG_4_THREADS = 32, 32, 32, 6


def log(msg: str) -> None:
    print(f"bench: {msg}", file=sys.stderr, flush=True)


def fixed_tokens(n: int, vocab: int):
    import numpy as np

    return ((np.arange(n, dtype=np.int64) * 1543 + 17) % vocab).astype(np.int32)


def gemv_bytes(k: int, n: int) -> int:
    """Algorithmic bytes of one Q4_0 x Q8 GEMV: Q4_0 weights + int8 act + f32 scales + f32 out."""
    return n * (k // 32) * 18 + k + 4 * (k // 32) + 4 * n


def model_weight_bytes(cfg, synth) -> int:
    """Bytes of every matrix a decode token reads (the embedding contributes one row)."""
    D, F, kv = cfg.dim, cfg.ffn, cfg.kv_heads * cfg.head_dim
    rb = synth.row_bytes
    per_layer = (D * rb(cfg.wtype, D) + 2 * kv * rb(cfg.wtype, D) + D * rb(cfg.wtype, D)
                 + 2 * F * rb(cfg.wtype, D) + D * rb(cfg.down_type or cfg.wtype, F) + 2 * 4 * D)
    return cfg.layers * per_layer + cfg.vocab * rb(cfg.out_type, D) + rb(cfg.embd_type, D) + 4 * D


def kv_read_bytes(cfg, first_pos: int, n: int) -> int:
    """F16 K and V bytes read by n decode steps starting at position first_pos."""
    kv = cfg.kv_heads * cfg.head_dim
    positions = sum(p + 1 for p in range(first_pos, first_pos + n))
    return cfg.layers * 2 * kv * 2 * positions


def rotation_copies(nbytes: int, rotate_mb: float) -> int:
    """Weight copies whose rotation streams at least rotate_mb MB between two
    uses of one copy (more than the 256 MB Infinity Cache: cold-HBM timing)."""
    return max(2, -(-int(rotate_mb * 1e6) // nbytes))


# ---------------------------------------------------------------- GPU side

def make_matrices():
    """Q4_0 weights N(0, 0.02) of every isolated shape, drawn and quantized on the device."""
    import torch

    from memvanta_amd import synth

    gen = torch.Generator(device="cuda")
    gen.manual_seed(MATRIX_SEED)
    return {(k, n): synth.quantize_torch(synth.Q4_0, torch.randn((n, k), generator=gen, device="cuda") * 0.02)
            .cpu().numpy() for k, n in ISOLATED_GEMVS}


def time_gemv_kernels(ctx, mats, launches: int, rotate_mb: float):
    """Average duration of the Q4_0 x Q8 GEMV kernel per shape (HIP events, graph replays)."""
    import numpy as np
    import torch

    from memvanta_amd import synth

    stream = torch.cuda.ExternalStream(ctx.stream)
    rng = np.random.default_rng(ACT_SEED)
    out = {}
    for k, n in ISOLATED_GEMVS:
        w = mats[(k, n)]
        copies = rotation_copies(w.nbytes, rotate_mb)
        ts = [ctx.upload("blk.0.attn_q.weight", synth.Q4_0, k, n, w) for _ in range(copies)]
        x = torch.from_numpy(synth.activations(rng, 1, k)[0]).cuda()
        q = torch.empty(k, dtype=torch.int8, device="cuda")
        d = torch.empty(k // 32, dtype=torch.float32, device="cuda")
        y = torch.empty(n, dtype=torch.float32, device="cuda")
        ctx.quantize_q8(x, q, d)
        ctx.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for i in range(launches):
                ctx.matvec_q8(ts[i % copies], q, d, y)
        ctx.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            g.replay()
            a.record(stream)
            for _ in range(3):
                g.replay()
            b.record(stream)
        b.synchronize()
        out[(k, n)] = a.elapsed_time(b) * 1e3 / (3 * launches)
        del g
        for t in ts:
            t.free()
    return out


def time_gemm_streams(ctx, ts, x, reps: int, lanes: int) -> float:
    """us per GEMM with `lanes` independent chains of reps GEMMs (own context, stream and
    output each) started together: the prefill's operating point, where consecutive chunks
    run on three streams and their M = 32 GEMMs overlap."""
    import torch

    from memvanta_amd import capi

    ctxs = [ctx] + [capi.Context(ctx.device) for _ in range(lanes - 1)]
    streams = [torch.cuda.ExternalStream(c.stream) for c in ctxs]
    ys = [torch.empty((x.shape[0], ts[0].ne1), dtype=torch.float32, device="cuda") for _ in ctxs]
    for c, y in zip(ctxs, ys):
        c.matmul_batch_v06(ts[0], x, capi.MVH_ACT_Q8, y=y)  # warm-up (each context's quantizer scratch)
        c.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(streams[0])
    for st in streams[1:]:
        st.wait_event(start)
    for r in range(reps):
        for i, (c, y) in enumerate(zip(ctxs, ys)):
            c.matmul_batch_v06(ts[(r * lanes + i) % len(ts)], x, capi.MVH_ACT_Q8, y=y)
    for st in streams[1:]:
        done = torch.cuda.Event()
        done.record(st)
        streams[0].wait_event(done)
    stop.record(streams[0])
    stop.synchronize()
    for c in ctxs[1:]:
        c.close()
    return start.elapsed_time(stop) * 1e3 / (reps * lanes)


def time_prefill_gemm(ctx, mats, reps: int, rotate_mb: float):
    """Q4_0 x Q8 prefill GEMM (int8 MFMA) at the GEMM config shapes: us, TOP/s, GB/s."""
    import numpy as np
    import torch

    from memvanta_amd import capi, synth

    stream = torch.cuda.ExternalStream(ctx.stream)
    rng = np.random.default_rng(5)
    out = []
    for k, n in PREFILL_GEMMS:
        w = mats[(k, n)]
        ts = [ctx.upload("blk.0.ffn_up.weight", synth.Q4_0, k, n, w) for _ in range(rotation_copies(w.nbytes, rotate_mb))]
        for m in PREFILL_M:
            x = torch.from_numpy(synth.activations(rng, m, k)).cuda()
            y = torch.empty((m, n), dtype=torch.float32, device="cuda")
            ctx.matmul_batch_v06(ts[0], x, capi.MVH_ACT_Q8, y=y)  # warm-up (includes the activation quantizer)
            ctx.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            with torch.cuda.stream(stream):
                a.record(stream)
                for r in range(reps):
                    ctx.matmul_batch_v06(ts[r % len(ts)], x, capi.MVH_ACT_Q8, y=y)
                b.record(stream)
            b.synchronize()
            us = a.elapsed_time(b) * 1e3 / reps
            ops = 2.0 * m * n * k
            byts = n * (k // 32) * 18 + m * (k + k // 8) + 4 * m * n
            e = {"K": k, "N": n, "M": m, "us": round(us, 2), "TOP/s": round(ops / us / 1e6, 2),
                 "frac_int8_peak": round(ops / us / 1e6 / INT8_PEAK_TOPS, 4), "GB/s": round(byts / us / 1e3, 1)}
            if m == BATCH:
                e["us_per_gemm_3_streams"] = round(time_gemm_streams(ctx, ts, x, reps, 3), 2)
            out.append(e)
        for t in ts:
            t.free()
    return out


def measure_hbm(ctx, nbytes: int = 1 << 30, reps: int = 8):
    """Measured device ceilings in GB/s: the library's streaming-read probe
    (mvh_stream_read) alternating over two nbytes buffers, so every pass reads
    nbytes that the previous pass did not touch (cold beyond the 256 MB
    Infinity Cache), and a device-to-device copy of nbytes (torch's copy
    kernel; read + write bytes)."""
    import torch

    stream = torch.cuda.ExternalStream(ctx.stream)
    bufs = [torch.full((nbytes,), 1, dtype=torch.uint8, device="cuda") for _ in range(2)]
    sink_words = 1 << 20
    sink = torch.zeros(sink_words, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    ctx.stream_read(bufs[1], nbytes, sink, sink_words)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        a.record(stream)
        for r in range(reps):
            ctx.stream_read(bufs[r % 2], nbytes, sink, sink_words)
        b.record(stream)
    b.synchronize()
    read_s = a.elapsed_time(b) * 1e-3 / reps
    src, dst = bufs
    dst.copy_(src)
    torch.cuda.synchronize()
    c, d = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    c.record()
    for _ in range(reps):
        dst.copy_(src)
    d.record()
    d.synchronize()
    copy_s = c.elapsed_time(d) * 1e-3 / reps
    del bufs, src, dst, sink
    return {"read": nbytes / read_s / 1e9, "read_us": read_s * 1e6, "copy": 2 * nbytes / copy_s / 1e9}


def measure_node_floor(ctx, launches: int = 200):
    """Cost of a near-empty node in a HIP graph: mvh_stream_read of 16 bytes
    (one workgroup, one load) replayed as a graph of `launches` nodes; the
    per-node time is the floor every dependent kernel of a decode step pays.
    Under rocprofv3 --kernel-trace the same launches show the trace's own
    per-dispatch floor."""
    import torch

    stream = torch.cuda.ExternalStream(ctx.stream)
    buf = torch.zeros(16, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(2048, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for _ in range(launches):
            ctx.stream_read(buf, 16, sink, sink.numel())
    ctx.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        g.replay()
        a.record(stream)
        for _ in range(3):
            g.replay()
        b.record(stream)
    b.synchronize()
    us = a.elapsed_time(b) * 1e3 / (3 * launches)
    del g
    return us


# exact FORCE_Q8 chain: 3 VALU lane-operations per (output, block) -- the
# int-to-float conversion of the block sum, the scale product d_w * d_a and the
# fma (no packed FP32); MI355X: 256 CUs x 64 lanes x 2.4 GHz
VALU_LANE_OPS_PER_S = 256 * 64 * 2.4e9


def prefill_roofline(gemm):
    """Roofline entries of the prefill GEMM: at M = 512 (4096 x 4096) the
    exact chain's VALU floor; at M = 32 the HBM bound of its weight bytes."""
    out = {}
    for e in gemm:
        k, n, m = e["K"], e["N"], e["M"]
        if (k, n) != (4096, 4096) or m not in (32, 512):
            continue
        floor_us = 3.0 * m * n * (k // 32) / VALU_LANE_OPS_PER_S * 1e6
        hbm_us = (n * (k // 32) * 18 + m * (k + k // 8) + 4 * m * n) / (HBM_PEAK_GBS * 1e3)
        out[f"M{m}"] = {"shape": f"{k}->{n}", "us": e["us"], "valu_floor_us": round(floor_us, 2),
                        "frac_of_valu_floor": round(floor_us / e["us"], 4), "hbm_bound_us": round(hbm_us, 2),
                        "frac_of_hbm_bound": round(hbm_us / e["us"], 4), "frac_int8_peak": e["frac_int8_peak"]}
    out["basis"] = ("VALU floor: 3 lane-operations per output-block (cvt, d_w*d_a, fma) at 256 CUs x 64 lanes x "
                    "2.4 GHz; HBM bound: the GEMM's algorithmic bytes at 8 TB/s; us includes the activation "
                    "quantizer launch")
    return out


def time_pp(m, prompt, reps: int = 1, batch: int = BATCH):
    """Prefill rate of prompt (chunks of `batch`, last-token logits) after one untimed run."""
    import torch

    m.reset()
    m.prefill(prompt, batch, logits=True)
    out = []
    for _ in range(reps):
        m.reset()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        m.prefill(prompt, batch, logits=True)
        torch.cuda.synchronize()
        out.append(len(prompt) / (time.perf_counter() - t0))
    return out


def pp_whole_prompt(m, prompt, reps: int):
    """The prompt as one prefill batch (every GEMM at M = len(prompt)): rate,
    and whether its last-token logits are bit-identical to chunks of BATCH
    (they are when the chunk boundaries fall on multiples of 8 tokens: every
    output then takes the same batch4/batch8 or FORCE_Q8 arithmetic)."""
    import numpy as np

    m.reset()
    ref = np.array(m.prefill(prompt, BATCH, logits=True), copy=True)
    rates = time_pp(m, prompt, reps, batch=len(prompt))
    m.reset()
    got = np.array(m.prefill(prompt, len(prompt), logits=True), copy=True)
    return rates, bool(np.array_equal(got.view(np.uint32), ref.view(np.uint32)))


def tg_reps(m, seed, gen: int, reps: int, warmup: int):
    """The reference bench's tg rep (benchmarks/real_model_bench.cpp:22):
    reset, untimed prefill of `seed` in chunks of BATCH, then `gen` greedy
    tokens from token 17 timed, here as the device-resident loop.  `warmup`
    untimed reps first (the first captures the decode graph), then `reps`
    timed ones.  Returns the per-rep wall seconds (between device
    synchronizations), the per-rep device seconds (HIP events on the model's
    stream around the decode), the ids of the last rep and whether every rep
    produced the same ids."""
    import torch

    stream = torch.cuda.ExternalStream(m.stream)
    wall, dev, first = [], [], None
    same = True
    ids = []
    for r in range(warmup + reps):
        m.reset()
        m.prefill(seed, BATCH, logits=False)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        with torch.cuda.stream(stream):
            e0.record(stream)
        ids = [int(i) for i in m.generate_greedy(FIRST_TOKEN, gen)]
        with torch.cuda.stream(stream):
            e1.record(stream)
        torch.cuda.synchronize()
        t = time.perf_counter() - t0
        if first is None:
            first = ids
        same = same and ids == first
        if r >= warmup:
            wall.append(t)
            dev.append(e0.elapsed_time(e1) * 1e-3)
    return wall, dev, ids, same


def time_tg(m, seed, gen: int, reps: int, warmup: int):
    """tg<gen> rate over `reps` timed reps: (tok/s, ids of the last rep)."""
    wall, _, ids, _ = tg_reps(m, seed, gen, reps, warmup)
    return gen * len(wall) / sum(wall), ids


def default_numerics_run(path: str, prompt, ctx_len: int, seed, n_ids: int, logits_path: str | None = None):
    """pp with tensor_matmul_batch_v06's default numerics (no
    MEMVANTA_FORCE_Q8_ACT: fp32 activations, batch8 / batch4 accumulators),
    and the greedy ids of n_ids decode steps after a default-numerics prefill
    of seed (the CPU leg's protocol, for the id comparison): forward() with the
    host argmax, each step's logits saved to logits_path (.npy, [n_ids][vocab])
    for the CPU leg's logits comparison; then the device-resident loop from the
    same state, whose ids must equal those.  Returns (pp tok/s, ids, pp as one
    batch tok/s, its logits equal to chunks of 32, graph ids equal)."""
    import numpy as np

    from memvanta_amd import capi

    m = capi.Model(path, ctx=ctx_len, page_tokens=PAGE, act_mode=capi.MVH_ACT_REF, max_batch=len(prompt))
    try:
        pp = time_pp(m, prompt)[0]
        whole, same = pp_whole_prompt(m, prompt, 1)
        m.reset()
        m.prefill(seed, BATCH, logits=False)
        ids, lgs, cur = [], [], FIRST_TOKEN
        for _ in range(n_ids):
            lg = np.array(m.forward(cur), dtype=np.float32, copy=True)
            cur = int(np.argmax(lg))
            ids.append(cur)
            lgs.append(lg)
        if logits_path:
            np.save(logits_path, np.stack(lgs))
        m.reset()
        m.prefill(seed, BATCH, logits=False)
        graph_same = [int(i) for i in m.generate_greedy(FIRST_TOKEN, n_ids)] == ids
        return pp, ids, whole[0], same, graph_same
    finally:
        m.close()


def time_kv_types(path: str, seed, prompt, reps: int, warmup: int):
    """tg128 and pp512 of the same model with the F32 and Q8 KV cache types
    (LlamaModel's kv_type; decode attention then runs as RoPE + KV write +
    scores + softmax-V launches instead of the fused F16 kernel)."""
    from memvanta_amd import capi

    out = []
    for kt in (capi.MVH_KV_F32, capi.MVH_KV_Q8):
        m = capi.Model(path, ctx=CTX, page_tokens=PAGE, act_mode=capi.MVH_ACT_Q8, max_batch=BATCH, kv_type=kt)
        pp = time_pp(m, prompt)[0]
        tg, ids = time_tg(m, seed, TG_TOKENS, reps, warmup)
        out.append({"kv": capi.kv_type_name(kt), "tg128_tok_s": round(tg, 2), "tg128_reps": reps,
                    "pp512_tok_s": round(pp, 1), "kv_bytes_after_tg": m.kv_bytes(), "greedy_ids_head": ids[:4]})
        m.close()
    return out


def time_other_model(tmpdir: str, label: str, cfg_name: str, ctx_len: int, pp_n: int, seed_n: int, tg_n: int,
                     prompt_seed: int, cpu_run, reps: int, warmup: int):
    """pp / tg of one of the other model configs (random-init, written on the device)."""
    import torch

    from memvanta_amd import capi, synth

    cfg = synth.CONFIGS[cfg_name]
    path = os.path.join(tmpdir, f"{cfg_name}.gguf")
    synth.write_model(cfg, path, seed=prompt_seed, device="cuda", digest=False)
    torch.cuda.synchronize()
    prompt = synth.prompt_tokens(prompt_seed, pp_n, cfg.vocab)
    seed = prompt[:seed_n]
    m = capi.Model(path, ctx=ctx_len, page_tokens=PAGE, act_mode=capi.MVH_ACT_Q8, max_batch=BATCH)
    try:
        pp = time_pp(m, prompt, reps=3)
        tg, ids = time_tg(m, seed, tg_n, reps, warmup)
    finally:
        m.close()
    cpu_seed, cpu_tg = cpu_run
    lg_path = os.path.join(tmpdir, f"{cfg_name}_gpu_logits.npy")
    pp_default, ref_ids, _, _, graph_same = default_numerics_run(path, prompt, ctx_len, prompt[:cpu_seed], cpu_tg,
                                                                 lg_path)
    res = {"workload": f"{label}: {cfg.name} (dim {cfg.dim}, FFN {cfg.ffn}, {cfg.layers} layers, "
                       f"{cfg.heads}/{cfg.kv_heads} heads, vocab {cfg.vocab}), ctx {ctx_len}, batch {BATCH}, "
                       f"paged F16 KV, prompt ids uniform from seed {prompt_seed}",
           "pp_tokens": pp_n, "pp_tok_s": round(sum(pp) / len(pp), 1), "pp_tok_s_reps": [round(v, 1) for v in pp],
           "pp_default_numerics_tok_s": round(pp_default, 1),
           "tg_tokens": tg_n, "tg_after_seed_tokens": seed_n, "tg_reps": reps, "tg_tok_s": round(tg, 2),
           "greedy_ids_head": ids[:8], "graph_ids_equal_forward_ids": graph_same}
    spec = {"path": path, "ctx": ctx_len, "seed_ids": [int(t) for t in prompt[:cpu_seed]], "tg_tokens": cpu_tg,
            "gpu_logits": lg_path}
    return res, spec, ref_ids


# ---------------------------------------------------------------- CPU side (child process)

def _lscpu() -> dict:
    keys = ("Model name", "Socket(s)", "Core(s) per socket", "Thread(s) per core", "CPU(s)", "NUMA node(s)",
            "L3 cache", "Flags")
    try:
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
    except (OSError, subprocess.SubprocessError):
        return {"lscpu": "unavailable"}
    out = {}
    for line in txt.splitlines():
        k, _, v = line.partition(":")
        if k.strip() in keys:
            v = v.strip()
            if k.strip() == "Flags":
                v = " ".join(f for f in ("avx2", "fma", "f16c", "avx512f", "avx512_vnni", "amx_int8")
                             if f in v.split())
                k = "Flags (relevant)"
            out[k.strip()] = v
    return out


def _logits_vs_gpu(cpu_logits, gpu_path):
    """Per-step logits of the CPU run against the GPU's saved ones: the largest
    relative L2 difference and the smallest bit-identical fraction over the
    steps both ran."""
    import numpy as np

    g = np.load(gpu_path, allow_pickle=False)
    n = min(len(cpu_logits), len(g))
    rels, fracs = [], []
    for c, x in zip(cpu_logits[:n], g[:n]):
        c64 = np.asarray(c, np.float64)
        rels.append(float(np.linalg.norm(np.asarray(x, np.float64) - c64) / np.linalg.norm(c64)))
        fracs.append(float((np.asarray(c, np.float32).view(np.uint32) == np.asarray(x, np.float32).view(np.uint32))
                           .mean()))
    return {"logits_steps_compared": n, "logits_max_rel_l2": max(rels) if rels else None,
            "logits_min_bit_identical_frac": round(min(fracs), 6) if fracs else None}


def _cpu_model_run(lib, path, ctx_len, threads, seed_ids, n_tg, force_q8=False, warm_chunk=True, gpu_logits=None):
    """Seed prefill + greedy decode on the CPU model: pp tok/s, tg tok/s, ids.
    One untimed chunk first touches every weight page.  With gpu_logits (a
    .npy of the GPU's per-step decode logits from the same state), every
    step's logits are compared with the GPU's after the timing."""
    import numpy as np

    m = lib.model(path, ctx=ctx_len, page=PAGE, threads=threads, force_q8=force_q8)
    keep = []
    try:
        if warm_chunk:
            m.prefill(seed_ids[:BATCH], BATCH, logits=False)
            m.reset()
        t0 = time.perf_counter()
        m.prefill(seed_ids, BATCH, logits=False)
        pp_s = time.perf_counter() - t0
        ids, cur = [], FIRST_TOKEN
        lg = m.forward(cur)  # first decode step: untimed
        cur = int(np.argmax(lg))
        ids.append(cur)
        if gpu_logits:
            keep.append(np.array(lg, np.float32, copy=True))
        t0 = time.perf_counter()
        for _ in range(n_tg - 1):
            lg = m.forward(cur)
            cur = int(np.argmax(lg))
            ids.append(cur)
            if gpu_logits:
                keep.append(np.array(lg, np.float32, copy=True))
        tg_s = time.perf_counter() - t0
    finally:
        m.close()
    res = {"pp_tok_s": round(len(seed_ids) / pp_s, 3), "pp_tokens": len(seed_ids), "pp_s": round(pp_s, 2),
           "tg_tok_s": round((n_tg - 1) / tg_s, 3), "tg_tokens_timed": n_tg - 1, "tg_s": round(tg_s, 2)}
    if gpu_logits:
        res.update(_logits_vs_gpu(keep, gpu_logits))
    return res, ids


def _cpu_pp_only(lib, path, ctx_len, threads, ids, force_q8):
    m = lib.model(path, ctx=ctx_len, page=PAGE, threads=threads, force_q8=force_q8)
    try:
        t0 = time.perf_counter()
        m.prefill(ids, BATCH, logits=True)
        return len(ids) / (time.perf_counter() - t0)
    finally:
        m.close()


def _mean_sd(v):
    import numpy as np

    return round(float(np.mean(v)), 3), round(float(np.std(v, ddof=1)) if len(v) > 1 else 0.0, 3)


def _cpu_kernels(lib, kind, spec, threads):
    """Isolated tensor_matvec / tensor_matmul_batch_v06 on the config shapes:
    1 warm-up + 5 reps, mean +- SD in ms."""
    import numpy as np

    from memvanta_amd import synth

    rng = np.random.default_rng(ACT_SEED)
    shapes = [tuple(x) for x in spec["shapes"]]
    names = {shp: nm for shp, nm in zip(shapes, spec["names"])}
    gemm_shapes = [tuple(x) for x in spec.get("gemm_shapes", [])]
    if kind == "reference":
        g = lib.gguf(spec["path"])
        mv = lambda k, n, x: g.matvec(names[(k, n)], x, n, threads)  # noqa: E731
        mm = lambda k, n, x, q8: g.matmul_batch_v06(names[(k, n)], x, n, q8, threads)  # noqa: E731
    else:
        w = {shp: np.load(p) for shp, p in zip(shapes, spec["npy"])}
        mv = lambda k, n, x: lib.matvec(w[(k, n)], synth.Q4_0, n, k, x, threads)  # noqa: E731
        mm = lambda k, n, x, q8: lib.matmul_batch_v06(w[(k, n)], synth.Q4_0, n, k, x,  # noqa: E731
                                                       "ffn" in names[(k, n)], q8, threads)

    def rep(fn):
        fn()
        ts = []
        for _ in range(5):
            t0 = time.perf_counter()
            fn()
            ts.append((time.perf_counter() - t0) * 1e3)
        return _mean_sd(ts)

    gemv = []
    for k, n in shapes:
        x = synth.activations(rng, 1, k)[0]
        ms, sd = rep(lambda: mv(k, n, x))
        gemv.append({"shape": f"{k}->{n}", "ms": ms, "sd": sd, "GB/s": round(gemv_bytes(k, n) / ms / 1e6, 2)})
    gemm = []
    if spec.get("gemm", True):
        for k, n in gemm_shapes:
            x = synth.activations(rng, 32, k)
            for q8 in (True, False):
                ms, sd = rep(lambda: mm(k, n, x, q8))
                gemm.append({"shape": f"{k}->{n}", "M": 32, "numerics": "FORCE_Q8" if q8 else "default",
                             "ms": ms, "sd": sd, "GFLOP/s": round(2 * 32 * k * n / ms / 1e6, 1)})
    return {"tensor_matvec": gemv, "tensor_matmul_batch_v06": gemm}


def cpu_leg(spec: dict) -> dict:
    """The CPU baseline, run in its own process (no HIP runtime loaded)."""
    from oracle import pyoracle

    t_all = spec["threads"]
    if pyoracle.ref_available():
        kind, lib = "reference", pyoracle.Ref()
        note = "MemVanta's own sources compiled here by oracle/Makefile (oracle/_ref/libmvref.so)"
    else:
        kind, lib = "port", pyoracle.Oracle()
        note = ("reference library absent (oracle/_ref/libmvref.so not built: no reference checkout when "
                "build() ran); timed the C restatement oracle/liboracle.so instead")
        print(f"bench: cpu leg: {note}", file=sys.stderr, flush=True)
    s = spec["llama7b"]
    res = {"kind": kind, "library": note, "threads": t_all, "lscpu": _lscpu(),
           "omp": {k: os.environ.get(k) for k in ("OMP_PROC_BIND", "OMP_PLACES", "OMP_NUM_THREADS")}}
    t0 = time.perf_counter()
    run, ids = _cpu_model_run(lib, s["path"], CTX, t_all, s["seed_ids"], s["tg_tokens"],
                              gpu_logits=s.get("gpu_logits"))
    res["llama7b"] = dict(run, greedy_ids=ids)
    log(f"cpu leg: 7B seed prefill + {s['tg_tokens']} decode tokens on {t_all} threads "
        f"({time.perf_counter() - t0:.1f} s)")
    n_q8 = s["pp_force_q8_tokens"]
    res["llama7b"]["pp_force_q8_tok_s"] = round(_cpu_pp_only(lib, s["path"], CTX, t_all, s["seed_ids"][:n_q8], True), 3)
    res["llama7b"]["pp_force_q8_tokens"] = n_q8
    log("cpu leg: 7B FORCE_Q8 prefill sample done")
    run4, _ = _cpu_model_run(lib, s["path"], CTX, 4, s["seed_ids"][:s["seed_4"]], s["tg_tokens_4"],
                             warm_chunk=False)
    res["llama7b_4_threads"] = run4
    log("cpu leg: 7B on 4 threads done")
    res["kernels"] = _cpu_kernels(lib, kind, spec["matrices"], t_all)
    res["kernels_4_threads"] = _cpu_kernels(lib, kind, dict(spec["matrices"], gemm=False), 4)
    log("cpu leg: isolated kernels done")
    res["other_models"] = []
    for o in spec["other_models"]:
        r, oids = _cpu_model_run(lib, o["path"], o["ctx"], t_all, o["seed_ids"], o["tg_tokens"],
                                 gpu_logits=o.get("gpu_logits"))
        res["other_models"].append(dict(r, greedy_ids=oids))
    log("cpu leg: other models done")
    return res


def run_cpu_leg(spec: dict, timeout_s: float):
    """cpu_leg in a child process; returns its JSON (or an error record)."""
    fd, spec_path = tempfile.mkstemp(prefix="mv_cpu_spec_", suffix=".json")
    out_path = spec_path[:-5] + "_out.json"
    with os.fdopen(fd, "w") as f:
        json.dump(dict(spec, out=out_path), f)
    env = dict(os.environ, OMP_PROC_BIND="close", OMP_PLACES="cores")
    try:
        p = subprocess.run([sys.executable, "-u", os.path.abspath(__file__), "--cpu-leg", spec_path], env=env,
                           timeout=timeout_s)
        if p.returncode != 0:
            return {"error": f"cpu leg exited {p.returncode}"}
        with open(out_path) as f:
            return json.load(f)
    except subprocess.TimeoutExpired:
        return {"error": f"cpu leg exceeded {timeout_s:.0f} s"}
    finally:
        for q in (spec_path, out_path):
            try:
                os.unlink(q)
            except OSError:
                pass


# ---------------------------------------------------------------- main

def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10,
                    help="timed tg128 reps (each: reset, untimed 128-token seed prefill, 128 timed decode tokens)")
    ap.add_argument("--warmup", type=int, default=2, help="untimed tg128 reps before them")
    ap.add_argument("--side-reps", type=int, default=3,
                    help="timed tg reps of the KV-type and other-model runs")
    ap.add_argument("--pp-reps", type=int, default=3)
    ap.add_argument("--api-tokens", type=int, default=32, help="decode tokens timed through forward()")
    ap.add_argument("--kernel-launches", type=int, default=96)
    ap.add_argument("--rotate-mb", type=float, default=640.0,
                    help="weight bytes streamed between two uses of one copy in the kernel timings (> 256 MB MALL)")
    ap.add_argument("--cpu-tg-tokens", type=int, default=CPU_TG_TOKENS_7B,
                    help="CPU decode tokens after the 128-token seed")
    ap.add_argument("--cpu-timeout", type=float, default=600.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-kv-types", action="store_true", help="skip the F32 / Q8 KV cache runs")
    ap.add_argument("--no-other-models", action="store_true", help="skip the tiny and TinyLlama-shape configs")
    ap.add_argument("--model", default=None, help="existing GGUF to use instead of the synthetic 7B shape")
    ap.add_argument("--kernels-only", action="store_true",
                    help="only the isolated kernel timings plus the read probe and a 256 MiB copy (counter runs)")
    ap.add_argument("--tg-only", action="store_true",
                    help="only the 7B tg128 reps (no pp512, kernel timings, other runs or CPU baseline)")
    ap.add_argument("--tg-api", action="store_true",
                    help="with --tg-only: decode through forward() + host argmax (no HIP graph; counter runs)")
    ap.add_argument("--cpu-leg", default=None, help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.cpu_leg:
        with open(args.cpu_leg) as f:
            spec = json.load(f)
        res = cpu_leg(spec)
        with open(spec["out"], "w") as f:
            json.dump(res, f)
        return
    if args.gpus != 1:
        print("bench.py measures one MI355X: this build runs on a single GPU (no multi-GPU path); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0 or args.side_reps < 1:
        print("--steps and --side-reps must be >= 1, --warmup >= 0", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from memvanta_amd import capi, synth

    if args.kernels_only:
        ctx = capi.Context(0)
        mats = make_matrices()
        gemm = time_prefill_gemm(ctx, mats, 10, args.rotate_mb)
        print(json.dumps({"prefill_gemm": gemm}), flush=True)
        us = time_gemv_kernels(ctx, mats, args.kernel_launches, args.rotate_mb)
        hbm = measure_hbm(ctx, 256 << 20, 2)
        node_us = measure_node_floor(ctx)
        src = torch.empty(64 << 20, dtype=torch.float32, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)  # calibration: 256 MiB read + 256 MiB written by one copy kernel
        torch.cuda.synchronize()
        print(json.dumps({"gemv_us": {f"{k}->{n}": round(v, 3) for (k, n), v in us.items()},
                          "copy_bytes": src.numel() * 4, "read_probe_bytes": 256 << 20,
                          "read_probe_gbs": round(hbm["read"], 1), "graph_node_us": round(node_us, 3)}))
        ctx.close()
        return

    cfg = synth.LLAMA7B
    tmpdir = tempfile.mkdtemp(prefix="mv_bench_")
    t_setup = time.perf_counter()
    if args.model:
        path = args.model
    else:
        path = os.path.join(tmpdir, "openllama-7b-shape-q4_0.gguf")
        synth.write_model(cfg, path, seed=1234, device="cuda", digest=False)
        torch.cuda.synchronize()
    t_write = time.perf_counter() - t_setup
    log(f"7B-shape model written ({t_write:.1f} s)")
    ctx = None
    try:
        t0 = time.perf_counter()
        m = capi.Model(path, ctx=CTX, page_tokens=PAGE, act_mode=capi.MVH_ACT_Q8, max_batch=PROMPT_TOKENS)
        t_load = time.perf_counter() - t0
        stream = torch.cuda.ExternalStream(m.stream)
        vocab = m.vocab
        prompt = synth.prompt_tokens(PROMPT_SEED_7B, PROMPT_TOKENS, vocab)
        seed = prompt[:SEED_TOKENS]

        if args.tg_only and args.tg_api:
            walls, ids = [], []
            for _ in range(args.warmup + args.steps):
                m.reset()
                m.prefill(seed, BATCH, logits=False)
                torch.cuda.synchronize()
                t0, cur, ids = time.perf_counter(), FIRST_TOKEN, []
                for _ in range(TG_TOKENS):
                    cur = int(np.argmax(m.forward(cur)))
                    ids.append(cur)
                walls.append(time.perf_counter() - t0)
            m.close()
            walls = walls[args.warmup:]
            print(json.dumps({"tg128_api_tok_s": round(TG_TOKENS * len(walls) / sum(walls), 2) if walls else None,
                              "ids_head": ids[:8]}), flush=True)
            return
        if args.tg_only:
            tg_wall, tg_dev, ids, ids_same = tg_reps(m, seed, TG_TOKENS, args.steps, args.warmup)
            m.close()
            print(json.dumps({"tg128_tok_s": round(TG_TOKENS * args.steps / sum(tg_wall), 2),
                              "tg128_tok_s_per_rep": [round(TG_TOKENS / t, 2) for t in tg_wall],
                              "gpu_ms_per_token": round(sum(tg_dev) / (TG_TOKENS * args.steps) * 1e3, 4),
                              "ids_head": ids[:8], "ids_identical_across_reps": ids_same,
                              "attn_ns": os.environ.get("MVH_ATTN_NS")}), flush=True)
            return

        # pp512 (host-driven chunks of 32, last-token logits), after one untimed run
        pp = time_pp(m, prompt, args.pp_reps)
        pp_whole, pp_whole_same = pp_whole_prompt(m, prompt, args.pp_reps)

        # tg128: W untimed reps (the first captures the decode graph), then K timed reps
        tg_wall, tg_dev, ids, ids_same = tg_reps(m, seed, TG_TOKENS, args.steps, args.warmup)
        wall = sum(tg_wall)
        gpu_s = sum(tg_dev)
        n_tok = TG_TOKENS * args.steps
        tg = n_tok / wall
        tg_rep_rates = [TG_TOKENS / t for t in tg_wall]
        tok_bytes = model_weight_bytes(cfg, synth) * TG_TOKENS + kv_read_bytes(cfg, SEED_TOKENS, TG_TOKENS)
        tg_gbs = tok_bytes * args.steps / wall / 1e9
        # one more rep seeded with the reference bench's fixed_tokens
        fx_wall, _, fx_ids, _ = tg_reps(m, fixed_tokens(SEED_TOKENS, vocab), TG_TOKENS, 1, 0)

        # the same decode through the per-call API: forward() + host argmax
        m.reset()
        m.prefill(seed, BATCH, logits=False)
        cur = FIRST_TOKEN
        cur = int(np.argmax(m.forward(cur)))
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.api_tokens):
            cur = int(np.argmax(m.forward(cur)))
        api_tg = args.api_tokens / (time.perf_counter() - t0)
        m.close()
        log(f"7B pp512 / {args.steps} x tg{TG_TOKENS} done")

        n_cpu_tg = args.cpu_tg_tokens
        gpu_logits_7b = os.path.join(tmpdir, "openllama-7b_gpu_logits.npy")
        pp_default, ref_ids, pp_default_whole, pp_default_whole_same, graph_ids_same = default_numerics_run(
            path, prompt, CTX, seed, n_cpu_tg, gpu_logits_7b)

        # dominant kernel alone: Q4_0 x Q8 GEMV; prefill GEMM; measured ceilings
        ctx = capi.Context(0)
        mats = make_matrices()
        us = time_gemv_kernels(ctx, mats, args.kernel_launches, args.rotate_mb)
        mix_bytes = sum(gemv_bytes(k, n) * c for k, n, c in DECODE_GEMVS)
        mix_us = sum(us[(k, n)] * c for k, n, c in DECODE_GEMVS)
        launches = sum(c for _, _, c in DECODE_GEMVS)
        achieved = mix_bytes / (mix_us * 1e-6) / 1e9
        per_shape = [{"shape": f"{k}->{n}", "us": round(us[(k, n)], 2),
                      "GB/s": round(gemv_bytes(k, n) / us[(k, n)] / 1e3, 1)} for k, n in ISOLATED_GEMVS]
        gemm = time_prefill_gemm(ctx, mats, 10, args.rotate_mb)
        hbm = measure_hbm(ctx)
        node_us = measure_node_floor(ctx)
        log("kernel timings done")

        traffic = None
        pmc = os.path.join(ROOT, "profiles", "gemv_q4_0_7b_decode_traffic.json")
        if os.path.exists(pmc):
            with open(pmc) as f:
                traffic = json.load(f).get("hbm_bytes_per_launch")

        kv_types = None if args.no_kv_types else time_kv_types(path, seed, prompt, args.side_reps,
                                                               min(args.warmup, 1))

        others, other_specs, other_ids = [], [], []
        if not args.no_other_models:
            for label, name, ctx_len, pp_n, seed_n, tg_n, pseed, cpu_run in OTHER_MODELS:
                r, s, oids = time_other_model(tmpdir, label, name, ctx_len, pp_n, seed_n, tg_n, pseed, cpu_run,
                                              args.side_reps, min(args.warmup, 1))
                others.append(r)
                other_specs.append(s)
                other_ids.append(oids)
                log(f"{name} done")
        ctx.close()
        ctx = None

        cpu = None
        if not args.no_cpu:
            mpath = os.path.join(tmpdir, "gemv-config-q4_0.gguf")
            w = synth.GgufWriter()
            w.add_str("general.architecture", "matrices")
            npys = []
            for k, n in GEMV_CONFIG:
                data = mats[(k, n)]
                w.add_tensor(MATRIX_NAMES[(k, n)], (k, n), synth.Q4_0, data.nbytes,
                             lambda d=data: iter([d.tobytes()]))
                npys.append(os.path.join(tmpdir, f"w_{k}x{n}.npy"))
                np.save(npys[-1], data)
            w.write(mpath)
            del mats
            spec = {"threads": len(os.sched_getaffinity(0)),
                    "llama7b": {"path": path, "seed_ids": [int(t) for t in seed], "tg_tokens": n_cpu_tg,
                                "gpu_logits": gpu_logits_7b,
                                "pp_force_q8_tokens": CPU_PP_FORCE_Q8_TOKENS, "seed_4": CPU_SEED_4_THREADS,
                                "tg_tokens_4": CPU_TG_4_THREADS},
                    "matrices": {"path": mpath, "shapes": GEMV_CONFIG, "npy": npys,
                                 "names": [MATRIX_NAMES[kn] for kn in GEMV_CONFIG], "gemm_shapes": PREFILL_GEMMS},
                    "other_models": other_specs}
            log("cpu leg started (child process)")
            cpu = run_cpu_leg(spec, args.cpu_timeout)
            log("cpu leg done")
    finally:
        if ctx is not None:
            ctx.close()
        for f in os.listdir(tmpdir):
            try:
                os.unlink(os.path.join(tmpdir, f))
            except OSError:
                pass
        try:
            os.rmdir(tmpdir)
        except OSError:
            pass

    cpu_baseline = None
    if cpu is not None and "error" in cpu:
        cpu_baseline = cpu
    elif cpu is not None:
        c7 = cpu["llama7b"]
        n_cmp = len(c7["greedy_ids"])
        c4 = cpu["llama7b_4_threads"]
        cpu_baseline = {
            "value": c7["tg_tok_s"], "unit": "tok/s", "cores": cpu["threads"], "kind": cpu["kind"],
            "library": cpu["library"],
            "sample": f"7B-shape model, same GGUF: default-numerics prefill of the same 128-token seed "
                      f"({c7['pp_s']} s, after one untimed 32-token chunk), then {n_cmp} greedy decode tokens from "
                      f"token {FIRST_TOKEN} at the GPU run's positions {SEED_TOKENS}..{SEED_TOKENS + n_cmp - 1} "
                      f"(the first of them untimed; forward + host argmax, {c7['tg_s']} s), {cpu['threads']} "
                      f"OpenMP threads",
            "greedy_ids_match_gpu": c7["greedy_ids"] == ref_ids[:n_cmp],
            "greedy_ids_compared": n_cmp,
            "greedy_ids_basis": "GPU ids after a default-numerics seed prefill (the CPU leg's); decode numerics "
                                "do not depend on the prefill mode, the seed's KV entries do",
            "logits_steps_compared": c7.get("logits_steps_compared"),
            "logits_max_rel_l2": c7.get("logits_max_rel_l2"),
            "logits_min_bit_identical_frac": c7.get("logits_min_bit_identical_frac"),
            "logits_basis": "every decode step's logits of the CPU run against the GPU's forward() logits at the "
                            "same step (same seed prefill, same ids); tolerance 1e-3 relative L2",
            "pp_sample_default_numerics_tok_s": c7["pp_tok_s"],
            "pp_sample_default_numerics_tokens": c7["pp_tokens"],
            "pp_sample_force_q8_tok_s": c7["pp_force_q8_tok_s"],
            "pp_sample_force_q8_tokens": c7["pp_force_q8_tokens"],
            "value_4_threads": c4["tg_tok_s"],
            "pp_sample_default_numerics_tok_s_4_threads": c4["pp_tok_s"],
            "sample_4_threads": f"default-numerics prefill of the first {c4['pp_tokens']} seed tokens "
                                f"({c4['pp_s']} s), then {c4['tg_tokens_timed'] + 1} decode tokens (first untimed) "
                                f"at positions {c4['pp_tokens']}.., 4 OpenMP threads",
            "isolated_kernels": cpu["kernels"],
            "isolated_kernels_4_threads": cpu["kernels_4_threads"],
            "kernel_protocol": "same weight bytes as the GPU timing, activations N(0,1) with 0.1% +-20 outliers "
                               "(seed 99); 1 warm-up + 5 reps, mean and SD in ms; GEMM at M=32 (the prefill "
                               "chunk), FORCE_Q8 and default numerics; host memory warm",
            "lscpu": cpu["lscpu"], "omp": cpu["omp"],
        }
        for r, c, g in zip(others, cpu.get("other_models", []), other_ids):
            n = len(c["greedy_ids"])
            r["cpu"] = {"kind": cpu["kind"], "threads": cpu["threads"],
                        "pp_sample_default_numerics_tok_s": c["pp_tok_s"], "pp_sample_tokens": c["pp_tokens"],
                        "tg_tok_s": c["tg_tok_s"], "tg_tokens_timed": c["tg_tokens_timed"],
                        "tg_after_seed_tokens": c["pp_tokens"],
                        "greedy_ids_match_gpu": c["greedy_ids"] == g[:n], "greedy_ids_compared": n,
                        "logits_steps_compared": c.get("logits_steps_compared"),
                        "logits_max_rel_l2": c.get("logits_max_rel_l2"),
                        "logits_min_bit_identical_frac": c.get("logits_min_bit_identical_frac"),
                        "greedy_ids_basis": "GPU ids after a default-numerics prefill of the same seed"}

    pp_mean = float(np.mean(pp))
    out = {
        "metric": METRIC,
        "value": round(tg, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": round(tg / REF_TG128_TOKS, 1),
        "dtype": "q4_0 x q8_0 int8 dot, f32 accumulate; f16 KV",
        "data": "synthetic",
        "config": {
            "workload": "tg128 + pp512, OpenLLaMA-7B-v2-shape random-init Q4_0 model (dim 4096, FFN 11008, "
                        "32 layers, 32 heads MHA, vocab 32000, output Q6_K), ctx 768, batch 32, paged F16 KV "
                        "(128-token pages), greedy, seeded uniform prompt ids",
            "step": f"one tg128 rep: reset, untimed prefill of a {SEED_TOKENS}-token seed (chunks of {BATCH}), "
                    f"then {TG_TOKENS} greedy decode tokens from token {FIRST_TOKEN} timed (positions "
                    f"{SEED_TOKENS}..{SEED_TOKENS + TG_TOKENS - 1}); value = {TG_TOKENS} x steps / the steps' "
                    f"decode seconds; ms_per_step = decode ms of one rep",
            "prompt_ids": f"uniform in [0, {vocab}) from seed {PROMPT_SEED_7B} (numpy default_rng); the tg seed "
                          f"is the prompt's first {SEED_TOKENS} ids",
            "tg_tok_s": round(tg, 2),
            "tg_tok_s_per_rep": [round(v, 2) for v in tg_rep_rates],
            "tg_tokens_timed": n_tok,
            "tg_ids_identical_across_reps": ids_same,
            "tg_hbm_gbs": round(tg_gbs, 1),
            "tg_hbm_frac": round(tg_gbs / HBM_PEAK_GBS, 4),
            "tg_bytes_per_token": tok_bytes // TG_TOKENS,
            "tg_bytes_basis": f"weights + F16 K and V read at positions {SEED_TOKENS}..{SEED_TOKENS + TG_TOKENS - 1}, "
                              f"averaged over the {TG_TOKENS} tokens",
            "tg_gpu_ms_per_token": round(gpu_s / n_tok * 1e3, 4),
            "tg128_fixed_tokens_seed_tok_s": round(TG_TOKENS / fx_wall[0], 2),
            "tg128_fixed_tokens_seed_ids_head": fx_ids[:8],
            "graph_ids_equal_forward_ids": graph_ids_same,
            "tg_api_tok_s": round(api_tg, 2),
            "pp512_tok_s": round(pp_mean, 1),
            "pp512_tok_s_reps": [round(v, 1) for v in pp],
            "pp_numerics": "tensor_matmul_batch_v06, MEMVANTA_FORCE_Q8_ACT=1",
            "pp512_default_numerics_tok_s": round(pp_default, 1),
            "pp_default_numerics": "tensor_matmul_batch_v06 without MEMVANTA_FORCE_Q8_ACT (fp32 activations, "
                                   "batch8 / batch4 accumulators)",
            "pp512_batch512_tok_s": round(float(np.mean(pp_whole)), 1),
            "pp512_batch512_default_numerics_tok_s": round(pp_default_whole, 1),
            "pp512_batch512_logits_identical_to_batch32": pp_whole_same and pp_default_whole_same,
            "pp512_batch512_basis": "the 512-token prompt as one prefill batch (every GEMM at M = 512), "
                                    "not the config's batch 32; last-token logits compared bit for bit with "
                                    "the batch-32 run in both numerics",
            "greedy_ids_head": ids[:8],
            "model_write_s": round(t_write, 1),
            "model_load_s": round(t_load, 2),
            "timing": "tg: device-resident greedy loop (HIP graphs of eight decode steps), wall clock between "
                      "device synchronizations; pp: host-driven chunks, wall clock",
            "vs_baseline_basis": "published reference tg128 1.52 tok/s (real OpenLLaMA-7B-v2 Q4_0, CPU, 4 threads); "
                                 "decode numerics do not depend on the prefill mode",
            "pp512_vs_published": round(pp_default / REF_PP512_TOKS, 1),
            "pp512_vs_published_basis": "default-numerics pp512 (the numerics of the published run) / published "
                                        "reference pp512 3.15 tok/s (same run as the tg128 figure)",
            "gemv_kernel_per_shape": per_shape,
            "prefill_gemm_int8_mfma": gemm,
            "prefill_gemm_note": "tensor_matmul_batch_v06 FORCE_Q8 numerics incl. the activation quantizer; "
                                 "frac_int8_peak vs 5 POP/s dense int8; us: one GEMM at a time; "
                                 "us_per_gemm_3_streams (M = 32): three independent chains of the same GEMM, "
                                 "each on its own stream, started together (the three-stream prefill's "
                                 "operating point)",
            "prefill_roofline": prefill_roofline(gemm),
            "other_kv_cache_types": kv_types,
            "other_models": others,
        },
        "roofline": {"bound": "hbm", "kernel": "gemv_q4_rows16 (Q4_0 x pre-quantized Q8, 16-lane row groups)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "avg_launch_us": round(mix_us / launches, 3),
                     "algorithmic_bytes_per_launch": mix_bytes // launches,
                     "launch_mix": "7B decode layer: 4096->12288 (q|k|v), 4096->4096 (o), 4096->22016 "
                                   "(gate|up), 11008->4096 (down)",
                     "measured_read_gbs": round(hbm["read"], 1),
                     "measured_read_basis": "mvh_stream_read over two alternated 1 GiB buffers (16-byte coalesced "
                                            "loads, 8 workgroups per CU), HIP events",
                     "measured_copy_gbs": round(hbm["copy"], 1),
                     "measured_graph_node_us": round(node_us, 3),
                     "graph_node_basis": "a one-workgroup 16-byte mvh_stream_read per node, graph of 200 nodes: "
                                         "the floor each dependent kernel of a decode step pays",
                     "frac_of_measured_read": round(achieved / hbm["read"], 4)},
        "cpu_baseline": cpu_baseline,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
