"""bench.py's CPU baseline leg on small models (CPU only): the protocol runs
end to end in-process and as the child process the bench starts, with the
compiled reference and with the C restatement, and both give the same greedy
ids (the restatement's model agrees with the reference's on a decode)."""
import json
import os

import numpy as np
import pytest

import bench
from memvanta_amd import synth
from oracle import pyoracle


@pytest.fixture(scope="module")
def spec(tmp_path_factory):
    d = tmp_path_factory.mktemp("cpuleg")
    big = str(d / "mixed2l.gguf")
    synth.write_model(synth.TINYLLAMA_MIXED_2L, big, seed=7, digest=False)
    tiny = str(d / "tiny.gguf")
    synth.write_model(synth.TINY, tiny, seed=2024, digest=False)
    rng = np.random.default_rng(1)
    shapes, names = [(256, 64), (512, 32)], ["blk.0.ffn_up.weight", "blk.0.attn_q.weight"]
    w = synth.GgufWriter()
    w.add_str("general.architecture", "matrices")
    npys = []
    for (k, n), nm in zip(shapes, names):
        data = synth.quantize(synth.Q4_0, rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
        w.add_tensor(nm, (k, n), synth.Q4_0, data.nbytes, lambda dd=data: iter([dd.tobytes()]))
        npys.append(str(d / f"w{k}x{n}.npy"))
        np.save(npys[-1], data)
    mp = str(d / "mats.gguf")
    w.write(mp)
    # the logits the GPU side would save: here the restatement's own run of the protocol
    seed_ids = synth.prompt_tokens(5, 40)
    o = pyoracle.Oracle().model(big, ctx=bench.CTX, page=bench.PAGE, threads=4)
    o.prefill(seed_ids, bench.BATCH, logits=False)
    lgs, cur = [], bench.FIRST_TOKEN
    for _ in range(5):
        lg = np.array(o.forward(cur), np.float32, copy=True)
        cur = int(np.argmax(lg))
        lgs.append(lg)
    o.close()
    lpath = str(d / "gpu_logits.npy")
    np.save(lpath, np.stack(lgs))
    return {"threads": 4,
            "llama7b": {"path": big, "seed_ids": seed_ids.tolist(), "tg_tokens": 5,
                        "pp_force_q8_tokens": 32, "seed_4": 32, "tg_tokens_4": 3, "gpu_logits": lpath},
            "matrices": {"path": mp, "shapes": shapes, "npy": npys, "names": names, "gemm_shapes": [shapes[0]]},
            "other_models": [{"path": tiny, "ctx": 256, "seed_ids": synth.prompt_tokens(2024, 40).tolist(),
                              "tg_tokens": 4}]}


def _check(res, kind, spec):
    assert res["kind"] == kind
    assert len(res["llama7b"]["greedy_ids"]) == spec["llama7b"]["tg_tokens"]
    assert res["llama7b"]["pp_tokens"] == len(spec["llama7b"]["seed_ids"])
    assert res["llama7b"]["tg_tok_s"] > 0 and res["llama7b"]["pp_force_q8_tok_s"] > 0
    assert [g["shape"] for g in res["kernels"]["tensor_matvec"]] == ["256->64", "512->32"]
    assert {g["numerics"] for g in res["kernels"]["tensor_matmul_batch_v06"]} == {"FORCE_Q8", "default"}
    assert res["kernels_4_threads"]["tensor_matmul_batch_v06"] == []
    assert len(res["other_models"][0]["greedy_ids"]) == 4
    assert "CPU(s)" in res["lscpu"]
    # every decode step's logits compared with the saved ones: the same numerics reproduce them exactly
    assert res["llama7b"]["logits_steps_compared"] == 5
    assert res["llama7b"]["logits_max_rel_l2"] == 0.0
    assert res["llama7b"]["logits_min_bit_identical_frac"] == 1.0
    assert "logits_steps_compared" not in res["other_models"][0]


def test_cpu_leg_port_and_reference_agree(spec, monkeypatch):
    runs = {}
    if pyoracle.ref_available():
        runs["reference"] = bench.cpu_leg(spec)
        _check(runs["reference"], "reference", spec)
    monkeypatch.setattr(pyoracle, "ref_available", lambda: False)
    runs["port"] = bench.cpu_leg(spec)
    _check(runs["port"], "port", spec)
    assert "absent" in runs["port"]["library"]
    if "reference" in runs:
        assert runs["port"]["llama7b"]["greedy_ids"] == runs["reference"]["llama7b"]["greedy_ids"]
        assert runs["port"]["other_models"][0]["greedy_ids"] == runs["reference"]["other_models"][0]["greedy_ids"]


def test_cpu_leg_child_process(spec):
    res = bench.run_cpu_leg(spec, 300)
    assert "error" not in res, res
    assert res["omp"]["OMP_PROC_BIND"] == "close" and res["omp"]["OMP_PLACES"] == "cores"
    json.dumps(res)


def test_logits_vs_gpu_reports_the_worst_step(tmp_path):
    rng = np.random.default_rng(3)
    cpu = [rng.standard_normal(1000).astype(np.float32) for _ in range(3)]
    gpu = np.stack(cpu).copy()
    gpu[1, :10] += np.float32(0.5)  # one step differs
    p = str(tmp_path / "g.npy")
    np.save(p, gpu)
    r = bench._logits_vs_gpu(cpu, p)
    want = np.linalg.norm(gpu[1].astype(np.float64) - cpu[1]) / np.linalg.norm(cpu[1].astype(np.float64))
    assert r["logits_steps_compared"] == 3
    assert abs(r["logits_max_rel_l2"] - want) < 1e-12 and r["logits_max_rel_l2"] > 1e-3
    assert r["logits_min_bit_identical_frac"] == 0.99


def test_prefill_roofline_floor():
    gemm = [{"K": 4096, "N": 4096, "M": 512, "us": 41.0, "frac_int8_peak": 0.1},
            {"K": 4096, "N": 4096, "M": 32, "us": 8.0, "frac_int8_peak": 0.01}]
    r = bench.prefill_roofline(gemm)
    # 3 lane-operations x 512 x 4096 x 128 blocks at 256 x 64 x 2.4e9 lane-ops/s
    assert r["M512"]["valu_floor_us"] == round(3 * 512 * 4096 * 128 / (256 * 64 * 2.4e9) * 1e6, 2) == 20.48
    assert r["M512"]["frac_of_valu_floor"] == round(20.4800 / 41.0, 4)
    assert r["M32"]["hbm_bound_us"] == round((4096 * 128 * 18 + 32 * (4096 + 512) + 4 * 32 * 4096) / 8e6, 2)
