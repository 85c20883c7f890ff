"""Kernel profiler (enable_kernel_profiling / kernel_profile_snapshot,
include/memvanta/gguf_kernels.hpp:11-23): the entries the C ABI records for a
sequence of tensor calls and for a model run, against the compiled
reference's entries for the same sequence (tests/golden/profile.npz).  Layer,
kind, tensor, call count and batch must match exactly; times are device
times and only checked to be non-negative (positive where kernels ran)."""
import numpy as np
import pytest

from conftest import golden
from memvanta_amd import capi, synth

pytestmark = pytest.mark.gpu

ROWS, COLS = 32, 64


@pytest.fixture
def ctx():
    c = capi.Context(0)
    capi.profile_enable(False)
    capi.profile_reset()
    yield c
    capi.profile_enable(False)
    capi.profile_reset()
    c.close()


def _upload_all(ctx, names):
    rng = np.random.default_rng(5)
    ts = []
    for n in names:
        w = synth.quantize(synth.Q4_0, rng.standard_normal((ROWS, COLS), dtype=np.float32) * np.float32(0.02))
        ts.append(ctx.upload(n, synth.Q4_0, COLS, ROWS, w))
    return ts


def _replay(ctx, ts, calls):
    rng = np.random.default_rng(6)
    for op, i, b in calls:
        if op == 0:
            ctx.matvec(ts[i], synth.activations(rng, 1, COLS)[0])
        elif op == 1:
            ctx.matmul_batch(ts[i], np.ascontiguousarray(synth.activations(rng, max(b, 1), COLS)[:b]))
        else:
            ctx.matmul_batch_v06(ts[i], synth.activations(rng, b, COLS),
                                 act_mode=capi.MVH_ACT_Q8 if op == 3 else capi.MVH_ACT_REF)


def test_tensor_call_entries_match_reference(ctx):
    g = golden("profile.npz")
    names = g["names"].tolist()
    ts = _upload_all(ctx, names)
    capi.profile_enable(True)
    _replay(ctx, ts, g["calls"].tolist())
    capi.profile_enable(False)
    got = capi.profile_snapshot()
    want = list(zip(g["e_layer"].tolist(), g["e_kind"].tolist(), g["e_tensor"].tolist(), g["e_calls"].tolist(),
                    g["e_batch"].tolist()))
    assert [(e["layer"], e["kind"], e["tensor"], e["calls"], e["batch"]) for e in got] == want
    for e in got:
        assert e["ms"] >= 0.0
        if e["batch"] > 0:
            assert e["ms"] > 0.0, e
        assert e["kind_name"] == capi.PROFILE_KINDS[e["kind"]]


def test_disabled_and_reset(ctx):
    ts = _upload_all(ctx, ["blk.3.attn_q.weight"])
    x = np.ones(COLS, np.float32)
    ctx.matvec(ts[0], x)  # profiling off: nothing recorded
    assert capi.profile_snapshot() == []
    capi.profile_enable(True)
    y_on = ctx.matvec(ts[0], x)
    capi.profile_enable(False)
    y_off = ctx.matvec(ts[0], x)
    assert np.array_equal(y_on, y_off)  # the events change nothing in the results
    snap = capi.profile_snapshot()
    assert [(e["layer"], e["kind_name"], e["calls"], e["batch"]) for e in snap] == [(3, "q_proj", 1, 1)]
    capi.profile_reset()
    assert capi.profile_snapshot() == []


def test_model_entries_match_reference(ctx, tmp_path):
    """A model run (5-token prefill in chunks of 4, two decode steps, Q8
    prefill numerics): a launch over fused weights is one entry named by its
    members joined with '+'; split into its members, every (tensor, batch)
    has the reference's call count, layer and kind."""
    g = golden("profile.npz")
    path = str(tmp_path / "tiny.gguf")
    synth.write_model(synth.TINY, path, seed=1234)
    m = capi.Model(path, ctx=256, act_mode=capi.MVH_ACT_Q8, max_batch=32)
    capi.profile_enable(True)
    m.prefill(g["m_prompt"], 4)
    m.forward(17)
    m.forward(23)
    capi.profile_enable(False)
    got = capi.profile_snapshot()
    m.close()
    split = {}
    for e in got:
        assert e["ms"] > 0.0, e
        members = e["tensor"].split("+")
        if len(members) > 1:
            assert e["kind_name"] == capi.PROFILE_KINDS[e["kind"]]
        for t in members:
            key = (t, e["batch"])
            assert key not in split, key
            split[key] = e["calls"]
    want = {(t, b): c for t, c, b in zip(g["m_tensor"].tolist(), g["m_calls"].tolist(), g["m_batch"].tolist())}
    assert split == want
    # unfused entries also carry the reference's layer and kind
    ref_lk = {(t, b): (l, k) for t, b, l, k in zip(g["m_tensor"].tolist(), g["m_batch"].tolist(),
                                                    g["m_layer"].tolist(), g["m_kind"].tolist())}
    for e in got:
        if "+" not in e["tensor"]:
            assert (e["layer"], e["kind"]) == ref_lk[(e["tensor"], e["batch"])], e


def test_profiled_greedy_equals_graph(ctx, tmp_path):
    """generate_greedy runs its steps without the HIP graph while profiling:
    the same ids, and one output-head entry per step."""
    path = str(tmp_path / "tiny.gguf")
    synth.write_model(synth.TINY, path, seed=1234)
    g = golden("model_tiny.npz")
    m = capi.Model(path, ctx=256, max_batch=32)
    m.prefill(g["prompt"], 32, logits=False)
    ids_graph, _ = m.generate_greedy(17, 6, logits=True)
    m.reset()
    m.prefill(g["prompt"], 32, logits=False)
    capi.profile_enable(True)
    ids_prof, _ = m.generate_greedy(17, 6, logits=True)
    capi.profile_enable(False)
    m.close()
    assert ids_prof.tolist() == ids_graph.tolist()
    out = [e for e in capi.profile_snapshot() if e["tensor"] == "output.weight"]
    assert [(e["calls"], e["batch"], e["kind_name"]) for e in out] == [(6, 1, "output")]
