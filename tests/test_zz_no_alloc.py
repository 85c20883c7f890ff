"""mvh_matmul_batch_v06_noalloc (the allocation-free variant of
mvh_matmul_batch_v06, static per-device scratch) against mvh_matmul_batch_v06
on the same device buffers, bit for bit: two FORCE_Q8 Q4_0 calls in a row (the
second smaller, so the scratch holds the first call's bytes beyond the second's
extent), the other branches (Q8_0 weights, default numerics, the per-token
fallback), and the size limit."""
import numpy as np
import pytest

from conftest import assert_bitexact
from memvanta_amd import capi, synth

pytestmark = pytest.mark.gpu


def _case(ctx, rng, ty, k, n, b, name="blk.0.ffn_up.weight"):
    import torch

    w = synth.quantize(ty, rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02))
    t = ctx.upload(name, ty, k, n, w)
    x = torch.from_numpy(synth.activations(rng, b, k)).to("cuda:0")
    return t, x


def _both(ctx, t, x, mode):
    import torch

    n = t.ne1
    y0 = torch.full((x.shape[0], n), float("nan"), dtype=torch.float32, device="cuda:0")
    y1 = torch.full_like(y0, float("nan"))
    torch.cuda.synchronize()
    ctx.matmul_batch_v06(t, x, mode, y=y0)
    ctx.matmul_batch_v06_noalloc(t, x, y1, mode)
    ctx.synchronize()
    return y1.cpu().numpy(), y0.cpu().numpy()


def test_noalloc_two_calls_second_smaller(ctx):
    rng = np.random.default_rng(404)
    t1, x1 = _case(ctx, rng, synth.Q4_0, 4096, 1024, 512)
    got, want = _both(ctx, t1, x1, capi.MVH_ACT_Q8)
    assert_bitexact(got, want, "first call: 512 tokens x 4096")
    t2, x2 = _case(ctx, rng, synth.Q4_0, 11008, 256, 37)
    got, want = _both(ctx, t2, x2, capi.MVH_ACT_Q8)
    assert_bitexact(got, want, "second call: 37 tokens x 11008")
    t3, x3 = _case(ctx, rng, synth.Q4_0, 4096, 300, 3)
    got, want = _both(ctx, t3, x3, capi.MVH_ACT_Q8)
    assert_bitexact(got, want, "third call: 3 tokens")
    for t in (t1, t2, t3):
        t.free()


@pytest.mark.parametrize("ty,k,n,b,mode", [(synth.Q4_0, 4096, 512, 40, capi.MVH_ACT_REF),
                                           (synth.Q8_0, 2048, 256, 9, capi.MVH_ACT_Q8),
                                           (synth.Q4_0, 288, 100, 5, capi.MVH_ACT_Q8),
                                           (synth.Q6_K, 1024, 64, 6, capi.MVH_ACT_Q8),
                                           (synth.Q4_0, 4096, 128, 1, capi.MVH_ACT_Q8)])
def test_noalloc_other_branches(ctx, ty, k, n, b, mode):
    """Default numerics, Q8_0 weights, K % 256 != 0 (per-token GEMVs from the
    scratch), the Q6_K and one-token fallbacks."""
    rng = np.random.default_rng(k + n + b)
    t, x = _case(ctx, rng, ty, k, n, b)
    got, want = _both(ctx, t, x, mode)
    assert_bitexact(got, want, f"type {ty} {k}->{n} x{b}")
    t.free()


def test_noalloc_rejects_batches_beyond_the_scratch(ctx):
    import torch

    rng = np.random.default_rng(5)
    t, x = _case(ctx, rng, synth.Q4_0, 11008, 64, 1024)
    y = torch.full((1024, 64), 7.0, dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    with pytest.raises(capi.MvhError, match="static scratch") as e:
        ctx.matmul_batch_v06_noalloc(t, x, y, capi.MVH_ACT_Q8)
    assert e.value.code == 5
    ctx.synchronize()
    assert bool((y == 7.0).all())
    t.free()


@pytest.mark.parametrize("mode,b", [(capi.MVH_ACT_Q8, 40), (capi.MVH_ACT_REF, 40), (capi.MVH_ACT_REF, 37)])
def test_noalloc_under_graph_capture(ctx, mode, b):
    """The entry point captured into a HIP graph on the context's stream (the
    callers it exists for) and replayed three times, with an eager call of a
    different input between the replays (it overwrites the static scratch):
    every replay equals the eager result bit for bit.  40 tokens in default
    numerics are five 8-token groups; 37 leaves a 5-token tail of per-token dots."""
    import torch

    rng = np.random.default_rng(77 + b + mode)
    t, x = _case(ctx, rng, synth.Q4_0, 4096, 512, b)
    _, x_other = _case(ctx, rng, synth.Q4_0, 4096, 8, 2 * b)
    y_other = torch.empty((2 * b, 512), dtype=torch.float32, device="cuda:0")
    want = torch.full((b, 512), float("nan"), dtype=torch.float32, device="cuda:0")
    y = torch.full_like(want, float("nan"))
    torch.cuda.synchronize()
    ctx.matmul_batch_v06_noalloc(t, x, want, mode)
    ctx.synchronize()
    want = want.cpu().numpy()
    stream = torch.cuda.ExternalStream(ctx.stream)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        ctx.matmul_batch_v06_noalloc(t, x, y, mode)
    ctx.synchronize()
    for r in range(3):
        y.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            g.replay()
        ctx.synchronize()
        assert_bitexact(y.cpu().numpy(), want, f"replay {r}")
        ctx.matmul_batch_v06_noalloc(t, x_other, y_other, mode)  # eager work between the replays
        ctx.synchronize()
    del g
    t.free()
