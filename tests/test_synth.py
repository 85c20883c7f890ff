"""The torch quantizers (used to synthesize multi-GB models on the device)
write the same bytes as the numpy quantizers the golden vectors were made with,
and both decode back to their input within the formats' step sizes."""
import numpy as np
import pytest
import torch

from memvanta_amd import synth


@pytest.mark.parametrize("ty", [synth.Q4_0, synth.Q8_0, synth.Q6_K])
def test_torch_quantizer_matches_numpy(ty):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((37, 512), dtype=np.float32) * np.float32(0.02)
    x[3, :64] = 0.0                       # all-zero blocks (d = 0)
    x[5, 7] = 1.5                         # an outlier
    x[9, 32:64] = np.float32(-0.01)       # a constant block: ties in the max search
    want = synth.quantize(ty, x)
    got = synth.quantize_torch(ty, torch.from_numpy(x)).numpy()
    assert got.shape == want.shape
    assert np.array_equal(got, want)
    # round trip: within one quantization step (Q4_0: amax/8, where the
    # clamp at q = 15 costs up to a full step) of each 32-element block
    back = synth.dequantize(ty, want, *x.shape)
    err = np.abs(back - x).reshape(37, 16, 32).max(axis=2)
    amax = np.abs(x).reshape(37, 16, 32).max(axis=2)
    ok = err <= amax / 8 * 1.001 + 1e-9
    if ty == synth.Q6_K:  # one 8-bit sub-block scale per 16: the outlier's super-block coarsens the others
        ok[5] = True
    assert ok.all()


def test_write_model_device_path(tmp_path):
    cfg = synth.dataclasses.replace(synth.TINY, name="tiny-torch", layers=1)
    p = str(tmp_path / "t.gguf")
    assert synth.write_model(cfg, p, seed=3, device="cpu", digest=False) is None
    sha1 = synth.write_model(cfg, p, seed=3, device="cpu")
    sha2 = synth.write_model(cfg, p, seed=3, device="cpu")
    assert sha1 == sha2


@pytest.mark.parametrize("ty", [synth.Q4_0, synth.Q8_0, synth.Q6_K])
def test_random_blocks_are_valid_and_reproducible(ty):
    """blocks="random" models: every scale a finite fp16 in its stated range,
    Q8_0 codes in [-127, 127], Q6_K sub-block scales in [-64, 63]; the same
    seed gives the same bytes, and the dequantized weights have the spread of
    N(0, 0.02) weights (std within a factor 2)."""
    rows, cols = 33, 512
    a = b"".join(synth.random_blocks(ty, rows, cols, np.random.default_rng(9), chunk_rows=8)())
    b = b"".join(synth.random_blocks(ty, rows, cols, np.random.default_rng(9), chunk_rows=8)())
    assert a == b and len(a) == rows * synth.row_bytes(ty, cols)
    raw = np.frombuffer(a, np.uint8)
    qk, bs = synth.BLOCK[ty]
    blk = raw.reshape(-1, bs)
    if ty == synth.Q6_K:
        d = blk[:, 208:210].copy().view(np.float16).astype(np.float64).ravel()
        sc = blk[:, 192:208].view(np.int8)
        assert sc.min() >= -64 and sc.max() <= 63
        assert (d >= 1.7e-5).all() and (d <= 3.7e-5).all()
    else:
        d = blk[:, 0:2].copy().view(np.float16).astype(np.float64).ravel()
        if ty == synth.Q8_0:
            assert blk[:, 2:].view(np.int8).min() >= -127
            assert (d >= 1.4e-4).all() and (d <= 3.6e-4).all()
        else:
            assert (np.abs(d) >= 0.0029).all() and (np.abs(d) <= 0.0061).all()
            assert (d < 0).any() and (d > 0).any()
    w = synth.dequantize(ty, raw.reshape(rows, -1), rows, cols)
    assert np.isfinite(w).all() and 0.014 <= float(w.std()) <= 0.028


def test_random_block_model_runs_on_the_oracle(tmp_path, oracle):
    """A blocks="random" model is a valid GGUF for the host restatement: a
    short prefill and decode give finite logits, and a second write of the
    same seed is byte-identical."""
    cfg = synth.dataclasses.replace(synth.TINYLLAMA_MIXED_2L, name="tl-random")
    p = str(tmp_path / "r.gguf")
    sha = synth.write_model(cfg, p, seed=4, blocks="random")
    assert synth.write_model(cfg, str(tmp_path / "r2.gguf"), seed=4, blocks="random") == sha
    m = oracle.model(p, ctx=64, threads=4)
    lg = m.prefill(synth.prompt_tokens(1, 9), 32)
    assert np.isfinite(lg).all() and lg.std() > 0
    assert np.isfinite(m.forward(int(np.argmax(lg)))).all()
    m.close()
