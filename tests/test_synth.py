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
