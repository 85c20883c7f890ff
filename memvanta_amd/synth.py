"""Synthetic GGUF inputs for the quantized-matmul hot path.

Writes GGUF v3 files with the reference's on-disk tensor layouts (GGML order:
ne0 = cols/K, ne1 = rows/N; Q4_0 18-byte, Q8_0 34-byte, Q6_K 210-byte blocks)
so that the HIP backend, the CPU oracle and the compiled reference all read the
same bytes.  Quantizers are deterministic numpy restatements of the GGML block
formats (any fixed choice is valid: every consumer reads the same bytes):

* Q4_0: d = v/-8 where v is the signed element of largest magnitude,
  q = min(15, int(x/d + 8.5)); nibble i holds q[i] | q[i+16] << 4
  (GGUF order, as documented in scripts/make_tiny_gguf.py:14-24).
* Q8_0: d = amax/127, q = round(x/d).
* Q6_K: per 16-element sub-block scale, super-block d = max|scale|/127,
  q in [-32, 31] stored with the bit map of q6_k_value
  (src/gguf_kernels.cpp:122-136).

Model configurations follow the random-init llama shapes the benchmarks use
(norm weights 1.0, eps 1e-5, rope theta 1e4, tokenizer = placeholder tokens).
"""
from __future__ import annotations

import dataclasses
import hashlib
import os
import struct
from typing import Callable, Iterable

import numpy as np

F32, F16, Q4_0, Q8_0, Q6_K = 0, 1, 2, 8, 14
TYPE_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q8_0: "Q8_0", Q6_K: "Q6_K"}
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q6_K: (256, 210), F32: (1, 4), F16: (1, 2)}


def row_bytes(ty: int, cols: int) -> int:
    qk, bs = BLOCK[ty]
    if cols % qk:
        raise ValueError(f"{TYPE_NAMES[ty]} needs cols % {qk} == 0, got {cols}")
    return cols // qk * bs


# --------------------------------------------------------------------------
# quantizers (x: float32 [rows, cols] -> uint8 [rows, row_bytes])
# --------------------------------------------------------------------------

def quantize_q4_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    b = x.reshape(rows, cols // 32, 32)
    idx = np.abs(b).argmax(axis=2)
    v = np.take_along_axis(b, idx[..., None], axis=2)[..., 0]
    d = (v / np.float32(-8.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    q = np.minimum(15, (b * inv[..., None] + np.float32(8.5)).astype(np.int8)).astype(np.uint8)
    out = np.empty((rows, cols // 32, 18), dtype=np.uint8)
    out[..., 0:2] = d.astype(np.float16).view(np.uint8).reshape(rows, cols // 32, 2)
    out[..., 2:18] = q[..., :16] | (q[..., 16:] << 4)
    return out.reshape(rows, -1)


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    b = x.reshape(rows, cols // 32, 32)
    d = (np.abs(b).max(axis=2) / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    q = np.clip(np.rint(b * inv[..., None]), -127, 127).astype(np.int8)
    out = np.empty((rows, cols // 32, 34), dtype=np.uint8)
    out[..., 0:2] = d.astype(np.float16).view(np.uint8).reshape(rows, cols // 32, 2)
    out[..., 2:34] = q.view(np.uint8)
    return out.reshape(rows, -1)


def _q6k_maps():
    i = np.arange(256)
    row32, j = i // 32, i % 32
    group, local = row32 // 4, row32 % 4
    ql_index = group * 64 + (local % 2) * 32 + j
    ql_shift = np.where(local < 2, 0, 4)
    qh_index = group * 32 + j
    qh_shift = local * 2
    # inverse maps: which element lands in each ql byte (shift 0, 4) / qh byte (shift 0,2,4,6)
    ql_src = np.zeros((128, 2), dtype=np.int64)
    qh_src = np.zeros((64, 4), dtype=np.int64)
    ql_src[ql_index, ql_shift // 4] = i
    qh_src[qh_index, qh_shift // 2] = i
    return ql_src, qh_src


_QL_SRC, _QH_SRC = _q6k_maps()


def quantize_q6_k(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    nsb = cols // 256
    b = x.reshape(rows * nsb, 16, 16)
    scale = (np.abs(b).max(axis=2) / np.float32(31.0)).astype(np.float32)  # [n,16]
    d = (scale.max(axis=1) / np.float32(127.0)).astype(np.float32)
    d16 = d.astype(np.float16)
    df = d16.astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(df[:, None] != 0, np.rint(scale / df[:, None]), 0)
    sc = np.clip(sc, -128, 127).astype(np.int8)
    eff = (df[:, None] * sc.astype(np.float32)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(eff[..., None] != 0, np.rint(b / eff[..., None]), 0)
    q = (np.clip(q, -32, 31) + 32).astype(np.uint8).reshape(-1, 256)
    lo, hi = q & 15, q >> 4
    out = np.empty((rows * nsb, 210), dtype=np.uint8)
    out[:, 0:128] = lo[:, _QL_SRC[:, 0]] | (lo[:, _QL_SRC[:, 1]] << 4)
    out[:, 128:192] = (hi[:, _QH_SRC[:, 0]] | (hi[:, _QH_SRC[:, 1]] << 2)
                       | (hi[:, _QH_SRC[:, 2]] << 4) | (hi[:, _QH_SRC[:, 3]] << 6))
    out[:, 192:208] = sc.view(np.uint8)
    out[:, 208:210] = d16.view(np.uint8).reshape(-1, 2)
    return out.reshape(rows, -1)


def quantize_torch(ty: int, x):
    """The same quantizers on a torch float32 [rows, cols] tensor, on any device
    (byte-identical to the numpy ones for the same input); returns uint8
    [rows, row_bytes] on x's device.  Used to synthesize multi-GB models fast."""
    import torch

    rows, cols = x.shape
    u8 = torch.uint8
    if ty == Q4_0:
        b = x.reshape(rows, cols // 32, 32)
        v = b.gather(2, b.abs().argmax(dim=2, keepdim=True))[..., 0]
        d = v / -8.0
        inv = torch.where(d != 0, 1.0 / d, torch.zeros_like(d))
        q = torch.clamp_max((b * inv[..., None] + 8.5).to(torch.int8), 15).to(u8)
        out = torch.empty((rows, cols // 32, 18), dtype=u8, device=x.device)
        out[..., 0:2] = d.to(torch.float16).view(u8).reshape(rows, cols // 32, 2)
        out[..., 2:18] = q[..., :16] | (q[..., 16:] << 4)
        return out.reshape(rows, -1)
    if ty == Q8_0:
        b = x.reshape(rows, cols // 32, 32)
        d = b.abs().amax(dim=2) / 127.0
        inv = torch.where(d != 0, 1.0 / d, torch.zeros_like(d))
        q = torch.clamp(torch.round(b * inv[..., None]), -127, 127).to(torch.int8)
        out = torch.empty((rows, cols // 32, 34), dtype=u8, device=x.device)
        out[..., 0:2] = d.to(torch.float16).view(u8).reshape(rows, cols // 32, 2)
        out[..., 2:34] = q.view(u8)
        return out.reshape(rows, -1)
    if ty == Q6_K:
        nsb = cols // 256
        b = x.reshape(rows * nsb, 16, 16)
        scale = b.abs().amax(dim=2) / 31.0
        d16 = (scale.amax(dim=1) / 127.0).to(torch.float16)
        df = d16.float()[:, None]
        sc = torch.where(df != 0, torch.round(scale / df), torch.zeros_like(scale))
        sc = torch.clamp(sc, -128, 127).to(torch.int8)
        eff = (df * sc.float())[..., None]
        q = torch.where(eff != 0, torch.round(b / eff), torch.zeros_like(b))
        q = (torch.clamp(q, -32, 31) + 32).to(u8).reshape(-1, 256)
        lo, hi = q & 15, q >> 4
        ql = torch.as_tensor(_QL_SRC, device=x.device)
        qh = torch.as_tensor(_QH_SRC, device=x.device)
        out = torch.empty((rows * nsb, 210), dtype=u8, device=x.device)
        out[:, 0:128] = lo[:, ql[:, 0]] | (lo[:, ql[:, 1]] << 4)
        out[:, 128:192] = (hi[:, qh[:, 0]] | (hi[:, qh[:, 1]] << 2) | (hi[:, qh[:, 2]] << 4)
                           | (hi[:, qh[:, 3]] << 6))
        out[:, 192:208] = sc.view(u8)
        out[:, 208:210] = d16.view(u8).reshape(-1, 2)
        return out.reshape(rows, -1)
    if ty == F32:
        return x.contiguous().view(u8).reshape(rows, -1)
    raise ValueError(f"unsupported type {ty}")


# ---- native MemVanta blocks (src/quant.cpp:44-85), not GGUF: BlockQ4_0 =
# {float d; uint8 qs[16]} (20 bytes, element 2i in the low nibble of qs[i],
# 2i+1 in the high nibble), BlockQ8_0 = {float d; int8 qs[32]} (36 bytes).
# Same arithmetic as quantize_q4_0 / quantize_q8_0 there: f32 amax/7 (amax/127),
# f32 reciprocal, f32 product, round half to even, clamp; a zero block stores
# d = 0 and zero bytes (not the nibble of zero).

def _native_scales(xb: np.ndarray, div: float):
    amax = np.max(np.abs(xb), axis=-1)
    d = (amax / np.float32(div)).astype(np.float32)
    with np.errstate(divide="ignore", over="ignore"):
        inv = np.where(d == 0, np.float32(0), np.float32(1) / np.where(d == 0, np.float32(1), d)).astype(np.float32)
    return d, inv


def _x86_round_int(v: np.ndarray) -> np.ndarray:
    """int(nearbyint(v)) as the reference's x86 build converts: round half to
    even, and INT_MIN for NaN / infinities (a block so small that 1/d overflows)."""
    with np.errstate(invalid="ignore"):
        r = np.rint(v)
        return np.where(np.abs(r) < 2.0 ** 31, r, -(2.0 ** 31))


def quantize_q8_0_native(x: np.ndarray) -> np.ndarray:
    """[..., K] fp32 -> uint8 [..., K/32, 36] (quantize_q8_0, src/quant.cpp:44-62)."""
    x = np.ascontiguousarray(x, np.float32)
    xb = x.reshape(x.shape[:-1] + (x.shape[-1] // 32, 32))
    d, inv = _native_scales(xb, 127.0)
    with np.errstate(invalid="ignore", over="ignore"):
        q = np.clip(_x86_round_int(xb * inv[..., None]), -127, 127).astype(np.int8)
    out = np.empty(xb.shape[:-1] + (36,), np.uint8)
    out[..., :4] = d[..., None].view(np.uint8).reshape(d.shape + (4,))
    out[..., 4:] = q.view(np.uint8)
    return out


def quantize_q4_0_native(x: np.ndarray) -> np.ndarray:
    """[..., K] fp32 -> uint8 [..., K/32, 20] (quantize_q4_0, src/quant.cpp:64-85)."""
    x = np.ascontiguousarray(x, np.float32)
    xb = x.reshape(x.shape[:-1] + (x.shape[-1] // 32, 32))
    d, inv = _native_scales(xb, 7.0)
    with np.errstate(invalid="ignore", over="ignore"):
        q = (np.clip(_x86_round_int(xb * inv[..., None]), -8, 7) + 8).astype(np.uint8)
    out = np.empty(xb.shape[:-1] + (20,), np.uint8)
    out[..., :4] = d[..., None].view(np.uint8).reshape(d.shape + (4,))
    out[..., 4:] = np.where((d == 0)[..., None], np.uint8(0), q[..., 0::2] | (q[..., 1::2] << 4))
    return out


def quantize(ty: int, x: np.ndarray) -> np.ndarray:
    if ty == Q4_0:
        return quantize_q4_0(x)
    if ty == Q8_0:
        return quantize_q8_0(x)
    if ty == Q6_K:
        return quantize_q6_k(x)
    if ty == F32:
        return np.ascontiguousarray(x, dtype=np.float32).view(np.uint8).reshape(x.shape[0], -1)
    if ty == F16:
        return np.ascontiguousarray(x, dtype=np.float16).view(np.uint8).reshape(x.shape[0], -1)
    raise ValueError(f"unsupported type {ty}")


# --------------------------------------------------------------------------
# dequantizers (fp64 brute-force references for tests)
# --------------------------------------------------------------------------

def _f16(b: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(b).view(np.float16).astype(np.float64)[..., 0]


def dequantize(ty: int, w: np.ndarray, rows: int, cols: int) -> np.ndarray:
    w = np.asarray(w, dtype=np.uint8).reshape(rows, -1)
    if ty == Q4_0:
        b = w.reshape(rows, cols // 32, 18)
        d = _f16(b[..., 0:2])
        qs = b[..., 2:18]
        q = np.concatenate([(qs & 15).astype(np.int64) - 8, (qs >> 4).astype(np.int64) - 8], axis=2)
        return (q * d[..., None]).reshape(rows, cols)
    if ty == Q8_0:
        b = w.reshape(rows, cols // 32, 34)
        d = _f16(b[..., 0:2])
        q = b[..., 2:34].view(np.int8).astype(np.int64)
        return (q * d[..., None]).reshape(rows, cols)
    if ty == Q6_K:
        b = w.reshape(rows * (cols // 256), 210)
        i = np.arange(256)
        row32, j = i // 32, i % 32
        group, local = row32 // 4, row32 % 4
        lo = (b[:, group * 64 + (local % 2) * 32 + j] >> np.where(local < 2, 0, 4)) & 15
        hi = (b[:, 128 + group * 32 + j] >> (local * 2)) & 3
        q = (lo | (hi << 4)).astype(np.int64) - 32
        sc = b[:, 192:208].view(np.int8).astype(np.float64)
        d = _f16(b[:, 208:210])
        # reference rounding: w = float32(float32(d*sc)*q)
        ds = (d.astype(np.float32)[:, None] * sc.astype(np.float32)).astype(np.float32)
        wv = (ds[:, i // 16] * q.astype(np.float32)).astype(np.float32)
        return wv.astype(np.float64).reshape(rows, cols)
    if ty == F32:
        return w.view(np.float32).astype(np.float64).reshape(rows, cols)
    if ty == F16:
        return w.view(np.float16).astype(np.float64).reshape(rows, cols)
    raise ValueError(ty)


# --------------------------------------------------------------------------
# GGUF v3 writer
# --------------------------------------------------------------------------

_U32, _F32, _BOOL, _STR, _ARR = 4, 6, 7, 8, 9


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


@dataclasses.dataclass
class _Tensor:
    name: str
    dims: tuple  # GGML order
    ty: int
    nbytes: int
    produce: Callable[[], Iterable[bytes]]


class GgufWriter:
    """Streams a GGUF v3 file; tensor bytes are produced lazily, chunk by chunk."""

    def __init__(self, alignment: int = 32):
        self.alignment = alignment
        self.meta: list[bytes] = []
        self.tensors: list[_Tensor] = []
        self.add_u32("general.alignment", alignment)

    def add_str(self, k, v):
        self.meta.append(_s(k) + struct.pack("<I", _STR) + _s(v))

    def add_u32(self, k, v):
        self.meta.append(_s(k) + struct.pack("<II", _U32, v))

    def add_f32(self, k, v):
        self.meta.append(_s(k) + struct.pack("<If", _F32, v))

    def add_str_array(self, k, arr):
        self.meta.append(_s(k) + struct.pack("<IIQ", _ARR, _STR, len(arr)) + b"".join(_s(a) for a in arr))

    def add_tensor(self, name, dims, ty, nbytes, produce):
        self.tensors.append(_Tensor(name, tuple(int(d) for d in dims), ty, int(nbytes), produce))

    def write(self, path: str) -> None:
        al = self.alignment
        offsets, off = [], 0
        for t in self.tensors:
            off = (off + al - 1) // al * al
            offsets.append(off)
            off += t.nbytes
        hdr = b"GGUF" + struct.pack("<IQQ", 3, len(self.tensors), len(self.meta)) + b"".join(self.meta)
        ti = b"".join(_s(t.name) + struct.pack("<I", len(t.dims)) + struct.pack(f"<{len(t.dims)}Q", *t.dims)
                      + struct.pack("<IQ", t.ty, o) for t, o in zip(self.tensors, offsets))
        prefix = hdr + ti
        data_start = (len(prefix) + al - 1) // al * al
        tmp = path + ".tmp"
        with open(tmp, "wb") as f:
            f.write(prefix + b"\0" * (data_start - len(prefix)))
            for t, o in zip(self.tensors, offsets):
                pos = f.tell() - data_start
                if pos < o:
                    f.write(b"\0" * (o - pos))
                n = 0
                for chunk in t.produce():
                    f.write(chunk)
                    n += len(chunk)
                if n != t.nbytes:
                    raise RuntimeError(f"{t.name}: produced {n} bytes, expected {t.nbytes}")
        os.replace(tmp, path)


def normal_quantized(ty: int, rows: int, cols: int, rng: np.random.Generator, std: float = 0.02,
                     chunk_rows: int = 1024):
    """Producer of N(0, std) weights quantized to `ty`, generated in row chunks."""

    def produce():
        for r0 in range(0, rows, chunk_rows):
            n = min(chunk_rows, rows - r0)
            x = rng.standard_normal((n, cols), dtype=np.float32) * np.float32(std)
            yield quantize(ty, x).tobytes()

    return produce


def normal_quantized_torch(ty: int, rows: int, cols: int, gen, std: float = 0.02, chunk_elems: int = 1 << 26):
    """Producer of N(0, std) weights drawn and quantized on gen's device (a
    torch.Generator); a different random stream from normal_quantized."""
    import torch

    chunk_rows = max(1, chunk_elems // cols)

    def produce():
        for r0 in range(0, rows, chunk_rows):
            n = min(chunk_rows, rows - r0)
            x = torch.randn((n, cols), generator=gen, device=gen.device, dtype=torch.float32) * std
            yield quantize_torch(ty, x).cpu().numpy().tobytes()

    return produce


def random_blocks(ty: int, rows: int, cols: int, rng: np.random.Generator, chunk_rows: int = 4096):
    """Producer of valid blocks drawn directly as bytes (no float weights to
    quantize, so a 7B-shape model takes seconds on any host and the bytes are
    the same on every machine): uniform random quant codes with scales that
    give the weights a standard deviation of about 0.02, as N(0, 0.02)
    weights have (larger weights make a deep random model amplify a
    one-ulp difference of a double sum's rounding layer after layer) --
    Q4_0: d = +-U(0.003, 0.006), nibbles uniform;
    Q8_0: d = U(1.5e-4, 3.5e-4), int8 codes uniform in [-127, 127];
    Q6_K: d = U(1.8e-5, 3.6e-5) (fp16 subnormals), 6-bit codes uniform, int8
    sub-block scales uniform in [-64, 63]."""
    if ty not in (Q4_0, Q8_0, Q6_K):
        raise ValueError(f"random blocks: unsupported type {TYPE_NAMES.get(ty, ty)}")
    _, bs = BLOCK[ty]

    def f16(v):
        return v.astype(np.float16).view(np.uint8).reshape(-1, 2)

    def produce():
        for r0 in range(0, rows, chunk_rows):
            n = min(chunk_rows, rows - r0)
            raw = rng.integers(0, 256, n * row_bytes(ty, cols), dtype=np.uint8)
            b = raw.reshape(-1, bs)
            nb = b.shape[0]
            if ty == Q4_0:
                sign = np.where(rng.integers(0, 256, nb, dtype=np.uint8) & 1, -1.0, 1.0)
                b[:, 0:2] = f16(rng.uniform(0.003, 0.006, nb) * sign)
            elif ty == Q8_0:
                b[:, 0:2] = f16(rng.uniform(1.5e-4, 3.5e-4, nb))
                q = b[:, 2:].view(np.int8)
                np.maximum(q, -127, out=q)
            else:
                b[:, 192:208] = rng.integers(-64, 64, (nb, 16), dtype=np.int8).view(np.uint8)
                b[:, 208:210] = f16(rng.uniform(1.8e-5, 3.6e-5, nb))
            yield raw.tobytes()

    return produce


# --------------------------------------------------------------------------
# model + matrix configurations
# --------------------------------------------------------------------------

@dataclasses.dataclass(frozen=True)
class ModelConfig:
    name: str
    dim: int
    ffn: int
    layers: int
    heads: int
    kv_heads: int
    vocab: int
    ctx: int
    wtype: int                # attention + FFN weights
    embd_type: int
    out_type: int
    down_type: int | None = None  # ffn_down override

    @property
    def head_dim(self):
        return self.dim // self.heads


TINY = ModelConfig("tiny-llama-288", 288, 768, 6, 6, 6, 32000, 256, Q4_0, Q8_0, Q8_0)
TINYLLAMA_MIXED = ModelConfig("tinyllama-1.1b-mixed", 2048, 5632, 22, 32, 4, 32000, 2048, Q8_0, Q8_0, Q6_K, Q6_K)
LLAMA7B = ModelConfig("openllama-7b-v2-q4_0", 4096, 11008, 32, 32, 32, 32000, 2048, Q4_0, Q4_0, Q6_K)
# reduced-depth variants of the two large shapes, for end-to-end parity runs
TINYLLAMA_MIXED_2L = dataclasses.replace(TINYLLAMA_MIXED, name="tinyllama-1.1b-mixed-2layer", layers=2, ctx=256)
LLAMA7B_1L = dataclasses.replace(LLAMA7B, name="openllama-7b-v2-q4_0-1layer", layers=1, ctx=256)
CONFIGS = {c.name: c for c in (TINY, TINYLLAMA_MIXED, LLAMA7B, TINYLLAMA_MIXED_2L, LLAMA7B_1L)}


def write_model(cfg: ModelConfig, path: str, seed: int = 1234, std: float = 0.02, device: str | None = None,
                digest: bool = True, blocks: str = "normal") -> str | None:
    """Random-init llama GGUF; returns the sha256 of the file (None when
    digest=False).  With `device` (e.g. "cuda"), weights are drawn and
    quantized there by torch: seconds for a 7B shape instead of minutes, but a
    different random stream from the default numpy one.  blocks="random":
    every matrix from random_blocks (seconds on the host, the same bytes
    everywhere; `device` and `std` are then unused)."""
    if blocks not in ("normal", "random"):
        raise ValueError(f"blocks must be 'normal' or 'random', got {blocks!r}")
    rng = np.random.default_rng(seed)
    gen = None
    if device is not None and blocks == "normal":
        import torch

        gen = torch.Generator(device=device)
        gen.manual_seed(seed)
    w = GgufWriter()
    w.add_str("general.architecture", "llama")
    w.add_str("general.name", cfg.name)
    w.add_u32("llama.context_length", cfg.ctx)
    w.add_u32("llama.embedding_length", cfg.dim)
    w.add_u32("llama.feed_forward_length", cfg.ffn)
    w.add_u32("llama.block_count", cfg.layers)
    w.add_u32("llama.attention.head_count", cfg.heads)
    w.add_u32("llama.attention.head_count_kv", cfg.kv_heads)
    w.add_f32("llama.attention.layer_norm_rms_epsilon", 1e-5)
    w.add_f32("llama.rope.freq_base", 10000.0)
    w.add_str_array("tokenizer.ggml.tokens", [f"<t{i}>" for i in range(cfg.vocab)])
    w.add_u32("tokenizer.ggml.bos_token_id", 1)
    w.add_u32("tokenizer.ggml.eos_token_id", 2)
    D, F, kv = cfg.dim, cfg.ffn, cfg.kv_heads * cfg.head_dim

    def mat(name, rows, cols, ty):
        if blocks == "random":
            prod = random_blocks(ty, rows, cols, rng)
        elif gen is None:
            prod = normal_quantized(ty, rows, cols, rng, std)
        else:
            prod = normal_quantized_torch(ty, rows, cols, gen, std)
        w.add_tensor(name, (cols, rows), ty, rows * row_bytes(ty, cols), prod)

    def ones(name, n):
        w.add_tensor(name, (n,), F32, 4 * n, lambda: iter([np.ones(n, np.float32).tobytes()]))

    mat("token_embd.weight", cfg.vocab, D, cfg.embd_type)
    for i in range(cfg.layers):
        ones(f"blk.{i}.attn_norm.weight", D)
        mat(f"blk.{i}.attn_q.weight", D, D, cfg.wtype)
        mat(f"blk.{i}.attn_k.weight", kv, D, cfg.wtype)
        mat(f"blk.{i}.attn_v.weight", kv, D, cfg.wtype)
        mat(f"blk.{i}.attn_output.weight", D, D, cfg.wtype)
        ones(f"blk.{i}.ffn_norm.weight", D)
        mat(f"blk.{i}.ffn_gate.weight", F, D, cfg.wtype)
        mat(f"blk.{i}.ffn_up.weight", F, D, cfg.wtype)
        mat(f"blk.{i}.ffn_down.weight", D, F, cfg.down_type if cfg.down_type is not None else cfg.wtype)
    ones("output_norm.weight", D)
    mat("output.weight", cfg.vocab, D, cfg.out_type)
    w.write(path)
    return file_sha256(path) if digest else None


def write_matrices(path: str, mats: list[tuple[str, int, int, int]], seed: int = 7, std: float = 0.02) -> None:
    """GGUF holding only weight matrices: (name, rows, cols, type) each N(0, std)."""
    rng = np.random.default_rng(seed)
    w = GgufWriter()
    w.add_str("general.architecture", "matrices")
    for name, rows, cols, ty in mats:
        w.add_tensor(name, (cols, rows), ty, rows * row_bytes(ty, cols), normal_quantized(ty, rows, cols, rng, std))
    w.write(path)


def file_sha256(path: str) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 24), b""):
            h.update(chunk)
    return h.hexdigest()


def activations(rng: np.random.Generator, m: int, k: int, outlier_frac: float = 0.001,
                outlier: float = 20.0) -> np.ndarray:
    """N(0,1) activations with a seeded fraction of +-outlier entries."""
    x = rng.standard_normal((m, k), dtype=np.float32)
    n_out = int(round(outlier_frac * m * k))
    if n_out:
        pos = rng.choice(m * k, size=n_out, replace=False)
        sign = rng.choice(np.array([-1.0, 1.0], np.float32), size=n_out)
        x.reshape(-1)[pos] = sign * np.float32(outlier)
    return x


def prompt_tokens(seed: int, n: int, vocab: int = 32000) -> np.ndarray:
    return np.random.default_rng(seed).integers(0, vocab, size=n, dtype=np.int64).astype(np.int32)
