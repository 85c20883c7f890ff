"""ctypes binding of the C ABI in include/memvanta_hip.h (libmemvanta_hip.so).

There is no fallback: if the HIP library is missing or a call fails, an
exception is raised.  Host arrays are numpy; device buffers are anything with
an integer device address (torch tensors' ``data_ptr()``).
"""
from __future__ import annotations

import ctypes as C
import os
import re
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmemvanta_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "memvanta_hip.h")

MVH_HOST, MVH_DEVICE = 0, 1
MVH_ACT_REF, MVH_ACT_Q8 = 0, 1
MVH_KV_F32, MVH_KV_F16, MVH_KV_Q8 = 0, 1, 2  # KVCacheType order
MVH_TYPE_NATIVE_Q4_0, MVH_TYPE_NATIVE_Q8_0 = 0x1002, 0x1008  # BlockQ4_0 (20 B) / BlockQ8_0 (36 B) of quant.hpp
KV_DTYPE = {MVH_KV_F32: np.float32, MVH_KV_F16: np.uint16, MVH_KV_Q8: np.int8}
STATUS = {0: "MVH_OK", 1: "MVH_E_INVALID", 2: "MVH_E_SHAPE", 3: "MVH_E_TYPE", 4: "MVH_E_DEVICE",
          5: "MVH_E_RANGE", 6: "MVH_E_NOMEM"}


class MvhError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{STATUS.get(code, code)}: {msg}")
        self.code = code
        self.msg = msg


def header_functions(path: str = HEADER) -> list[str]:
    """Names of every function the C header declares."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mvh_[a-z0-9_]+)\s*\(", text)))


_vp, _sz, _u32, _u64, _int = C.c_void_p, C.c_size_t, C.c_uint32, C.c_uint64, C.c_int
_SIGS = {
    "mvh_last_error": (C.c_char_p, []),
    "mvh_version": (_int, []),
    "mvh_device_count": (_int, [C.POINTER(_int)]),
    "mvh_context_create": (_int, [_int, C.POINTER(_vp)]),
    "mvh_context_destroy": (_int, [_vp]),
    "mvh_context_stream": (_int, [_vp, C.POINTER(_vp)]),
    "mvh_context_synchronize": (_int, [_vp]),
    "mvh_tensor_upload": (_int, [_vp, C.c_char_p, _u32, _u64, _u64, _vp, _u64, C.POINTER(_vp)]),
    "mvh_tensor_wrap": (_int, [_vp, C.c_char_p, _u32, _u64, _u64, _vp, _u64, C.POINTER(_vp)]),
    "mvh_tensor_free": (_int, [_vp]),
    "mvh_tensor_info": (_int, [_vp, C.POINTER(_u32), C.POINTER(_u64), C.POINTER(_u64), C.POINTER(_u64),
                               C.POINTER(_vp)]),
    "mvh_quantize_q8": (_int, [_vp, _vp, _sz, _sz, _vp, _vp, _int]),
    "mvh_matvec": (_int, [_vp, _vp, _vp, _vp, _int]),
    "mvh_matvec_q8": (_int, [_vp, _vp, _vp, _vp, _vp, _int]),
    "mvh_matmul_batch": (_int, [_vp, _vp, _vp, _vp, _sz, _int]),
    "mvh_matmul_batch_v06": (_int, [_vp, _vp, _vp, _vp, _sz, _int, _int]),
    "mvh_matmul_batch_v06_noalloc": (_int, [_vp, _vp, _vp, _vp, _sz, _int]),
    "mvh_read_row_f32": (_int, [_vp, _vp, _sz, _vp, _sz, _int]),
    "mvh_argmax": (_int, [_vp, _vp, _sz, _sz, _vp, _int]),
    "mvh_stream_read": (_int, [_vp, _vp, _sz, _vp, _sz]),
    "mvh_fp32_to_fp16": (_int, [_vp, _vp, _vp, _sz, _int]),
    "mvh_fp16_to_fp32": (_int, [_vp, _vp, _vp, _sz, _int]),
    "mvh_kv_parse_type": (_int, [C.c_char_p, C.POINTER(_int)]),
    "mvh_kv_type_name": (C.c_char_p, [_int]),
    "mvh_kv_create": (_int, [_vp, _sz, _sz, _sz, _sz, _int, C.POINTER(_vp)]),
    "mvh_kv_type": (_int, [_vp, C.POINTER(_int)]),
    "mvh_kv_destroy": (_int, [_vp]),
    "mvh_kv_reset": (_int, [_vp]),
    "mvh_kv_bytes_allocated": (_int, [_vp, C.POINTER(_sz)]),
    "mvh_kv_write": (_int, [_vp, _vp, _sz, _sz, _sz, _vp, _vp, _int]),
    "mvh_kv_read_row": (_int, [_vp, _vp, _sz, _sz, _int, _vp, C.POINTER(C.c_float)]),
    "mvh_attn_decode": (_int, [_vp, _vp, _sz, _vp, _sz, _sz, _sz, _sz, _vp, _int]),
    "mvh_attn_batch": (_int, [_vp, _vp, _sz, _vp, _sz, _sz, _sz, _sz, _sz, _vp, _int]),
    "mvh_model_open": (_int, [C.c_char_p, _int, _sz, _sz, _int, _int, _sz, C.POINTER(_vp)]),
    "mvh_model_kv_type": (_int, [_vp, C.POINTER(_int)]),
    "mvh_model_close": (_int, [_vp]),
    "mvh_model_config": (_int, [_vp, C.POINTER(_sz)]),
    "mvh_model_reset": (_int, [_vp]),
    "mvh_model_forward": (_int, [_vp, _int, _vp]),
    "mvh_model_prefill": (_int, [_vp, _vp, _sz, _sz, _vp]),
    "mvh_model_generate_greedy": (_int, [_vp, _int, _sz, _vp, _vp]),
    "mvh_model_position": (_int, [_vp, C.POINTER(_sz)]),
    "mvh_model_kv_bytes": (_int, [_vp, C.POINTER(_sz)]),
    "mvh_model_stream": (_int, [_vp, C.POINTER(_vp)]),
    "mvh_quantize_q8_0": (_int, [_vp, _vp, _sz, _vp, _int]),
    "mvh_quantize_q4_0": (_int, [_vp, _vp, _sz, _vp, _int]),
    "mvh_matvec_q4_q8": (_int, [_vp, _vp, _vp, _vp, _int]),
    "mvh_matmul_q4_0_batch": (_int, [_vp, _vp, _vp, _vp, _sz, _int]),
    "mvh_matvec_q4_0": (_int, [_vp, _vp, _vp, _vp, _int]),
    "mvh_matvec_q8_0": (_int, [_vp, _vp, _vp, _vp, _int]),
    "mvh_profile_enable": (None, [_int]),
    "mvh_profile_reset": (None, []),
    "mvh_profile_snapshot": (_int, [_vp, _sz, C.POINTER(_sz)]),
    "mvh_profile_kind_name": (C.c_char_p, [_int]),
}


class ProfileEntry(C.Structure):
    """mvh_profile_entry (KernelProfileEntry of include/memvanta/gguf_kernels.hpp:12-19)."""

    _fields_ = [("layer", C.c_int), ("kind", C.c_int), ("tensor", C.c_char * 192), ("calls", C.c_size_t),
                ("batch", C.c_size_t), ("ms", C.c_double)]

_lib = None


def _finalize(release, _finalizing=sys.is_finalizing) -> None:
    """Release a handle from __del__, except while the interpreter is finalizing.

    At interpreter exit the HIP runtime (torch's and this library's) may already
    be tearing down its device state; a hipFree / hipStreamDestroy issued then
    from a garbage-collected handle can touch freed runtime structures.  The
    process is ending and the driver reclaims every allocation, so the handle
    is left alone.  Explicit close()/free() calls are unaffected.  The
    finalizing test and this function are bound as default arguments: module
    globals may already be cleared when a late __del__ runs."""
    if _finalizing():
        return
    try:
        release()
    except Exception:
        pass


def load_library(path: str = LIB_PATH) -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(f"HIP backend not built: {path} is missing (run __graft_entry__.build())")
    # One HIP runtime per process: PyTorch ships its own libamdhip64.  Loaded
    # first, it also serves this library (same soname); loaded after this
    # library had brought in the system runtime, torch finds no device.  So
    # when torch is installed it is imported before the library is opened.
    if "torch" not in sys.modules:
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
    lib = C.CDLL(path)
    for name, (res, args) in _SIGS.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    _lib = lib
    return lib


def _ptr(a) -> int | None:
    if a is None:
        return None
    if isinstance(a, np.ndarray):
        if not a.flags["C_CONTIGUOUS"]:
            raise ValueError("host array must be C-contiguous")
        return a.ctypes.data
    if hasattr(a, "data_ptr"):
        return a.data_ptr()
    return int(a)


def _kind(*arrs) -> int:
    dev = [not isinstance(a, np.ndarray) for a in arrs if a is not None]
    if all(dev):
        return MVH_DEVICE
    if not any(dev):
        return MVH_HOST
    raise ValueError("mix of host and device buffers in one call")


class Context:
    """One device + one HIP stream (mvh_context)."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        h = _vp()
        self._check(self.lib.mvh_context_create(device, C.byref(h)))
        self.h = h.value
        self.device = device

    def _check(self, rc: int):
        if rc != 0:
            raise MvhError(rc, self.lib.mvh_last_error().decode())

    def close(self):
        if getattr(self, "h", None):
            self.lib.mvh_context_destroy(self.h)
            self.h = None

    def __del__(self, _fin=_finalize):
        _fin(self.close)

    @property
    def stream(self) -> int:
        s = _vp()
        self._check(self.lib.mvh_context_stream(self.h, C.byref(s)))
        return s.value

    def synchronize(self):
        self._check(self.lib.mvh_context_synchronize(self.h))

    # -- weights --
    def upload(self, name: str, ggml_type: int, ne0: int, ne1: int, data: np.ndarray) -> "Tensor":
        data = np.ascontiguousarray(data, dtype=np.uint8)
        t = _vp()
        self._check(self.lib.mvh_tensor_upload(self.h, name.encode(), ggml_type, ne0, ne1, data.ctypes.data,
                                               data.nbytes, C.byref(t)))
        return Tensor(self, t.value, name, ggml_type, ne0, ne1)

    def wrap(self, name: str, ggml_type: int, ne0: int, ne1: int, dev_ptr: int, nbytes: int) -> "Tensor":
        t = _vp()
        self._check(self.lib.mvh_tensor_wrap(self.h, name.encode(), ggml_type, ne0, ne1, dev_ptr, nbytes,
                                             C.byref(t)))
        return Tensor(self, t.value, name, ggml_type, ne0, ne1)

    # -- kernels (host numpy in/out, or device pointers) --
    def quantize_q8(self, x, q=None, d=None):
        if isinstance(x, np.ndarray):
            x = np.ascontiguousarray(x, np.float32)
            m = 1 if x.ndim == 1 else x.shape[0]
            k = x.shape[-1]
            q = np.empty(x.shape, np.int8)
            d = np.empty(x.shape[:-1] + (k // 32,), np.float32)
            self._check(self.lib.mvh_quantize_q8(self.h, x.ctypes.data, m, k, q.ctypes.data, d.ctypes.data, MVH_HOST))
            return q, d
        m = 1 if x.dim() == 1 else x.shape[0]
        k = x.shape[-1]
        self._check(self.lib.mvh_quantize_q8(self.h, _ptr(x), m, k, _ptr(q), _ptr(d), MVH_DEVICE))
        return q, d

    def matvec(self, w: "Tensor", x, y=None):
        if y is None:
            y = np.empty(w.ne1, np.float32)
            x = np.ascontiguousarray(x, np.float32)
        self._check(self.lib.mvh_matvec(self.h, w.h, _ptr(x), _ptr(y), _kind(x, y)))
        return y

    def matvec_q8(self, w: "Tensor", q, d, y=None):
        if y is None:
            q = np.ascontiguousarray(q, np.int8)
            d = np.ascontiguousarray(d, np.float32)
            y = np.empty(w.ne1, np.float32)
        self._check(self.lib.mvh_matvec_q8(self.h, w.h, _ptr(q), _ptr(d), _ptr(y), _kind(q, d, y)))
        return y

    def matmul_batch(self, w: "Tensor", x, y=None):
        b = x.shape[0]
        if y is None:
            x = np.ascontiguousarray(x, np.float32)
            y = np.empty((b, w.ne1), np.float32)
        self._check(self.lib.mvh_matmul_batch(self.h, w.h, _ptr(x), _ptr(y), b, _kind(x, y)))
        return y

    def matmul_batch_v06(self, w: "Tensor", x, act_mode: int = MVH_ACT_REF, y=None):
        b = x.shape[0]
        if y is None:
            x = np.ascontiguousarray(x, np.float32)
            y = np.empty((b, w.ne1), np.float32)
        self._check(self.lib.mvh_matmul_batch_v06(self.h, w.h, _ptr(x), _ptr(y), b, act_mode, _kind(x, y)))
        return y

    def matmul_batch_v06_noalloc(self, w: "Tensor", x, y, act_mode: int = MVH_ACT_REF):
        """mvh_matmul_batch_v06_noalloc: device x [batch][ne0] -> device y [batch][ne1], no device allocation."""
        self._check(self.lib.mvh_matmul_batch_v06_noalloc(self.h, w.h, _ptr(x), _ptr(y), x.shape[0], act_mode))
        return y

    def read_row(self, w: "Tensor", row: int, out=None, cols: int | None = None):
        """tensor_read_row_f32: row `row` of w as fp32 (cols defaults to ne0)."""
        cols = w.ne0 if cols is None else cols
        if out is None:
            out = np.empty(cols, np.float32)
        self._check(self.lib.mvh_read_row_f32(self.h, w.h, row, _ptr(out), cols, _kind(out)))
        return out

    def stream_read(self, buf, nbytes: int, sink, sink_words: int):
        """Enqueue the streaming-read probe over nbytes of device buffer buf (device sink of sink_words words)."""
        self._check(self.lib.mvh_stream_read(self.h, _ptr(buf), nbytes, _ptr(sink), sink_words))

    def argmax(self, logits, out=None):
        """Greedy sampling per row (first index of the max) of [rows][n] logits."""
        if out is None:
            logits = np.ascontiguousarray(logits, np.float32)
            rows = 1 if logits.ndim == 1 else logits.shape[0]
            out = np.empty(rows, np.int32)
        else:
            rows = 1 if logits.dim() == 1 else logits.shape[0]
        n = logits.shape[-1]
        self._check(self.lib.mvh_argmax(self.h, _ptr(logits), n, rows, _ptr(out), _kind(logits, out)))
        return out

    def fp32_to_fp16(self, x, out=None):
        if out is None:
            x = np.ascontiguousarray(x, np.float32).ravel()
            out = np.empty(x.size, np.uint16)
        n = x.size if isinstance(x, np.ndarray) else x.numel()
        self._check(self.lib.mvh_fp32_to_fp16(self.h, _ptr(x), _ptr(out), n, _kind(x, out)))
        return out

    def fp16_to_fp32(self, h, out=None):
        if out is None:
            h = np.ascontiguousarray(h, np.uint16).ravel()
            out = np.empty(h.size, np.float32)
        n = h.size if isinstance(h, np.ndarray) else h.numel()
        self._check(self.lib.mvh_fp16_to_fp32(self.h, _ptr(h), _ptr(out), n, _kind(h, out)))
        return out

    # -- native block formats (src/quant.cpp, src/quant_kernels.cpp) --
    def quantize_native(self, x, bsize: int, out=None):
        """quantize_q8_0 (bsize 36) / quantize_q4_0 (bsize 20) of the flattened x -> uint8 [n/32, bsize]."""
        fn = self.lib.mvh_quantize_q8_0 if bsize == 36 else self.lib.mvh_quantize_q4_0
        if out is None:
            x = np.ascontiguousarray(x, np.float32).ravel()
            out = np.empty((x.size // 32, bsize), np.uint8)
        n = x.size if isinstance(x, np.ndarray) else x.numel()
        self._check(fn(self.h, _ptr(x), n, _ptr(out), _kind(x, out)))
        return out

    def matvec_q4_q8(self, a: "Tensor", xq, y=None):
        if y is None:
            xq = np.ascontiguousarray(xq, np.uint8)
            y = np.empty(a.ne1, np.float32)
        self._check(self.lib.mvh_matvec_q4_q8(self.h, a.h, _ptr(xq), _ptr(y), _kind(xq, y)))
        return y

    def matmul_q4_0_batch(self, a: "Tensor", x, y=None):
        b = 1 if x.ndim == 1 else x.shape[0]
        if y is None:
            x = np.ascontiguousarray(x, np.float32)
            y = np.empty((b, a.ne1), np.float32)
        self._check(self.lib.mvh_matmul_q4_0_batch(self.h, a.h, _ptr(x), _ptr(y), b, _kind(x, y)))
        return y

    def matvec_native(self, a: "Tensor", x, y=None):
        """matvec_q4_0 / matvec_q8_0 by the tensor's native type."""
        fn = self.lib.mvh_matvec_q8_0 if a.type == MVH_TYPE_NATIVE_Q8_0 else self.lib.mvh_matvec_q4_0
        if y is None:
            x = np.ascontiguousarray(x, np.float32)
            y = np.empty(a.ne1, np.float32)
        self._check(fn(self.h, a.h, _ptr(x), _ptr(y), _kind(x, y)))
        return y

    def kv_cache(self, n_layer: int, kv_dim: int, page_tokens: int = 128, max_tokens: int = 2048,
                 kv_type: int = MVH_KV_F16) -> "KVCache":
        return KVCache(self, n_layer, kv_dim, page_tokens, max_tokens, kv_type)


class Tensor:
    def __init__(self, ctx: Context, h: int, name: str, ggml_type: int, ne0: int, ne1: int):
        self.ctx, self.h, self.name, self.type, self.ne0, self.ne1 = ctx, h, name, ggml_type, ne0, ne1

    def free(self):
        if self.h:
            self.ctx.lib.mvh_tensor_free(self.h)
            self.h = None

    def __del__(self, _fin=_finalize):
        _fin(self.free)

    def info(self):
        ty, n0, n1, nb, dp = _u32(), _u64(), _u64(), _u64(), _vp()
        self.ctx._check(self.ctx.lib.mvh_tensor_info(self.h, C.byref(ty), C.byref(n0), C.byref(n1), C.byref(nb),
                                                     C.byref(dp)))
        return ty.value, n0.value, n1.value, nb.value, dp.value


PROFILE_KINDS = ("q_proj", "k_proj", "v_proj", "o_proj", "ffn_gate", "ffn_up", "ffn_down", "output", "other")


def profile_enable(on: bool = True) -> None:
    """enable_kernel_profiling: time every tensor call and model GEMV/GEMM on the device."""
    load_library().mvh_profile_enable(1 if on else 0)


def profile_reset() -> None:
    """reset_kernel_profile."""
    load_library().mvh_profile_reset()


def profile_snapshot() -> list[dict]:
    """kernel_profile_snapshot: one dict per (layer, kind, tensor, batch) entry, in first-call order."""
    lib = load_library()
    n = _sz()
    if lib.mvh_profile_snapshot(None, 0, C.byref(n)) != 0:
        raise MvhError(1, lib.mvh_last_error().decode())
    arr = (ProfileEntry * max(1, n.value))()
    if lib.mvh_profile_snapshot(C.cast(arr, _vp), n.value, C.byref(n)) != 0:
        raise MvhError(1, lib.mvh_last_error().decode())
    return [{"layer": e.layer, "kind": e.kind, "kind_name": profile_kind_name(e.kind), "tensor": e.tensor.decode(),
             "calls": e.calls, "batch": e.batch, "ms": e.ms} for e in arr[: n.value]]


def profile_kind_name(kind: int) -> str:
    """kernel_profile_kind_name."""
    return load_library().mvh_profile_kind_name(kind).decode()


def kv_parse_type(s: str) -> int:
    """parse_kv_cache_type: "f32" / "f16" / "q8" / "q8_0" -> MVH_KV_*."""
    lib = load_library()
    t = _int()
    if lib.mvh_kv_parse_type(s.encode(), C.byref(t)) != 0:
        raise MvhError(1, lib.mvh_last_error().decode())
    return t.value


def kv_type_name(t: int) -> str:
    return load_library().mvh_kv_type_name(t).decode()


class KVCache:
    def __init__(self, ctx: Context, n_layer, kv_dim, page_tokens, max_tokens, kv_type: int = MVH_KV_F16):
        self.ctx, self.kv_dim, self.kv_type = ctx, kv_dim, kv_type
        h = _vp()
        ctx._check(ctx.lib.mvh_kv_create(ctx.h, n_layer, kv_dim, page_tokens, max_tokens, kv_type, C.byref(h)))
        self.h = h.value

    def close(self):
        if getattr(self, "h", None):
            self.ctx.lib.mvh_kv_destroy(self.h)
            self.h = None

    def __del__(self, _fin=_finalize):
        _fin(self.close)

    def reset(self):
        self.ctx._check(self.ctx.lib.mvh_kv_reset(self.h))

    def bytes_allocated(self) -> int:
        n = _sz()
        self.ctx._check(self.ctx.lib.mvh_kv_bytes_allocated(self.h, C.byref(n)))
        return n.value

    def write(self, layer, pos, k, v):
        if isinstance(k, np.ndarray):
            k = np.ascontiguousarray(k, np.float32)
            v = np.ascontiguousarray(v, np.float32)
            n = k.size // self.kv_dim
        else:
            n = k.numel() // self.kv_dim
        self.ctx._check(self.ctx.lib.mvh_kv_write(self.ctx.h, self.h, layer, pos, n, _ptr(k), _ptr(v), _kind(k, v)))

    def read_row(self, layer, pos, which):
        """(stored row: float32 / fp16 bits / int8 by cache type, Q8 row scale or 1.0)"""
        out = np.empty(self.kv_dim, KV_DTYPE[self.kv_type])
        sc = C.c_float()
        self.ctx._check(self.ctx.lib.mvh_kv_read_row(self.ctx.h, self.h, layer, pos, which, out.ctypes.data,
                                                     C.byref(sc)))
        return out, np.float32(sc.value)

    def type(self) -> int:
        t = _int()
        self.ctx._check(self.ctx.lib.mvh_kv_type(self.h, C.byref(t)))
        return t.value

    def attn_batch(self, layer, q, pos, n_tokens, n_head, n_head_kv, head_dim, out=None):
        """causal attention of n_tokens query tokens at positions pos.. (q: [n_tokens][n_head*head_dim])"""
        if out is None:
            q = np.ascontiguousarray(q, np.float32)
            out = np.empty((n_tokens, n_head * head_dim), np.float32)
        self.ctx._check(self.ctx.lib.mvh_attn_batch(self.ctx.h, self.h, layer, _ptr(q), pos, n_tokens, n_head,
                                                    n_head_kv, head_dim, _ptr(out), _kind(q, out)))
        return out

    def attn_decode(self, layer, q, pos, n_head, n_head_kv, head_dim, out=None):
        if out is None:
            q = np.ascontiguousarray(q, np.float32)
            out = np.empty(n_head * head_dim, np.float32)
        self.ctx._check(self.ctx.lib.mvh_attn_decode(self.ctx.h, self.h, layer, _ptr(q), pos, n_head, n_head_kv,
                                                     head_dim, _ptr(out), _kind(q, out)))
        return out


class Model:
    """LlamaModel on one device (mvh_model_*)."""

    def __init__(self, path: str, device: int = 0, ctx: int = 0, page_tokens: int = 128,
                 act_mode: int = MVH_ACT_Q8, max_batch: int = 64, kv_type: int = MVH_KV_F16):
        self.lib = load_library()
        h = _vp()
        rc = self.lib.mvh_model_open(path.encode(), device, ctx, page_tokens, kv_type, act_mode, max_batch,
                                     C.byref(h))
        self._check(rc)
        self.h = h.value
        cfg = (_sz * 7)()
        self._check(self.lib.mvh_model_config(self.h, cfg))
        self.n_ctx, self.n_embd, self.n_ff, self.n_layer, self.n_head, self.n_head_kv, self.vocab = list(cfg)

    def _check(self, rc):
        if rc != 0:
            raise MvhError(rc, self.lib.mvh_last_error().decode())

    def close(self):
        if getattr(self, "h", None):
            self.lib.mvh_model_close(self.h)
            self.h = None

    def __del__(self, _fin=_finalize):
        _fin(self.close)

    def reset(self):
        self._check(self.lib.mvh_model_reset(self.h))

    def forward(self, token: int, logits: bool = True):
        out = np.empty(self.vocab, np.float32) if logits else None
        self._check(self.lib.mvh_model_forward(self.h, int(token), out.ctypes.data if logits else None))
        return out

    def prefill(self, tokens, batch: int = 32, logits: bool = True):
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.empty(self.vocab, np.float32) if logits else None
        self._check(self.lib.mvh_model_prefill(self.h, t.ctypes.data, t.size, batch, out.ctypes.data if logits else None))
        return out

    def generate_greedy(self, token: int, n: int, logits: bool = False):
        ids = np.empty(n, np.int32)
        out = np.empty(self.vocab, np.float32) if logits else None
        self._check(self.lib.mvh_model_generate_greedy(self.h, int(token), n, ids.ctypes.data,
                                                       out.ctypes.data if logits else None))
        return (ids, out) if logits else ids

    @property
    def position(self) -> int:
        p = _sz()
        self._check(self.lib.mvh_model_position(self.h, C.byref(p)))
        return p.value

    def kv_type(self) -> int:
        t = _int()
        self._check(self.lib.mvh_model_kv_type(self.h, C.byref(t)))
        return t.value

    def kv_bytes(self) -> int:
        p = _sz()
        self._check(self.lib.mvh_model_kv_bytes(self.h, C.byref(p)))
        return p.value

    @property
    def stream(self) -> int:
        s = _vp()
        self._check(self.lib.mvh_model_stream(self.h, C.byref(s)))
        return s.value
