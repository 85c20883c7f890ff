"""ctypes bindings of the oracle libraries -- TEST INFRASTRUCTURE ONLY.

* ``Oracle`` wraps liboracle.so, the C restatement of MemVanta's path
  (mv_oracle.c).
* ``Ref`` wraps _ref/libmvref.so, MemVanta's own sources compiled by
  oracle/Makefile; present only where the reference checkout was available at
  build time.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only to check or time the CPU side.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libmvref.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_szp = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")
_sz = C.c_size_t

# KV cache types (PagedKVCache's KVCacheType order) and their stored element types
KV_F32, KV_F16, KV_Q8 = 0, 1, 2
KV_DTYPE = {KV_F32: np.float32, KV_F16: np.uint16, KV_Q8: np.int8}


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class _Native:
    """Native block formats of src/quant.cpp / src/quant_kernels.cpp (BlockQ4_0 =
    20 bytes, BlockQ8_0 = 36 bytes, as uint8 arrays [..., nblocks, 20 or 36])."""

    _nq = ""  # symbol prefix: "mvo_nq_" (oracle) or "mvr_nq_" (reference)

    def _bind_native(self):
        L, p = self.lib, self._nq
        getattr(L, p + "quantize_q8_0").argtypes = [_f32p, _sz, _u8p]
        getattr(L, p + "quantize_q4_0").argtypes = [_f32p, _sz, _u8p]
        getattr(L, p + "matvec_q4_q8").argtypes = [_u8p, _u8p, _f32p, _sz, _sz, C.c_uint]
        getattr(L, p + "matmul_q4_0_batch").argtypes = [_u8p, _f32p, _f32p, _sz, _sz, _sz, C.c_uint]
        getattr(L, p + "matvec_q4_0").argtypes = [_u8p, _f32p, _f32p, _sz, _sz, C.c_uint]
        getattr(L, p + "matvec_q8_0").argtypes = [_u8p, _f32p, _f32p, _sz, _sz, C.c_uint]

    def nq_quantize(self, x, bsize):
        """quantize_q8_0 (bsize 36) / quantize_q4_0 (bsize 20) of the flattened x."""
        x = _f32(x).ravel()
        out = np.zeros((max(x.size // 32, 1), bsize), np.uint8)
        fn = getattr(self.lib, self._nq + ("quantize_q8_0" if bsize == 36 else "quantize_q4_0"))
        self._check(fn(x, x.size, out))
        return out[: x.size // 32]

    def nq_matvec_q4_q8(self, A, xq, rows, cols, threads=8):
        y = np.empty(rows, np.float32)
        self._check(getattr(self.lib, self._nq + "matvec_q4_q8")(np.ascontiguousarray(A, np.uint8).ravel(),
                                                                   np.ascontiguousarray(xq, np.uint8).ravel(), y, rows,
                                                                   cols, threads))
        return y

    def nq_matmul_q4_0_batch(self, A, X, rows, cols, threads=8):
        X = _f32(X)
        batch = 1 if X.ndim == 1 else X.shape[0]
        y = np.empty((batch, rows), np.float32)
        self._check(getattr(self.lib, self._nq + "matmul_q4_0_batch")(np.ascontiguousarray(A, np.uint8).ravel(),
                                                                        X.ravel(), y, rows, cols, batch, threads))
        return y

    def nq_matvec(self, A, x, rows, cols, bsize, threads=8):
        """matvec_q4_0 (bsize 20) / matvec_q8_0 (bsize 36), fp32 activations."""
        y = np.empty(rows, np.float32)
        fn = getattr(self.lib, self._nq + ("matvec_q8_0" if bsize == 36 else "matvec_q4_0"))
        self._check(fn(np.ascontiguousarray(A, np.uint8).ravel(), _f32(x).ravel(), y, rows, cols, threads))
        return y


class Oracle(_Native):
    _nq = "mvo_nq_"

    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle oracle`")
        L = self.lib = C.CDLL(path)
        L.mvo_last_error.restype = C.c_char_p
        L.mvo_fp16_to_fp32.restype = C.c_float
        L.mvo_fp16_to_fp32.argtypes = [C.c_uint16]
        L.mvo_fp32_to_fp16.restype = C.c_uint16
        L.mvo_fp32_to_fp16.argtypes = [C.c_float]
        L.mvo_fp32_to_fp16_n.argtypes = [_f32p, _u16p, _sz]
        L.mvo_fp32_to_fp16_bits.argtypes = [C.c_uint32, C.c_uint64, _u16p]
        L.mvo_fp32_to_fp16_count_mismatch.argtypes = [C.c_uint32, C.c_uint64, _u16p]
        L.mvo_fp32_to_fp16_count_mismatch.restype = C.c_uint64
        L.mvo_quantize_q8.argtypes = [_f32p, _sz, _i8p, _f32p]
        L.mvo_quantize_act_q8.argtypes = [_f32p, _sz, _sz, _i8p, _f32p]
        L.mvo_matvec.argtypes = [_u8p, C.c_int, _sz, _sz, _f32p, _f32p, C.c_int]
        L.mvo_matmul_batch.argtypes = [_u8p, C.c_int, _sz, _sz, _f32p, _f32p, _sz, C.c_int]
        L.mvo_matmul_batch_v06.argtypes = [_u8p, C.c_int, _sz, _sz, C.c_int, C.c_int, _f32p, _f32p, _sz, C.c_int]
        L.mvo_read_row_f32.argtypes = [_u8p, C.c_int, _sz, _sz, _sz, _f32p]
        L.mvo_kv_parse_type.argtypes = [C.c_char_p]
        L.mvo_kv_type_name.restype = C.c_char_p
        L.mvo_kv_type_name.argtypes = [C.c_int]
        L.mvo_kv_create.restype = C.c_void_p
        L.mvo_kv_create.argtypes = [_sz, _sz, C.c_int]
        L.mvo_kv_destroy.argtypes = [C.c_void_p]
        L.mvo_kv_reset.argtypes = [C.c_void_p]
        L.mvo_kv_write.argtypes = [C.c_void_p, _sz, _f32p, _f32p]
        L.mvo_kv_dot_key.restype = C.c_float
        L.mvo_kv_dot_key.argtypes = [C.c_void_p, _sz, _sz, _f32p, _sz]
        L.mvo_kv_add_value.argtypes = [C.c_void_p, _sz, _sz, C.c_float, _f32p, _sz]
        L.mvo_kv_bytes_allocated.restype = _sz
        L.mvo_kv_bytes_allocated.argtypes = [C.c_void_p]
        L.mvo_kv_row.restype = C.c_void_p
        L.mvo_kv_row.argtypes = [C.c_void_p, _sz, C.c_int, C.POINTER(C.c_float)]
        L.mvo_attn_decode.argtypes = [C.c_void_p, _f32p, _sz, _sz, _sz, _sz, _f32p]
        L.mvo_rmsnorm.argtypes = [_f32p, _f32p, _sz, C.c_float, _f32p]
        L.mvo_rope_table.argtypes = [_sz, _sz, C.c_float, _f32p, _f32p]
        L.mvo_rope.argtypes = [_f32p, _f32p, _sz, _sz, _sz, _f32p, _f32p]
        L.mvo_swiglu.argtypes = [_f32p, _f32p, _f32p, _sz]
        L.mvo_argmax.argtypes = [_f32p, _sz]
        L.mvo_model_open.restype = C.c_void_p
        L.mvo_model_open.argtypes = [C.c_char_p, _sz, _sz, C.c_int, C.c_int, C.c_int]
        L.mvo_model_close.argtypes = [C.c_void_p]
        L.mvo_model_reset.argtypes = [C.c_void_p]
        L.mvo_model_config.argtypes = [C.c_void_p, _szp]
        L.mvo_model_forward.argtypes = [C.c_void_p, C.c_int, C.c_void_p]
        L.mvo_model_prefill.argtypes = [C.c_void_p, _i32p, _sz, _sz, C.c_void_p]
        L.mvo_model_position.restype = _sz
        L.mvo_model_position.argtypes = [C.c_void_p]
        L.mvo_model_kv_bytes.restype = _sz
        L.mvo_model_kv_bytes.argtypes = [C.c_void_p]
        self._bind_native()

    def _check(self, rc):
        if rc != 0:
            raise RuntimeError(self.lib.mvo_last_error().decode())

    # conversions
    def fp32_to_fp16(self, x):
        x = _f32(x).ravel()
        out = np.empty(x.size, np.uint16)
        self.lib.mvo_fp32_to_fp16_n(x, out, x.size)
        return out

    def fp32_to_fp16_bits(self, first, count):
        out = np.empty(count, np.uint16)
        self.lib.mvo_fp32_to_fp16_bits(first, count, out)
        return out

    def fp16_to_fp32(self, h):
        return np.array([self.lib.mvo_fp16_to_fp32(int(v)) for v in np.asarray(h).ravel()], np.float32)

    def quantize_q8(self, x):
        x = _f32(x)
        m = 1 if x.ndim == 1 else x.shape[0]
        k = x.shape[-1]
        q = np.empty(m * k, np.int8)
        d = np.empty(m * (k // 32), np.float32)
        self._check(self.lib.mvo_quantize_act_q8(x.ravel(), m, k, q, d))
        return q.reshape(x.shape), d.reshape(x.shape[:-1] + (k // 32,))

    def matvec(self, w, ty, rows, cols, x, threads=8):
        y = np.empty(rows, np.float32)
        self._check(self.lib.mvo_matvec(np.ascontiguousarray(w, np.uint8).ravel(), ty, rows, cols, _f32(x).ravel(),
                                        y, threads))
        return y

    def matmul_batch(self, w, ty, rows, cols, x, threads=8):
        x = _f32(x)
        m = x.shape[0]
        y = np.empty((m, rows), np.float32)
        self._check(self.lib.mvo_matmul_batch(np.ascontiguousarray(w, np.uint8).ravel(), ty, rows, cols, x.ravel(),
                                              y.ravel(), m, threads))
        return y

    def matmul_batch_v06(self, w, ty, rows, cols, x, is_ffn=False, force_q8=False, threads=8):
        x = _f32(x)
        m = x.shape[0]
        y = np.empty((m, rows), np.float32)
        self._check(self.lib.mvo_matmul_batch_v06(np.ascontiguousarray(w, np.uint8).ravel(), ty, rows, cols,
                                                  int(is_ffn), int(force_q8), x.ravel(), y.ravel(), m, threads))
        return y

    def read_row(self, w, ty, rows, cols, row):
        out = np.empty(cols, np.float32)
        self._check(self.lib.mvo_read_row_f32(np.ascontiguousarray(w, np.uint8).ravel(), ty, rows, cols, row, out))
        return out

    def rmsnorm(self, x, w, eps=1e-5):
        x = _f32(x)
        out = np.empty_like(x)
        self.lib.mvo_rmsnorm(x, _f32(w), x.size, eps, out)
        return out

    def rope_table(self, n_ctx, hd, theta=10000.0):
        co = np.empty(n_ctx * (hd // 2), np.float32)
        si = np.empty_like(co)
        self.lib.mvo_rope_table(n_ctx, hd, theta, co, si)
        return co.reshape(n_ctx, hd // 2), si.reshape(n_ctx, hd // 2)

    def rope(self, q, k, n_head, n_head_kv, hd, co_row, si_row):
        q = _f32(q).copy()
        k = _f32(k).copy()
        self.lib.mvo_rope(q, k, n_head, n_head_kv, hd, _f32(co_row), _f32(si_row))
        return q, k

    def swiglu(self, g, u):
        g = _f32(g)
        out = np.empty_like(g)
        self.lib.mvo_swiglu(g, _f32(u), out, g.size)
        return out

    def kv_parse_type(self, s):
        t = self.lib.mvo_kv_parse_type(s.encode())
        if t < 0:
            raise RuntimeError(self.lib.mvo_last_error().decode())
        return t

    def kv_type_name(self, t):
        return self.lib.mvo_kv_type_name(t).decode()

    def kv(self, kv_dim, page_tokens=128, kv_type=KV_F16):
        return OracleKV(self, kv_dim, page_tokens, kv_type)

    def model(self, path, ctx=0, page=128, threads=8, force_q8=False, kv_type=KV_F16):
        return OracleModel(self, path, ctx, page, threads, force_q8, kv_type)


class OracleKV:
    def __init__(self, o: Oracle, kv_dim, page_tokens, kv_type=KV_F16):
        self.o, self.kv_dim, self.kv_type = o, kv_dim, kv_type
        self.h = o.lib.mvo_kv_create(kv_dim, page_tokens, kv_type)
        if not self.h:
            raise RuntimeError(o.lib.mvo_last_error().decode())

    def __del__(self):
        if getattr(self, "h", None):
            self.o.lib.mvo_kv_destroy(self.h)
            self.h = None

    def write(self, pos, k, v):
        self.o.lib.mvo_kv_write(self.h, pos, _f32(k), _f32(v))

    def dot_key(self, pos, offset, q):
        q = _f32(q)
        return self.o.lib.mvo_kv_dot_key(self.h, pos, offset, q, q.size)

    def add_value(self, pos, offset, alpha, out):
        self.o.lib.mvo_kv_add_value(self.h, pos, offset, alpha, out, out.size)

    def row(self, pos, which):
        """(stored row as floats / fp16 bits / int8, Q8 scale or 1.0)"""
        sc = C.c_float()
        p = self.o.lib.mvo_kv_row(self.h, pos, which, C.byref(sc))
        if not p:
            raise RuntimeError("KV page missing")
        dt = np.dtype(KV_DTYPE[self.kv_type])
        raw = C.string_at(p, self.kv_dim * dt.itemsize)
        return np.frombuffer(raw, dt).copy(), np.float32(sc.value)

    def bytes_allocated(self):
        return self.o.lib.mvo_kv_bytes_allocated(self.h)

    def attn_decode(self, q, pos, n_head, n_head_kv, hd):
        out = np.empty(n_head * hd, np.float32)
        self.o.lib.mvo_attn_decode(self.h, _f32(q), pos, n_head, n_head_kv, hd, out)
        return out


class OracleModel:
    def __init__(self, o: Oracle, path, ctx, page, threads, force_q8, kv_type=KV_F16):
        self.o = o
        self.h = o.lib.mvo_model_open(path.encode(), ctx, page, kv_type, threads, int(force_q8))
        if not self.h:
            raise RuntimeError(o.lib.mvo_last_error().decode())
        cfg = np.zeros(7, np.uint64)
        o.lib.mvo_model_config(self.h, cfg)
        self.n_ctx, self.n_embd, self.n_ff, self.n_layer, self.n_head, self.n_head_kv, self.vocab = map(int, cfg)

    def close(self):
        if self.h:
            self.o.lib.mvo_model_close(self.h)
            self.h = None

    __del__ = close

    def reset(self):
        self.o.lib.mvo_model_reset(self.h)

    def forward(self, token, logits=True):
        out = np.empty(self.vocab, np.float32) if logits else None
        self.o._check(self.o.lib.mvo_model_forward(self.h, int(token), out.ctypes.data if logits else None))
        return out

    def prefill(self, tokens, batch=32, logits=True):
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.empty(self.vocab, np.float32) if logits else None
        self.o._check(self.o.lib.mvo_model_prefill(self.h, t, t.size, batch, out.ctypes.data if logits else None))
        return out

    @property
    def position(self):
        return self.o.lib.mvo_model_position(self.h)

    def kv_bytes(self):
        return self.o.lib.mvo_model_kv_bytes(self.h)


class Ref(_Native):
    """The compiled reference (public C++ API via ref_shim.cpp)."""

    _nq = "mvr_nq_"

    def __init__(self, path: str = REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = self.lib = C.CDLL(path)
        L.mvr_last_error.restype = C.c_char_p
        L.mvr_fp32_to_fp16_bits.argtypes = [C.c_uint32, C.c_uint64, _u16p]
        L.mvr_fp16_to_fp32.restype = C.c_float
        L.mvr_fp16_to_fp32.argtypes = [C.c_uint16]
        L.mvr_gguf_open.restype = C.c_void_p
        L.mvr_gguf_open.argtypes = [C.c_char_p]
        L.mvr_gguf_close.argtypes = [C.c_void_p]
        L.mvr_matvec.argtypes = [C.c_void_p, C.c_char_p, _f32p, _f32p, C.c_uint]
        L.mvr_matmul_batch.argtypes = [C.c_void_p, C.c_char_p, _f32p, _f32p, _sz, C.c_uint]
        L.mvr_matmul_batch_v06.argtypes = [C.c_void_p, C.c_char_p, _f32p, _f32p, _sz, C.c_uint, C.c_int]
        L.mvr_read_row.argtypes = [C.c_void_p, C.c_char_p, _sz, _f32p, _sz]
        L.mvr_kv_create.restype = C.c_void_p
        L.mvr_kv_create.argtypes = [_sz, _sz, C.c_int]
        L.mvr_kv_parse_type.argtypes = [C.c_char_p, C.POINTER(C.c_int)]
        L.mvr_kv_type_name.restype = C.c_char_p
        L.mvr_kv_type_name.argtypes = [C.c_int]
        L.mvr_kv_destroy.argtypes = [C.c_void_p]
        L.mvr_kv_write.argtypes = [C.c_void_p, _sz, _f32p, _f32p]
        L.mvr_kv_dot_key.argtypes = [C.c_void_p, _sz, _sz, _f32p, _sz, C.POINTER(C.c_float)]
        L.mvr_kv_add_value.argtypes = [C.c_void_p, _sz, _sz, C.c_float, _f32p, _sz]
        L.mvr_kv_bytes.restype = _sz
        L.mvr_kv_bytes.argtypes = [C.c_void_p]
        L.mvr_model_open.restype = C.c_void_p
        L.mvr_model_open.argtypes = [C.c_char_p, C.c_uint, _sz, _sz, C.c_int, C.c_int]
        L.mvr_model_close.argtypes = [C.c_void_p]
        L.mvr_model_reset.argtypes = [C.c_void_p]
        L.mvr_model_config.argtypes = [C.c_void_p, _szp]
        L.mvr_model_forward.argtypes = [C.c_void_p, C.c_int, C.c_void_p]
        L.mvr_model_prefill.argtypes = [C.c_void_p, _i32p, _sz, _sz, C.c_void_p]
        L.mvr_model_position.restype = _sz
        L.mvr_model_position.argtypes = [C.c_void_p]
        L.mvr_model_kv_bytes.restype = _sz
        L.mvr_model_kv_bytes.argtypes = [C.c_void_p]
        L.mvr_profile_enable.argtypes = [C.c_int]
        L.mvr_profile_kind_name.restype = C.c_char_p
        L.mvr_profile_kind_name.argtypes = [C.c_int]
        L.mvr_profile_snapshot.restype = _sz
        L.mvr_profile_snapshot.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, _sz, _sz]
        self._bind_native()

    def _check(self, rc):
        if rc != 0:
            raise RuntimeError(self.lib.mvr_last_error().decode())

    def fp32_to_fp16_bits(self, first, count):
        out = np.empty(count, np.uint16)
        self.lib.mvr_fp32_to_fp16_bits(first, count, out)
        return out

    def gguf(self, path):
        return RefGguf(self, path)

    def kv_parse_type(self, s):
        t = C.c_int()
        self._check(self.lib.mvr_kv_parse_type(s.encode(), C.byref(t)))
        return t.value

    def kv_type_name(self, t):
        return self.lib.mvr_kv_type_name(t).decode()

    def kv(self, kv_dim, page_tokens=128, kv_type=KV_F16):
        return RefKV(self, kv_dim, page_tokens, kv_type)

    def profile_enable(self, on=True):
        self.lib.mvr_profile_enable(int(on))

    def profile_reset(self):
        self.lib.mvr_profile_reset()

    def profile_kind_name(self, kind):
        return self.lib.mvr_profile_kind_name(kind).decode()

    def profile_snapshot(self):
        """[(layer, kind, tensor, calls, batch)] in the reference's snapshot order."""
        L = self.lib
        n = L.mvr_profile_snapshot(None, None, None, None, None, 0, 0)
        layer, kind = np.zeros(max(1, n), np.int32), np.zeros(max(1, n), np.int32)
        calls, batch = np.zeros(max(1, n), np.uint64), np.zeros(max(1, n), np.uint64)
        names = C.create_string_buffer(256 * max(1, n))
        L.mvr_profile_snapshot(layer.ctypes.data, kind.ctypes.data, calls.ctypes.data, batch.ctypes.data,
                               C.addressof(names), len(names), n)
        tensors = names.raw.split(b"\0")[:n]
        return [(int(layer[i]), int(kind[i]), tensors[i].decode(), int(calls[i]), int(batch[i])) for i in range(n)]

    def model(self, path, ctx=0, page=128, threads=8, force_q8=False, kv_type=KV_F16):
        return RefModel(self, path, ctx, page, threads, force_q8, kv_type)


class RefGguf:
    def __init__(self, r: Ref, path):
        self.r = r
        self.h = r.lib.mvr_gguf_open(path.encode())
        if not self.h:
            raise RuntimeError(r.lib.mvr_last_error().decode())

    def __del__(self):
        if getattr(self, "h", None):
            self.r.lib.mvr_gguf_close(self.h)
            self.h = None

    def matvec(self, name, x, rows, threads=8):
        y = np.empty(rows, np.float32)
        self.r._check(self.r.lib.mvr_matvec(self.h, name.encode(), _f32(x).ravel(), y, threads))
        return y

    def matmul_batch(self, name, x, rows, threads=8):
        x = _f32(x)
        y = np.empty((x.shape[0], rows), np.float32)
        self.r._check(self.r.lib.mvr_matmul_batch(self.h, name.encode(), x.ravel(), y.ravel(), x.shape[0], threads))
        return y

    def matmul_batch_v06(self, name, x, rows, force_q8=False, threads=8):
        x = _f32(x)
        y = np.empty((x.shape[0], rows), np.float32)
        self.r._check(self.r.lib.mvr_matmul_batch_v06(self.h, name.encode(), x.ravel(), y.ravel(), x.shape[0],
                                                      threads, int(force_q8)))
        return y

    def read_row(self, name, row, cols):
        out = np.empty(cols, np.float32)
        self.r._check(self.r.lib.mvr_read_row(self.h, name.encode(), row, out, cols))
        return out


class RefKV:
    def __init__(self, r: Ref, kv_dim, page_tokens, kv_type=KV_F16):
        self.r = r
        self.h = r.lib.mvr_kv_create(kv_dim, page_tokens, kv_type)

    def __del__(self):
        if getattr(self, "h", None):
            self.r.lib.mvr_kv_destroy(self.h)
            self.h = None

    def write(self, pos, k, v):
        self.r._check(self.r.lib.mvr_kv_write(self.h, pos, _f32(k), _f32(v)))

    def dot_key(self, pos, offset, q):
        q = _f32(q)
        out = C.c_float()
        self.r._check(self.r.lib.mvr_kv_dot_key(self.h, pos, offset, q, q.size, C.byref(out)))
        return out.value

    def add_value(self, pos, offset, alpha, out):
        self.r._check(self.r.lib.mvr_kv_add_value(self.h, pos, offset, alpha, out, out.size))

    def bytes_allocated(self):
        return self.r.lib.mvr_kv_bytes(self.h)


class RefModel:
    def __init__(self, r: Ref, path, ctx, page, threads, force_q8, kv_type=KV_F16):
        self.r = r
        self.h = r.lib.mvr_model_open(path.encode(), threads, ctx, page, kv_type, int(force_q8))
        if not self.h:
            raise RuntimeError(r.lib.mvr_last_error().decode())
        cfg = np.zeros(7, np.uint64)
        r.lib.mvr_model_config(self.h, cfg)
        self.n_ctx, self.n_embd, self.n_ff, self.n_layer, self.n_head, self.n_head_kv, self.vocab = map(int, cfg)

    def close(self):
        if self.h:
            self.r.lib.mvr_model_close(self.h)
            self.h = None

    __del__ = close

    def reset(self):
        self.r.lib.mvr_model_reset(self.h)

    def forward(self, token, logits=True):
        out = np.empty(self.vocab, np.float32) if logits else None
        self.r._check(self.r.lib.mvr_model_forward(self.h, int(token), out.ctypes.data if logits else None))
        return out

    def prefill(self, tokens, batch=32, logits=True):
        t = np.ascontiguousarray(tokens, np.int32)
        out = np.empty(self.vocab, np.float32) if logits else None
        self.r._check(self.r.lib.mvr_model_prefill(self.h, t, t.size, batch, out.ctypes.data if logits else None))
        return out

    @property
    def position(self):
        return self.r.lib.mvr_model_position(self.h)

    def kv_bytes(self):
        return self.r.lib.mvr_model_kv_bytes(self.h)


def ref_available() -> bool:
    return os.path.exists(REF_SO)
