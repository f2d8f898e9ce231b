"""ctypes front end of libtmac_attn.so (the C ABI in include/tmac_attn.h).

Mirrors the reference's per-layer dispatch surface (metal_backend.hpp:354-453):
``attention_op``, ``rope_op``, ``elem_op`` plus the fused layer step, batched and
ragged decode, and step capture into a hipGraph.  Device memory is handled by
the library itself (``Context.upload`` / ``DeviceArray``), so no framework is
needed to drive it.

There is no CPU fallback: if the library is not built this module raises on
import of the library, and every op runs on the GPU through the C ABI.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# TMAC_ATTN_LIB selects another build of the same library (the host sanitizer
# build, lib/libtmac_attn_san.so, in tests/test_sanitize.py).
LIB_PATH = os.environ.get("TMAC_ATTN_LIB") or os.path.join(HERE, "lib", "libtmac_attn.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "tmac_attn.h")

TMAC_OK = 0
TMAC_ERR_INVALID_ARG = 1
TMAC_ERR_NULL_POINTER = 2
TMAC_ERR_MISALIGNED = 3
TMAC_ERR_UNSUPPORTED = 4
TMAC_ERR_CAPACITY = 5
TMAC_ERR_NOT_INITIALIZED = 6
TMAC_ERR_CAPTURE = 7
TMAC_ERR_DEVICE_FAULT = 8
TMAC_ERR_NOT_FOUND = 9
TMAC_ERR_IO = 10
TMAC_ERR_HIP_BASE = 1000

TMAC_Q5_0 = 6
TMAC_Q8_0 = 8
TMAC_Q4_K = 12
TMAC_Q6_K = 14
TMAC_KV_F32 = 0
TMAC_KV_BF16 = 1
TMAC_KV_F16 = 2
TMAC_KV_Q8_0 = 3
PAGE_ROWS = 16           # rows per page of a paged cache
Q8_HEAD_BYTES = 68       # Q8_0 cache: bytes per (row, kv head): int8 q[64], fp16 d0, d1
TMAC_OPT_SPLIT_LEN = 1
TMAC_OPT_TARGET_GROUPS = 2
TMAC_OPT_KERNEL = 3
TMAC_OPT_ROTATE = 4
TMAC_OPT_HEAD_WAVES = 5
TMAC_OPT_WAVE_ORDER = 6
TMAC_OPT_GROUP_WAVES = 7
TMAC_OPT_MFMA_DECODE = 8
TMAC_OPT_STREAM_K = 9
TMAC_OPT_HV_SPLIT = 10
TMAC_KERNEL_AUTO = 0
TMAC_KERNEL_GROUP = 1
TMAC_KERNEL_HEAD = 2
TMAC_KERNEL_HEADV = 3

_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t
_i64 = ctypes.c_int64

# name -> (restype, argtypes); every entry point of include/tmac_attn.h
SIGNATURES = {
    "tmac_status_string": (ctypes.c_char_p, [_i]),
    "tmac_last_error": (ctypes.c_char_p, [_vp]),
    "tmac_abi_version": (_i, []),
    "tmac_init": (_i, [ctypes.POINTER(_vp), _i]),
    "tmac_shutdown": (_i, [_vp]),
    "tmac_attention_op": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i]),
    "tmac_rope_op": (_i, [_vp, _vp, _vp, _i, _i, _i, _f]),
    "tmac_elem_op": (_i, [_vp, _vp, _i, _vp, _vp, _i]),
    "tmac_fused_qkv_op": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i]),
    "tmac_fused_qkv_bias": (_i, [_vp] * 12 + [_i] * 5),
    "tmac_attention_decode_batched_kv": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i64]),
    "tmac_attention_decode_ragged_kv": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                             _i64]),
    "tmac_layer_attention_kv": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f]),
    "tmac_layer_attention_devpos_kv": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp, _i,
                                            _f]),
    "tmac_kv_convert": (_i, [_vp, _vp, _i, _vp, _vp, _i64]),
    "tmac_attention_decode_paged": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _i, _vp, _i, _vp, _vp, _i, _i, _i, _i, _i,
                                         _i64]),
    "tmac_layer_attention_paged": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _i, _vp, _i, _vp, _vp, _i, _i, _i,
                                        _i, _i, _f]),
    "tmac_matmul_q8_0": (_i, [_vp, _vp, _i, _i, _vp, _vp, _vp]),
    "tmac_matmul_q5_0": (_i, [_vp, _vp, _i, _i, _vp, _vp, _vp]),
    "tmac_matmul_add": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp]),
    "tmac_matmul_q4_k": (_i, [_vp, _vp, _i, _i, _vp, _vp, _vp]),
    "tmac_matmul_q6_k": (_i, [_vp, _vp, _i, _i, _vp, _vp, _vp]),
    "tmac_layer_attention": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f]),
    "tmac_layer_attention_devpos": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp, _i, _f]),
    "tmac_pos_update": (_i, [_vp, _vp, _vp, _i, _i]),
    "tmac_rope_prepare": (_i, [_vp, _i, _f, _i]),
    "tmac_attention_decode_batched": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i64]),
    "tmac_attention_decode_ragged": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i64]),
    "tmac_attention_decode_ragged_noalloc": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                                  _i64]),
    "tmac_attention_prefill": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i64, _i, _i, _i]),
    "tmac_attention_prefill_kv": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _vp, _i, _i, _i, _i64, _i, _i, _i]),
    "tmac_attention_prefill_paged": (_i, [_vp, _vp, _i, _vp, _vp, _vp, _i, _vp, _i, _vp, _i, _i, _i, _i, _i, _i]),
    "tmac_prefill_tiles_bytes": (_sz, [_i, _i, _i]),
    "tmac_prefill_pack_rows": (_i, [_vp, _vp, _i, _vp, _vp, _i64, _vp, _i, _i, _i, _i, _i, _i]),
    "tmac_attention_prefill_tiles": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _i, _i, _i, _i, _i, _i]),
    "tmac_rope_rows": (_i, [_vp, _vp, _vp, _i, _i64, _i, _i, _i, _f]),
    "tmac_set_option": (_i, [_vp, _i, _i64]),
    "tmac_query_split": (_i, [_vp, _i, _i, _i, _i, ctypes.POINTER(_i), ctypes.POINTER(_i)]),
    "tmac_check_device_error": (_i, [_vp]),
    "tmac_synth_normal": (_i, [ctypes.c_uint64, _vp, _sz]),
    "tmac_synth_uniform": (_i, [ctypes.c_uint64, _vp, _sz]),
    "tmac_step_begin": (_i, [_vp, _vp]),
    "tmac_step_end": (_i, [_vp, _vp, ctypes.POINTER(_vp)]),
    "tmac_graph_launch": (_i, [_vp, _vp, _vp]),
    "tmac_graph_destroy": (_i, [_vp, _vp]),
    "tmac_malloc": (_i, [_vp, ctypes.POINTER(_vp), _sz]),
    "tmac_free": (_i, [_vp, _vp]),
    "tmac_memcpy_h2d": (_i, [_vp, _vp, _vp, _vp, _sz]),
    "tmac_memcpy_d2h": (_i, [_vp, _vp, _vp, _vp, _sz]),
    "tmac_memcpy_d2d": (_i, [_vp, _vp, _vp, _vp, _sz]),
    "tmac_memset": (_i, [_vp, _vp, _vp, _i, _sz]),
    "tmac_stream_create": (_i, [_vp, ctypes.POINTER(_vp)]),
    "tmac_stream_destroy": (_i, [_vp, _vp]),
    "tmac_stream_synchronize": (_i, [_vp, _vp]),
    "tmac_device_synchronize": (_i, [_vp]),
    "tmac_event_create": (_i, [_vp, ctypes.POINTER(_vp)]),
    "tmac_event_destroy": (_i, [_vp, _vp]),
    "tmac_event_record": (_i, [_vp, _vp, _vp]),
    "tmac_event_elapsed_ms": (_i, [_vp, _vp, _vp, ctypes.POINTER(_f)]),
    "tmac_device_info": (_i, [_vp, ctypes.c_char_p, _sz, ctypes.POINTER(_i)]),
    "tmac_model_load": (_i, [_vp, ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "tmac_model_count": (_i, [_vp]),
    "tmac_model_tensor": (_i, [_vp, _i, _vp]),
    "tmac_model_find": (_i, [_vp, ctypes.c_char_p, _vp]),
    "tmac_model_free": (_i, [_vp, _vp]),
}


class TensorInfo(ctypes.Structure):
    """tmac_tensor_info."""
    _fields_ = [("name", ctypes.c_char_p), ("rows", ctypes.c_uint64), ("cols", ctypes.c_uint64),
                ("type", ctypes.c_uint32), ("n_bytes", ctypes.c_uint64), ("data", ctypes.c_void_p)]


class Model:
    """A loaded TMAC weight file (tmac_model_load).  `ctx=None` keeps the
    tensors in host memory; with a Context they live on the device."""

    def __init__(self, path: str, ctx: Optional["Context"] = None):
        self.lib = load_library()
        self.ctx = ctx
        h = _vp()
        rc = self.lib.tmac_model_load(ctx.handle if ctx else None, os.fsencode(path), ctypes.byref(h))
        if rc != TMAC_OK:
            detail = self.lib.tmac_last_error(ctx.handle).decode() if ctx else path
            raise TmacError(rc, "model_load", detail)
        self.handle = h.value

    def __len__(self) -> int:
        return self.lib.tmac_model_count(self.handle)

    def _info(self, rc: int, info: TensorInfo, what: str) -> dict:
        if rc != TMAC_OK:
            raise TmacError(rc, what)
        return {"name": info.name.decode(), "rows": info.rows, "cols": info.cols, "type": info.type,
                "n_bytes": info.n_bytes, "data": info.data}

    def tensor(self, index: int) -> dict:
        info = TensorInfo()
        return self._info(self.lib.tmac_model_tensor(self.handle, index, ctypes.byref(info)), info, "model_tensor")

    def find(self, name: str) -> Optional[dict]:
        info = TensorInfo()
        rc = self.lib.tmac_model_find(self.handle, name.encode(), ctypes.byref(info))
        if rc == TMAC_ERR_NOT_FOUND:
            return None
        return self._info(rc, info, "model_find")

    def free(self) -> None:
        if self.handle:
            rc = self.lib.tmac_model_free(self.ctx.handle if self.ctx else None, self.handle)
            if rc != TMAC_OK:
                raise TmacError(rc, "model_free")
            self.handle = None

_lib: Optional[ctypes.CDLL] = None


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Loads the in-tree library; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is missing: build it with __graft_entry__.build() (there is no CPU fallback)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


class TmacError(RuntimeError):
    def __init__(self, status: int, what: str, detail: str = ""):
        self.status = status
        lib = load_library()
        msg = lib.tmac_status_string(status).decode()
        super().__init__(f"{what}: status {status} ({msg}) {detail}".strip())


def status_string(status: int) -> str:
    return load_library().tmac_status_string(status).decode()


def synth_normal(seed: int, shape, out: Optional[np.ndarray] = None) -> np.ndarray:
    """N(0,1) fp32 values of stream `seed` (tmac_synth_normal; host only, no GPU)."""
    if out is None:
        out = np.empty(shape, np.float32)
    assert out.dtype == np.float32 and out.flags["C_CONTIGUOUS"]
    rc = load_library().tmac_synth_normal(ctypes.c_uint64(seed), out.ctypes.data, out.size)
    if rc:
        raise TmacError(rc, "synth_normal")
    return out


def synth_uniform(seed: int, n: int) -> np.ndarray:
    """Uniforms in [0, 1) of stream `seed` (tmac_synth_uniform)."""
    out = np.empty(n, np.float64)
    rc = load_library().tmac_synth_uniform(ctypes.c_uint64(seed), out.ctypes.data, n)
    if rc:
        raise TmacError(rc, "synth_uniform")
    return out


class DeviceArray:
    """A device allocation with a numpy-like shape/dtype."""

    def __init__(self, ctx: "Context", shape, dtype=np.float32):
        self.ctx = ctx
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = _vp()
        ctx._check(ctx.lib.tmac_malloc(ctx.handle, ctypes.byref(p), self.nbytes), "tmac_malloc")
        self.ptr = p.value

    @property
    def size(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64))

    def at(self, elem_offset: int) -> int:
        """Device address of element `elem_offset` (flat)."""
        return self.ptr + int(elem_offset) * self.dtype.itemsize

    def copy_from(self, host: np.ndarray, stream=None) -> None:
        host = np.ascontiguousarray(host, dtype=self.dtype)
        assert host.nbytes == self.nbytes, (host.nbytes, self.nbytes)
        self.ctx._check(self.ctx.lib.tmac_memcpy_h2d(self.ctx.handle, stream, self.ptr,
                                                     host.ctypes.data, host.nbytes), "memcpy_h2d")
        self.ctx.synchronize(stream)

    def numpy(self, stream=None) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        self.ctx.synchronize(stream)
        self.ctx._check(self.ctx.lib.tmac_memcpy_d2h(self.ctx.handle, stream, out.ctypes.data,
                                                     self.ptr, self.nbytes), "memcpy_d2h")
        self.ctx.synchronize(stream)
        return out

    def fill_bytes(self, value: int, stream=None) -> None:
        self.ctx._check(self.ctx.lib.tmac_memset(self.ctx.handle, stream, self.ptr, value, self.nbytes),
                        "memset")

    def free(self) -> None:
        if self.ptr:
            self.ctx.lib.tmac_free(self.ctx.handle, self.ptr)
            self.ptr = 0


def _p(x) -> Optional[int]:
    if x is None:
        return None
    if isinstance(x, DeviceArray):
        return x.ptr
    return int(x)


class Context:
    """One tmac_context on one device (the analogue of metal_backend::Context)."""

    def __init__(self, device: int = 0):
        self.lib = load_library()
        h = _vp()
        rc = self.lib.tmac_init(ctypes.byref(h), device)
        if rc != TMAC_OK:
            raise TmacError(rc, "tmac_init")
        self.handle = h.value
        self.device = device

    # -- plumbing --------------------------------------------------------------
    def _check(self, rc: int, what: str) -> None:
        if rc != TMAC_OK:
            raise TmacError(rc, what, self.lib.tmac_last_error(self.handle).decode())

    def close(self) -> None:
        if self.handle:
            self.lib.tmac_shutdown(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def empty(self, shape, dtype=np.float32) -> DeviceArray:
        return DeviceArray(self, shape, dtype)

    def upload(self, host: np.ndarray, dtype=None) -> DeviceArray:
        host = np.ascontiguousarray(host, dtype=dtype or host.dtype)
        d = DeviceArray(self, host.shape, host.dtype)
        d.copy_from(host)
        return d

    def synchronize(self, stream=None) -> None:
        if stream is None:
            self._check(self.lib.tmac_device_synchronize(self.handle), "device_synchronize")
        else:
            self._check(self.lib.tmac_stream_synchronize(self.handle, stream), "stream_synchronize")

    def stream(self) -> int:
        s = _vp()
        self._check(self.lib.tmac_stream_create(self.handle, ctypes.byref(s)), "stream_create")
        return s.value

    def destroy_stream(self, s) -> None:
        self._check(self.lib.tmac_stream_destroy(self.handle, s), "stream_destroy")

    def event(self) -> int:
        e = _vp()
        self._check(self.lib.tmac_event_create(self.handle, ctypes.byref(e)), "event_create")
        return e.value

    def record(self, ev, stream=None) -> None:
        self._check(self.lib.tmac_event_record(self.handle, ev, stream), "event_record")

    def elapsed_ms(self, start, stop) -> float:
        ms = _f()
        self._check(self.lib.tmac_event_elapsed_ms(self.handle, start, stop, ctypes.byref(ms)), "elapsed")
        return float(ms.value)

    def destroy_event(self, ev) -> None:
        self._check(self.lib.tmac_event_destroy(self.handle, ev), "event_destroy")

    def device_info(self) -> tuple[str, int]:
        buf = ctypes.create_string_buffer(512)
        n = _i()
        self._check(self.lib.tmac_device_info(self.handle, buf, 512, ctypes.byref(n)), "device_info")
        return buf.value.decode(), n.value

    def set_option(self, option: int, value: int) -> None:
        self._check(self.lib.tmac_set_option(self.handle, option, value), "set_option")

    def query_split(self, n_seq: int, n_pos: int, n_head: int, n_kv_head: int) -> tuple[int, int]:
        a, b = _i(), _i()
        self._check(self.lib.tmac_query_split(self.handle, n_seq, n_pos, n_head, n_kv_head,
                                              ctypes.byref(a), ctypes.byref(b)), "query_split")
        return a.value, b.value

    def check_device_error(self) -> int:
        return self.lib.tmac_check_device_error(self.handle)

    # -- the reference's dispatch surface --------------------------------------
    def attention_op(self, q, k_cache, v_cache, out, n_head, n_kv_head, head_dim, past_len,
                     stream=None, check=True) -> int:
        rc = self.lib.tmac_attention_op(self.handle, stream, _p(q), _p(k_cache), _p(v_cache), _p(out),
                                        n_head, n_kv_head, head_dim, past_len)
        if check:
            self._check(rc, "attention_op")
        return rc

    def rope_rows(self, data, n_rows, row_stride, n_heads, head_dim, first_pos, base=1e6, stream=None,
                  check=True) -> int:
        rc = self.lib.tmac_rope_rows(self.handle, stream, _p(data), n_rows, row_stride, n_heads, head_dim, first_pos,
                                     base)
        if check:
            self._check(rc, "rope_rows")
        return rc

    def rope_op(self, data, n_heads, head_dim, pos, base=1e6, stream=None, check=True) -> int:
        rc = self.lib.tmac_rope_op(self.handle, stream, _p(data), n_heads, head_dim, pos, base)
        if check:
            self._check(rc, "rope_op")
        return rc

    def elem_op(self, op, data, aux, dim, stream=None, check=True) -> int:
        rc = self.lib.tmac_elem_op(self.handle, stream, op, _p(data), _p(aux), dim)
        if check:
            self._check(rc, "elem_op")
        return rc

    def fused_qkv(self, w_q, w_k, w_v, x, y_q, y_k, y_v, q_rows, k_rows, v_rows, cols, v_is_q8,
                  b_q=None, b_k=None, b_v=None, stream=None, check=True, with_bias=None) -> int:
        """tmac_fused_qkv_bias when any bias is given (or with_bias is True), else
        tmac_fused_qkv_op."""
        if with_bias is None:
            with_bias = any(b is not None for b in (b_q, b_k, b_v))
        if with_bias:
            rc = self.lib.tmac_fused_qkv_bias(self.handle, stream, _p(w_q), _p(w_k), _p(w_v), _p(x), _p(b_q),
                                              _p(b_k), _p(b_v), _p(y_q), _p(y_k), _p(y_v), q_rows, k_rows,
                                              v_rows, cols, int(v_is_q8))
        else:
            rc = self.lib.tmac_fused_qkv_op(self.handle, stream, _p(w_q), _p(w_k), _p(w_v), _p(x), _p(y_q),
                                            _p(y_k), _p(y_v), q_rows, k_rows, v_rows, cols, int(v_is_q8))
        if check:
            self._check(rc, "fused_qkv")
        return rc

    def matmul(self, qtype, rows, cols, w, x, y, accumulate=False, stream=None, check=True) -> int:
        """tmac_matmul_q5_0 / _q8_0 (y = W x), or tmac_matmul_add (y += W x)."""
        if accumulate:
            rc = self.lib.tmac_matmul_add(self.handle, stream, qtype, rows, cols, _p(w), _p(x), _p(y))
        elif qtype == TMAC_Q8_0:
            rc = self.lib.tmac_matmul_q8_0(self.handle, stream, rows, cols, _p(w), _p(x), _p(y))
        elif qtype == TMAC_Q4_K:
            rc = self.lib.tmac_matmul_q4_k(self.handle, stream, rows, cols, _p(w), _p(x), _p(y))
        elif qtype == TMAC_Q6_K:
            rc = self.lib.tmac_matmul_q6_k(self.handle, stream, rows, cols, _p(w), _p(x), _p(y))
        else:
            rc = self.lib.tmac_matmul_q5_0(self.handle, stream, rows, cols, _p(w), _p(x), _p(y))
        if check:
            self._check(rc, "matmul")
        return rc

    def layer_attention(self, q, k_new, v_new, k_cache, v_cache, out, n_head, n_kv_head, head_dim,
                        pos, capacity, base=1e6, stream=None, check=True, kv_dtype=TMAC_KV_F32) -> int:
        if kv_dtype == TMAC_KV_F32:
            rc = self.lib.tmac_layer_attention(self.handle, stream, _p(q), _p(k_new), _p(v_new),
                                               _p(k_cache), _p(v_cache), _p(out), n_head, n_kv_head,
                                               head_dim, pos, capacity, base)
        else:
            rc = self.lib.tmac_layer_attention_kv(self.handle, stream, kv_dtype, _p(q), _p(k_new), _p(v_new),
                                                  _p(k_cache), _p(v_cache), _p(out), n_head, n_kv_head,
                                                  head_dim, pos, capacity, base)
        if check:
            self._check(rc, "layer_attention")
        return rc

    def layer_attention_devpos(self, q, k_new, v_new, k_cache, v_cache, out, n_head, n_kv_head,
                               head_dim, pos_dev, capacity, base=1e6, stream=None, check=True,
                               kv_dtype=TMAC_KV_F32) -> int:
        if kv_dtype == TMAC_KV_F32:
            rc = self.lib.tmac_layer_attention_devpos(self.handle, stream, _p(q), _p(k_new), _p(v_new),
                                                      _p(k_cache), _p(v_cache), _p(out), n_head,
                                                      n_kv_head, head_dim, _p(pos_dev), capacity, base)
        else:
            rc = self.lib.tmac_layer_attention_devpos_kv(self.handle, stream, kv_dtype, _p(q), _p(k_new),
                                                         _p(v_new), _p(k_cache), _p(v_cache), _p(out), n_head,
                                                         n_kv_head, head_dim, _p(pos_dev), capacity, base)
        if check:
            self._check(rc, "layer_attention_devpos")
        return rc

    def pos_update(self, pos_dev, value, add=False, stream=None) -> None:
        self._check(self.lib.tmac_pos_update(self.handle, stream, _p(pos_dev), value, 1 if add else 0),
                    "pos_update")

    def rope_prepare(self, head_dim, base, n_pos) -> None:
        self._check(self.lib.tmac_rope_prepare(self.handle, head_dim, base, n_pos), "rope_prepare")

    def decode_batched(self, q, k, v, out, n_seq, n_head, n_kv_head, head_dim, n_pos, seq_stride,
                       stream=None, check=True, kv_dtype=TMAC_KV_F32) -> int:
        if kv_dtype == TMAC_KV_F32:
            rc = self.lib.tmac_attention_decode_batched(self.handle, stream, _p(q), _p(k), _p(v), _p(out),
                                                        n_seq, n_head, n_kv_head, head_dim, n_pos, seq_stride)
        else:
            rc = self.lib.tmac_attention_decode_batched_kv(self.handle, stream, kv_dtype, _p(q), _p(k), _p(v),
                                                           _p(out), n_seq, n_head, n_kv_head, head_dim, n_pos,
                                                           seq_stride)
        if check:
            self._check(rc, "decode_batched")
        return rc

    def decode_ragged(self, q, k_pool, v_pool, offsets, lengths, out, n_seq, n_head, n_kv_head,
                      head_dim, max_len, total_rows=0, stream=None, check=True, kv_dtype=TMAC_KV_F32) -> int:
        if kv_dtype == TMAC_KV_F32:
            rc = self.lib.tmac_attention_decode_ragged(self.handle, stream, _p(q), _p(k_pool), _p(v_pool),
                                                       _p(offsets), _p(lengths), _p(out), n_seq, n_head,
                                                       n_kv_head, head_dim, max_len, total_rows)
        else:
            rc = self.lib.tmac_attention_decode_ragged_kv(self.handle, stream, kv_dtype, _p(q), _p(k_pool),
                                                          _p(v_pool), _p(offsets), _p(lengths), _p(out), n_seq,
                                                          n_head, n_kv_head, head_dim, max_len, total_rows)
        if check:
            self._check(rc, "decode_ragged")
        return rc

    def kv_convert(self, kv_dtype, src, dst, n, stream=None, check=True) -> int:
        rc = self.lib.tmac_kv_convert(self.handle, stream, kv_dtype, _p(src), _p(dst), n)
        if check:
            self._check(rc, "kv_convert")
        return rc

    def decode_paged(self, q, k_pages, v_pages, n_pages, block_table, max_pages, lengths, out, n_seq, n_head,
                     n_kv_head, head_dim, max_len, total_rows=0, stream=None, check=True,
                     kv_dtype=TMAC_KV_F32) -> int:
        rc = self.lib.tmac_attention_decode_paged(self.handle, stream, kv_dtype, _p(q), _p(k_pages), _p(v_pages),
                                                  n_pages, _p(block_table), max_pages, _p(lengths), _p(out),
                                                  n_seq, n_head, n_kv_head, head_dim, max_len, total_rows)
        if check:
            self._check(rc, "decode_paged")
        return rc

    def layer_attention_paged(self, q, k_new, v_new, k_pages, v_pages, n_pages, block_table, max_pages,
                              positions, out, n_seq, n_head, n_kv_head, head_dim, max_len, base=1e6, stream=None,
                              check=True, kv_dtype=TMAC_KV_F32) -> int:
        rc = self.lib.tmac_layer_attention_paged(self.handle, stream, kv_dtype, _p(q), _p(k_new), _p(v_new),
                                                 _p(k_pages), _p(v_pages), n_pages, _p(block_table), max_pages,
                                                 _p(positions), _p(out), n_seq, n_head, n_kv_head, head_dim,
                                                 max_len, base)
        if check:
            self._check(rc, "layer_attention_paged")
        return rc

    def prefill(self, q, k, v, out, n_seq, n_q, prefix_len, seq_stride, n_head, n_kv_head, head_dim,
                stream=None, check=True, kv_dtype=TMAC_KV_F32) -> int:
        if kv_dtype == TMAC_KV_F32:
            rc = self.lib.tmac_attention_prefill(self.handle, stream, _p(q), _p(k), _p(v), _p(out), n_seq, n_q,
                                                 prefix_len, seq_stride, n_head, n_kv_head, head_dim)
        else:
            rc = self.lib.tmac_attention_prefill_kv(self.handle, stream, kv_dtype, _p(q), _p(k), _p(v), _p(out),
                                                    n_seq, n_q, prefix_len, seq_stride, n_head, n_kv_head, head_dim)
        if check:
            self._check(rc, "prefill")
        return rc

    def prefill_tiles_bytes(self, n_seq, n_kv_head, capacity) -> int:
        return int(self.lib.tmac_prefill_tiles_bytes(n_seq, n_kv_head, capacity))

    def prefill_pack_rows(self, k, v, seq_stride, tiles, capacity, n_seq, n_kv_head, head_dim, row_begin, row_end,
                          stream=None, check=True, kv_dtype=TMAC_KV_F32) -> int:
        rc = self.lib.tmac_prefill_pack_rows(self.handle, stream, kv_dtype, _p(k), _p(v), seq_stride, _p(tiles),
                                             capacity, n_seq, n_kv_head, head_dim, row_begin, row_end)
        if check:
            self._check(rc, "prefill_pack_rows")
        return rc

    def prefill_tiles(self, q, tiles, capacity, out, n_seq, n_q, prefix_len, n_head, n_kv_head, head_dim,
                      stream=None, check=True) -> int:
        rc = self.lib.tmac_attention_prefill_tiles(self.handle, stream, _p(q), _p(tiles), capacity, _p(out), n_seq,
                                                   n_q, prefix_len, n_head, n_kv_head, head_dim)
        if check:
            self._check(rc, "prefill_tiles")
        return rc

    def prefill_paged(self, q, k_pages, v_pages, n_pages, block_table, max_pages, out, n_seq, n_q, prefix_len,
                      n_head, n_kv_head, head_dim, stream=None, check=True, kv_dtype=TMAC_KV_F32) -> int:
        rc = self.lib.tmac_attention_prefill_paged(self.handle, stream, kv_dtype, _p(q), _p(k_pages), _p(v_pages),
                                                   n_pages, _p(block_table), max_pages, _p(out), n_seq, n_q,
                                                   prefix_len, n_head, n_kv_head, head_dim)
        if check:
            self._check(rc, "prefill_paged")
        return rc

    # -- step capture ----------------------------------------------------------
    def step_begin(self, stream) -> None:
        self._check(self.lib.tmac_step_begin(self.handle, stream), "step_begin")

    def step_end(self, stream, graph: Optional[int] = None) -> int:
        g = _vp(graph)
        self._check(self.lib.tmac_step_end(self.handle, stream, ctypes.byref(g)), "step_end")
        return g.value

    def graph_launch(self, graph, stream) -> None:
        self._check(self.lib.tmac_graph_launch(self.handle, graph, stream), "graph_launch")

    def graph_destroy(self, graph) -> None:
        self._check(self.lib.tmac_graph_destroy(self.handle, graph), "graph_destroy")


def declared_symbols(header: str = HEADER) -> list[str]:
    """Function names declared in include/tmac_attn.h."""
    import re
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tmac_[a-z0-9_]+)\s*\(", text)))
