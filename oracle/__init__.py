"""CPU oracle for the attention hot path -- TEST INFRASTRUCTURE ONLY.

numpy/ctypes front end of ``oracle/tmac_oracle.c``, the C restatement of the
reference's CPU path (liuwantao3/tmac_gguf.cpp):

* ``rope``            -- tmac_gguf.cpp:990-1016 (apply_rope)
* ``cache_write``     -- tmac_gguf.cpp:1090-1091
* ``attention``       -- tmac_gguf.cpp:1093-1128
* ``layer_step``      -- tmac_gguf.cpp:1085-1128 (rope -> cache write -> attention)
* ``attention_ragged``/``prefill`` -- the same per-head loop over many sequences

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
may import this module.  It is the checker, never the thing measured or shipped:
the product (``libtmac_attn.so``) has no CPU fallback and never loads it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "lib")
PARITY_LIB = os.environ.get("TMAC_ORACLE_LIB") or os.path.join(LIB_DIR, "libtmac_oracle.so")  # the sanitizer build in tests/test_sanitize.py
TIMING_LIB = os.path.join(LIB_DIR, "libtmac_oracle_o3.so")

# Compiler flags of the two builds (oracle/Makefile; a CPU test keeps the two in step).
BUILD_FLAGS = {
    "parity": "gcc -std=c11 -O2 -ffp-contract=off -fno-fast-math -fno-builtin -fopenmp -fPIC",
    "timing": "gcc -std=c11 -O3 -fopenmp -fPIC",
}

_F = ctypes.POINTER(ctypes.c_float)
_I64 = ctypes.POINTER(ctypes.c_int64)
_I32 = ctypes.POINTER(ctypes.c_int32)
_libs: dict[str, ctypes.CDLL] = {}


def build(force: bool = False) -> None:
    """Compile the oracle with its Makefile (gcc; runs anywhere)."""
    args = ["make", "-s", "-C", HERE]
    if force:
        args.insert(1, "-B")
    subprocess.run(args, check=True)


def _load(path: str) -> ctypes.CDLL:
    if path in _libs:
        return _libs[path]
    if not os.path.exists(path):
        build()
    lib = ctypes.CDLL(path)
    lib.tmac_fill_normal.argtypes = [ctypes.c_uint64, _F, ctypes.c_size_t]
    lib.tmac_fill_normal.restype = None
    lib.tmac_splitmix64.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
    lib.tmac_splitmix64.restype = ctypes.c_uint64
    lib.tmac_rng_set_state.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint64)]
    lib.tmac_rng_set_state.restype = None
    lib.tmac_rng_next.argtypes = [ctypes.c_void_p]
    lib.tmac_rng_next.restype = ctypes.c_uint64
    lib.oracle_rope_heads.argtypes = [_F, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float]
    lib.oracle_rope_heads.restype = None
    lib.oracle_rope_theta.argtypes = [_F, ctypes.c_int, ctypes.c_float]
    lib.oracle_rope_theta.restype = None
    lib.oracle_cache_write.argtypes = [_F, _F, ctypes.c_int]
    lib.oracle_cache_write.restype = None
    lib.oracle_attention.argtypes = [_F, _F, _F, _F] + [ctypes.c_int] * 4
    lib.oracle_attention.restype = ctypes.c_int
    lib.oracle_layer_step.argtypes = [_F, _F, _F, _F, _F, _F] + [ctypes.c_int] * 4 + [ctypes.c_float]
    lib.oracle_layer_step.restype = ctypes.c_int
    lib.oracle_decode_step.argtypes = [_F] * 6 + [ctypes.c_int] * 6 + [ctypes.c_float]
    lib.oracle_decode_step.restype = ctypes.c_int
    lib.oracle_attention_ragged.argtypes = [_F, _F, _F, _I64, _I32, _F] + [ctypes.c_int] * 5
    lib.oracle_attention_ragged.restype = ctypes.c_int
    lib.oracle_prefill.argtypes = [_F, _F, _F, _F] + [ctypes.c_int] * 8
    lib.oracle_prefill.restype = ctypes.c_int
    lib.oracle_max_threads.argtypes = []
    lib.oracle_max_threads.restype = ctypes.c_int
    lib.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
    lib.oracle_f16_to_f32.restype = ctypes.c_float
    lib.oracle_dequant.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_uint64]
    lib.oracle_dequant.restype = ctypes.c_float
    lib.oracle_matmul_q.argtypes = [ctypes.c_int, ctypes.c_void_p, _F, _F, ctypes.c_int, ctypes.c_int]
    lib.oracle_matmul_q.restype = ctypes.c_int
    lib.oracle_qkv.argtypes = ([ctypes.c_void_p] * 3 + [ctypes.c_int, _F] + [ctypes.c_void_p] * 3 + [_F] * 3 +
                               [ctypes.c_int] * 4)
    lib.oracle_qkv.restype = ctypes.c_int
    lib.oracle_f32_to_f16_trunc.argtypes = [ctypes.c_float]
    lib.oracle_f32_to_f16_trunc.restype = ctypes.c_uint16
    lib.oracle_quantize_q8_0_block.argtypes = [_F, ctypes.c_void_p]
    lib.oracle_quantize_q8_0_block.restype = None
    lib.oracle_q8_kv_rows.argtypes = [_F, ctypes.c_int64, ctypes.c_void_p]
    lib.oracle_q8_kv_rows.restype = None
    lib.oracle_q8_kv_widen.argtypes = [ctypes.c_void_p, ctypes.c_int64, _F]
    lib.oracle_q8_kv_widen.restype = None
    _libs[path] = lib
    return lib


def lib(timing: bool = False) -> ctypes.CDLL:
    return _load(TIMING_LIB if timing else PARITY_LIB)


def _fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_F)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---------------------------------------------------------------- RNG
def normal(seed: int, shape) -> np.ndarray:
    """N(0,1) fp32 from stream ``seed`` (splitmix64 -> xoshiro256** -> Box-Muller)."""
    out = np.empty(shape, dtype=np.float32)
    lib().tmac_fill_normal(ctypes.c_uint64(seed), _fp(out), out.size)
    return out


def xoshiro256ss(state, n: int) -> list[int]:
    """First n outputs of xoshiro256** from the raw 4-word state."""
    buf = ctypes.create_string_buffer(64)  # tmac_rng: 4 x u64 + int + double
    st = (ctypes.c_uint64 * 4)(*state)
    lib().tmac_rng_set_state(buf, st)
    return [lib().tmac_rng_next(buf) for _ in range(n)]


def splitmix64(state: int, n: int) -> list[int]:
    st = ctypes.c_uint64(state)
    return [lib().tmac_splitmix64(ctypes.byref(st)) for _ in range(n)]


# ---------------------------------------------------------------- path
def rope_heads(x, n_heads: int, head_dim: int, pos: int, base: float = 1e6) -> np.ndarray:
    y = _f32(x).copy()
    assert y.size == n_heads * head_dim
    lib().oracle_rope_heads(_fp(y), n_heads, head_dim, pos, base)
    return y


def rope(q, k, n_head: int, n_kv_head: int, head_dim: int, pos: int, base: float = 1e6):
    return (rope_heads(q, n_head, head_dim, pos, base), rope_heads(k, n_kv_head, head_dim, pos, base))


def rope_theta(head_dim: int, base: float = 1e6) -> np.ndarray:
    t = np.empty(head_dim // 2, dtype=np.float32)
    lib().oracle_rope_theta(_fp(t), head_dim, base)
    return t


def cache_write(cache: np.ndarray, row: int, src) -> None:
    """In place: cache[row, ...] = src (cache is [n_pos][kv_dim] float32)."""
    src = _f32(src).ravel()
    dst = cache.reshape(cache.shape[0], -1)
    assert dst.base is cache or dst is cache or np.shares_memory(dst, cache)
    view = dst[row]
    lib().oracle_cache_write(view.ctypes.data_as(_F), _fp(src), src.size)


def attention(q, k_cache, v_cache, n_head: int, n_kv_head: int, head_dim: int, past_len: int) -> np.ndarray:
    q = _f32(q)
    k_cache = _f32(k_cache)
    v_cache = _f32(v_cache)
    if past_len < 0 or k_cache.size < (past_len + 1) * n_kv_head * head_dim or v_cache.size < k_cache.size:
        raise ValueError("oracle_attention: cache smaller than past_len + 1 rows")
    out = np.empty(n_head * head_dim, dtype=np.float32)
    rc = lib().oracle_attention(_fp(q), _fp(k_cache), _fp(v_cache), _fp(out),
                                n_head, n_kv_head, head_dim, past_len)
    if rc != 0:
        raise ValueError("oracle_attention: bad arguments")
    return out


def layer_step(q, k_new, v_new, k_cache: np.ndarray, v_cache: np.ndarray, n_head: int,
               n_kv_head: int, head_dim: int, pos: int, base: float = 1e6):
    """Reference decode slice for one layer; updates k_cache/v_cache in place.
    Returns (out, q_roped, k_roped)."""
    q = _f32(q).copy()
    k = _f32(k_new).copy()
    v = _f32(v_new)
    assert k_cache.dtype == np.float32 and k_cache.flags["C_CONTIGUOUS"]
    assert v_cache.dtype == np.float32 and v_cache.flags["C_CONTIGUOUS"]
    out = np.empty(n_head * head_dim, dtype=np.float32)
    rc = lib().oracle_layer_step(_fp(q), _fp(k), _fp(v), _fp(k_cache), _fp(v_cache), _fp(out),
                                 n_head, n_kv_head, head_dim, pos, base)
    if rc != 0:
        raise ValueError("oracle_layer_step: bad arguments")
    return out, q, k


def decode_step(q, k_new, v_new, k_cache: np.ndarray, v_cache: np.ndarray, n_head: int, n_kv_head: int,
                head_dim: int, pos: int, base: float = 1e6, timing: bool = False) -> np.ndarray:
    """One decode step over every layer: q [L][n_head*hd], k_new / v_new [L][kdim], caches
    [L][capacity][kdim] (updated in place).  Returns out [L][n_head*hd]."""
    q = _f32(q).copy()
    k = _f32(k_new).copy()
    v = _f32(v_new)
    n_layers, capacity = k_cache.shape[0], k_cache.shape[1]
    assert k_cache.dtype == np.float32 and k_cache.flags["C_CONTIGUOUS"] and k_cache.shape == v_cache.shape
    assert v_cache.dtype == np.float32 and v_cache.flags["C_CONTIGUOUS"]
    out = np.empty((n_layers, n_head * head_dim), dtype=np.float32)
    rc = lib(timing).oracle_decode_step(_fp(q), _fp(k), _fp(v), _fp(k_cache), _fp(v_cache), _fp(out), n_layers,
                                        capacity, n_head, n_kv_head, head_dim, pos, base)
    if rc != 0:
        raise ValueError("oracle_decode_step: bad arguments")
    return out


def attention_ragged(q, k_pool, v_pool, offsets, lengths, n_head: int, n_kv_head: int,
                     head_dim: int, n_threads: int = 1, timing: bool = False) -> np.ndarray:
    q = _f32(q)
    k_pool = _f32(k_pool)
    v_pool = _f32(v_pool)
    offsets = np.ascontiguousarray(offsets, dtype=np.int64)
    lengths = np.ascontiguousarray(lengths, dtype=np.int32)
    n_seq = lengths.size
    out = np.empty((n_seq, n_head * head_dim), dtype=np.float32)
    rc = lib(timing).oracle_attention_ragged(
        _fp(q), _fp(k_pool), _fp(v_pool), offsets.ctypes.data_as(_I64),
        lengths.ctypes.data_as(_I32), _fp(out), n_seq, n_head, n_kv_head, head_dim, n_threads)
    if rc != 0:
        raise ValueError("oracle_attention_ragged: bad arguments")
    return out


def prefill(q, k_cache, v_cache, n_seq: int, n_q: int, prefix_len: int, seq_capacity: int,
            n_head: int, n_kv_head: int, head_dim: int, n_threads: int = 1) -> np.ndarray:
    q = _f32(q)
    k_cache = _f32(k_cache)
    v_cache = _f32(v_cache)
    out = np.empty((n_seq, n_q, n_head * head_dim), dtype=np.float32)
    rc = lib().oracle_prefill(_fp(q), _fp(k_cache), _fp(v_cache), _fp(out), n_seq, n_q,
                              prefix_len, seq_capacity, n_head, n_kv_head, head_dim, n_threads)
    if rc != 0:
        raise ValueError("oracle_prefill: bad arguments")
    return out


def max_threads(timing: bool = False) -> int:
    return lib(timing).oracle_max_threads()


# ---- quantized weights (tmac_gguf.cpp:219-231, 240-250, 311-327, 510-514, 1046-1081) ----
Q5_0, Q8_0, Q4_K, Q6_K = 6, 8, 12, 14
BLOCK_BYTES = {Q5_0: 22, Q8_0: 34, Q4_K: 144, Q6_K: 210}
BLOCK_ELEMS = {Q5_0: 32, Q8_0: 32, Q4_K: 256, Q6_K: 256}


def _u8(a) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint8)
    return a


def f16_to_f32(h: int) -> float:
    return float(lib().oracle_f16_to_f32(int(h) & 0xFFFF))


def dequant(qtype: int, data, idx: int) -> float:
    data = _u8(data)
    return float(lib().oracle_dequant(qtype, data.ctypes.data, idx))


def matmul_q(qtype: int, w, x, rows: int, cols: int) -> np.ndarray:
    """y = W x with the reference's per-row sequential fp32 sum; W is `rows`
    rows of cols/32 blocks of `qtype`."""
    w = _u8(w)
    x = _f32(x)
    if w.size < rows * (cols // BLOCK_ELEMS.get(qtype, 32)) * BLOCK_BYTES.get(qtype, 0) or x.size < cols:
        raise ValueError("matmul_q: buffers too small")
    y = np.empty(rows, dtype=np.float32)
    if lib().oracle_matmul_q(qtype, w.ctypes.data, _fp(x), _fp(y), rows, cols) != 0:
        raise ValueError("oracle_matmul_q: bad arguments")
    return y


def qkv(wq, wk, wv, v_is_q8: bool, x, bq, bk, bv, q_rows: int, k_rows: int, v_rows: int, cols: int):
    """The QKV projection of one layer plus its biases (None = absent)."""
    wq, wk, wv, x = _u8(wq), _u8(wk), _u8(wv), _f32(x)
    bias = [None if b is None else _f32(b) for b in (bq, bk, bv)]
    out = [np.empty(n, dtype=np.float32) for n in (q_rows, k_rows, v_rows)]
    rc = lib().oracle_qkv(wq.ctypes.data, wk.ctypes.data, wv.ctypes.data, int(v_is_q8), _fp(x),
                          *[None if b is None else b.ctypes.data for b in bias], *[_fp(o) for o in out],
                          q_rows, k_rows, v_rows, cols)
    if rc != 0:
        raise ValueError("oracle_qkv: bad arguments")
    return tuple(out)


Q8_HEAD_BYTES = 68  # Q8_0 KV head row: int8 q[64], fp16 d0 (dims 0..31), fp16 d1 (dims 32..63)


def f32_to_f16_trunc(v: float) -> int:
    """fp16 bits as scripts/extract_tmac.py:53-74 (float_to_fp16) writes them."""
    return int(lib().oracle_f32_to_f16_trunc(float(np.float32(v))))


def quantize_q8_0_block(x) -> np.ndarray:
    """32 fp32 values -> the 34-byte Q8_0 block of scripts/extract_tmac.py:159-173."""
    x = _f32(x)
    assert x.size == 32
    out = np.zeros(34, np.uint8)
    lib().oracle_quantize_q8_0_block(_fp(x), out.ctypes.data)
    return out


def q8_kv_rows(x) -> np.ndarray:
    """fp32 values (a multiple of 64) -> Q8_0 KV head rows, uint8 [n / 64][68]."""
    x = _f32(x)
    assert x.size % 64 == 0
    n = x.size // 64
    out = np.zeros((n, Q8_HEAD_BYTES), np.uint8)
    lib().oracle_q8_kv_rows(_fp(x), n, out.ctypes.data)
    return out


def q8_kv_widen(rows) -> np.ndarray:
    """Q8_0 KV head rows (uint8, 68 bytes each) -> fp32 [n_head_rows * 64]."""
    rows = _u8(rows)
    assert rows.size % Q8_HEAD_BYTES == 0
    n = rows.size // Q8_HEAD_BYTES
    out = np.zeros(n * 64, np.float32)
    lib().oracle_q8_kv_widen(rows.ctypes.data, n, _fp(out))
    return out
