"""Synthetic inputs of the benchmark configurations.

Every value comes from a seeded stream of tmac_synth_normal / tmac_synth_uniform
(splitmix64 -> xoshiro256** -> Box-Muller in double, rounded to fp32), so the
benchmark and the parity tests draw identical inputs.  Host only: nothing here
touches the GPU.

Stream ids:
  config 1  q, K, V = streams 10, 11, 12 (one stream per tensor)
  config 2  layer l: stream 2*1000 + l, each decode step taking the pre-RoPE
            q [n_head*64], then k_new [n_kv*64], then v_new [n_kv*64] in turn
  config 3-5  stream_id(config, tensor, index) = ((config*16 + tensor) << 32) + index,
            tensor Q = 0, K = 1, V = 2, LENGTHS = 5 (uniforms); index = sequence.
            Sequence s's query rows and cache rows each come from their own
            stream, so large caches fill in parallel.
  config 4  lengths L_s = 1 + floor(u_s * max_len), u = the first n_seq uniforms
            of stream_id(4, LENGTHS)
"""
from __future__ import annotations

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

import tmac_attn

NH, NKV, HD = 14, 2, 64
QD = NH * HD
KVD = NKV * HD
Q, K, V, LENGTHS = 0, 1, 2, 5


def stream_id(config: int, tensor: int, index: int = 0) -> int:
    return ((config * 16 + tensor) << 32) + index


def _threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def fill_streams(out: np.ndarray, row_starts, seeds) -> np.ndarray:
    """out[row_starts[i]:row_starts[i+1]] = normals of stream seeds[i] (2-D `out`, in parallel)."""
    assert out.dtype == np.float32 and out.flags["C_CONTIGUOUS"] and out.ndim == 2
    bounds = list(row_starts) + [out.shape[0]]

    def one(i):
        lo, hi = bounds[i], bounds[i + 1]
        if hi > lo:
            tmac_attn.synth_normal(seeds[i], None, out=out[lo:hi])

    with ThreadPoolExecutor(_threads()) as pool:
        list(pool.map(one, range(len(seeds))))
    return out


def per_sequence(config: int, tensor: int, n_seq: int, rows: int, cols: int) -> np.ndarray:
    """[n_seq * rows, cols]: sequence s's rows from stream_id(config, tensor, s)."""
    out = np.empty((n_seq * rows, cols), np.float32)
    return fill_streams(out, [s * rows for s in range(n_seq)], [stream_id(config, tensor, s) for s in range(n_seq)])


def c1():
    """Config 1: q [14*64], 256 cache rows of K and V; the query sits at position 255."""
    return (tmac_attn.synth_normal(10, QD), tmac_attn.synth_normal(11, (256, KVD)),
            tmac_attn.synth_normal(12, (256, KVD)))


def c2(layers: int = 24, steps: int = 256):
    """Config 2: pre-RoPE q [steps][layers][14*64], k_new / v_new [steps][layers][2*64]."""
    q = np.empty((steps, layers, QD), np.float32)
    kn = np.empty((steps, layers, KVD), np.float32)
    vn = np.empty((steps, layers, KVD), np.float32)
    for layer in range(layers):
        x = tmac_attn.synth_normal(2 * 1000 + layer, steps * (QD + 2 * KVD)).reshape(steps, -1)
        q[:, layer] = x[:, :QD]
        kn[:, layer] = x[:, QD:QD + KVD]
        vn[:, layer] = x[:, QD + KVD:]
    return q, kn, vn


def c3(n_seq: int = 256, n_pos: int = 4096):
    """Config 3: q [n_seq][14*64]; K, V [n_seq * n_pos][2*64] (sequence s at rows s*n_pos..)."""
    q = per_sequence(3, Q, n_seq, 1, QD)
    k = per_sequence(3, K, n_seq, n_pos, KVD)
    v = per_sequence(3, V, n_seq, n_pos, KVD)
    return q, k, v


def c4_lengths(n_seq: int = 16, max_len: int = 32768) -> np.ndarray:
    u = tmac_attn.synth_uniform(stream_id(4, LENGTHS), n_seq)
    return (1 + np.floor(u * max_len)).astype(np.int32)


def c4(n_seq: int = 16, max_len: int = 32768):
    """Config 4: ragged lengths, packed pool (sequence s at offsets[s]).
    Returns q [n_seq][14*64], K, V [sum L][2*64], offsets (int64), lengths (int32)."""
    lens = c4_lengths(n_seq, max_len)
    offs = np.concatenate([[0], np.cumsum(lens[:-1], dtype=np.int64)]).astype(np.int64)
    total = int(lens.sum())
    q = per_sequence(4, Q, n_seq, 1, QD)
    k = fill_streams(np.empty((total, KVD), np.float32), offs, [stream_id(4, K, s) for s in range(n_seq)])
    v = fill_streams(np.empty((total, KVD), np.float32), offs, [stream_id(4, V, s) for s in range(n_seq)])
    return q, k, v, offs, lens


def c5(n_seq: int = 4, n_q: int = 512, prefix: int = 1536):
    """Config 5: q [n_seq][n_q][14*64]; K, V [n_seq][prefix + n_q][2*64]."""
    cap = prefix + n_q
    q = per_sequence(5, Q, n_seq, n_q, QD).reshape(n_seq, n_q, QD)
    k = per_sequence(5, K, n_seq, cap, KVD).reshape(n_seq, cap, KVD)
    v = per_sequence(5, V, n_seq, cap, KVD).reshape(n_seq, cap, KVD)
    return q, k, v
