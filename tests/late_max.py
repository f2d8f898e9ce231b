"""Inputs whose online-softmax running max rises late, for the parity tests.

With q, k ~ N(0, 1) at head_dim 64 a score q.k / 8 has a standard deviation of 1
(1.44 in the log2 units the kernels use), so after the first few rows no later
score beats the running max by more than the kernels' lazy-rescale threshold of
8 log2 units: the branch that raises the max and rescales the running sums then
never runs after the first step.  That branch is where the reference's own GPU
kernel is wrong (kernel_flash_attn.metal:76-79: the rescale test can never be
true); the CPU path it must match takes the max over all rows first
(tmac_gguf.cpp:1114-1118).

The helpers here rewrite chosen key rows so that their scores sit at stated
heights (in log2 units) above every other row, for every query head of a kv
group at once:
  * plant: key row p gets the least-norm change (float64, then rounded to fp32)
    that puts the score of every query head h of its kv group at
    B_h + level, B_h = the largest score of head h over the rows not planted.
    Levels 9, 18, 27, ... on ascending rows make each planted row raise the max
    by 9 > 8 over everything before it; a level above 150 (104 in natural
    units) makes one row's weight 1 and every other weight underflow to 0 in
    fp32, so the output must equal that row's V exactly (the closed form of the
    reference's softmax: expf(s - L) with L = s_max).
  * plant_common / common_queries: for prefill, where one key row serves many
    query rows, every query gets a common component mu along the all-ones
    direction and the planted key rows are lambda * ones, so a planted row's
    score is lambda * sum(q) / sqrt(head_dim) for every query and head.
  * gain_ramp: keys scaled up along the sequence (1 -> gain), so the spread of
    the scores, and with it the running max, keeps growing to the last row.
  * rise_margins: float64 check of what the planted inputs do: for each planted
    row, the least (over query heads) amount by which its score exceeds every
    earlier row's score.
"""
from __future__ import annotations

import numpy as np

LOG2E = 1.4426950408889634


def scores_log2(q, k, n_head: int, n_kv: int, hd: int) -> np.ndarray:
    """float64 [n_head][n_rows] scores q_h . k_p * log2(e) / sqrt(hd) of one query against
    fp32 key rows k [n_rows][n_kv * hd]; head h reads kv head h / (n_head / n_kv)."""
    g = n_head // n_kv
    qh = np.asarray(q, np.float64).reshape(n_head, hd)
    kk = np.asarray(k, np.float64).reshape(-1, n_kv, hd)
    s = np.empty((n_head, kk.shape[0]))
    for h in range(n_head):
        s[h] = kk[:, h // g] @ qh[h]
    return s * (LOG2E / np.sqrt(hd))


def key_for_scores(q_group: np.ndarray, z: np.ndarray, target_log2: np.ndarray, hd: int) -> np.ndarray:
    """The least-norm change of key z (float64) after which q_group[i] . key * log2(e) / sqrt(hd)
    equals target_log2[i] for every query row i of q_group [G][hd]."""
    raw = np.asarray(target_log2, np.float64) * (np.sqrt(hd) / LOG2E)
    qg = np.asarray(q_group, np.float64)
    z = np.asarray(z, np.float64)
    return z + qg.T @ np.linalg.solve(qg @ qg.T, raw - qg @ z)


def plant(q, k, rows, levels, n_head: int, n_kv: int, hd: int) -> np.ndarray:
    """Copy of k [n_rows][n_kv * hd] (fp32) in which key row rows[j] scores levels[j] log2 units
    above the largest score, per query head, of the rows not planted."""
    k = np.array(k, np.float32, copy=True)
    rows = [int(r) for r in rows]
    g = n_head // n_kv
    s = scores_log2(q, k, n_head, n_kv, hd)
    keep = np.ones(k.shape[0], bool)
    keep[rows] = False
    base = s[:, keep].max(axis=1) if keep.any() else np.zeros(n_head)
    qh = np.asarray(q, np.float64).reshape(n_head, hd)
    for r, lev in zip(rows, levels):
        for kv in range(n_kv):
            hs = slice(kv * g, (kv + 1) * g)
            new = key_for_scores(qh[hs], k[r, kv * hd:(kv + 1) * hd], base[hs] + lev, hd)
            k[r, kv * hd:(kv + 1) * hd] = new.astype(np.float32)
    return k


def rise_margins(q, k, rows, n_head: int, n_kv: int, hd: int) -> np.ndarray:
    """For each row in rows: min over query heads of (its score - the largest score of the rows
    before it), float64, in log2 units."""
    s = scores_log2(q, k, n_head, n_kv, hd)
    out = []
    for r in rows:
        out.append(float(np.min(s[:, r] - s[:, :r].max(axis=1))) if r > 0 else np.inf)
    return np.array(out)


def dominance(q, k, row: int, n_head: int, n_kv: int, hd: int) -> float:
    """min over query heads of (score of `row` - the largest score of every other row), log2 units."""
    s = scores_log2(q, k, n_head, n_kv, hd)
    others = np.delete(s, row, axis=1)
    return float(np.min(s[:, row] - others.max(axis=1)))


def gain_ramp(k, gain: float) -> np.ndarray:
    """Key row p of k [n_rows][...] multiplied by 1 + (gain - 1) p / (n_rows - 1), fp32."""
    n = k.shape[0]
    f = 1.0 + (gain - 1.0) * np.arange(n, dtype=np.float64) / max(n - 1, 1)
    return (np.asarray(k, np.float64) * f[:, None]).astype(np.float32)


def common_queries(q, mu: float) -> np.ndarray:
    """q + mu (every element), fp32: a common component along the all-ones direction."""
    return (np.asarray(q, np.float64) + mu).astype(np.float32)


def plant_common(k, rows, lambdas) -> np.ndarray:
    """Copy of k [n_rows][width] with row rows[j] = lambdas[j] (every element), fp32."""
    k = np.array(k, np.float32, copy=True)
    for r, lam in zip(rows, lambdas):
        k[int(r)] = np.float32(lam)
    return k
