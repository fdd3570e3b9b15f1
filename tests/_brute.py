"""Independent fp64 brute force of masked attention with LSE, for tiny inputs.

Written from the definition, not from the oracle: for every (batch, query head, query row)
the visible keys are listed explicitly (k_pos >= 0 and, when causal, k_pos <= q_pos), the
scores scale * q.k are formed one key at a time, lse = log sum exp(score) and
out = sum softmax(score) * v.  A row without a visible key gives (0, -inf).  Query head h
reads KV head kv_map[h] (default h // (Hq / Hkv)).
"""

from __future__ import annotations

import math

import numpy as np


def attention(q, k, v, q_pos, k_pos, causal=True, scale=None, kv_map=None):
    """Arrays q [B,Sq,Hq,D], k/v [B,Sk,Hkv,D], positions [B,S] -> out [B,Sq,Hq,D], lse [B,Hq,Sq]."""
    q, k, v = (np.asarray(t, dtype=np.float64) for t in (q, k, v))
    q_pos, k_pos = np.asarray(q_pos), np.asarray(k_pos)
    B, Sq, Hq, D = q.shape
    Sk, Hkv = k.shape[1], k.shape[2]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if kv_map is None:
        kv_map = [h // (Hq // Hkv) for h in range(Hq)]
    out = np.zeros((B, Sq, Hq, D))
    lse = np.full((B, Hq, Sq), -np.inf)
    for b in range(B):
        for h in range(Hq):
            kh = kv_map[h]
            for i in range(Sq):
                keys = [j for j in range(Sk)
                        if k_pos[b, j] >= 0 and (not causal or k_pos[b, j] <= q_pos[b, i])]
                if not keys:
                    continue
                s = np.array([scale * float(np.dot(q[b, i, h], k[b, j, kh])) for j in keys])
                m = s.max()
                l = m + math.log(float(np.exp(s - m).sum()))
                p = np.exp(s - l)
                out[b, i, h] = sum(p[n] * v[b, j, kh] for n, j in enumerate(keys))
                lse[b, h, i] = l
    return out, lse


def visible_count(q_pos, k_pos, causal=True) -> int:
    """Number of (query, key) pairs with the key visible, per batch row summed."""
    q_pos, k_pos = np.asarray(q_pos), np.asarray(k_pos)
    n = 0
    for b in range(q_pos.shape[0]):
        kp = k_pos[b][k_pos[b] >= 0]
        for qp in q_pos[b]:
            n += int((kp <= qp).sum()) if causal else int(kp.size)
    return n
