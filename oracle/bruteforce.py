"""fp64 brute-force attention by explicit loops — TEST INFRASTRUCTURE ONLY.

Independent of torch's kernels: plain Python/numpy loops over every (query,
head, key) for tiny inputs, used to pin the torch restatement in
``oracle/naive.py``. Only tests import it.
"""

from __future__ import annotations

import math

import numpy as np


def attention_loops(
    q: np.ndarray, k: np.ndarray, v: np.ndarray, allowed: np.ndarray, scale: float, n_rep: int
) -> np.ndarray:
    """``q`` [B, Sq, H, D]; ``k``/``v`` [B, T, H_kv, D] (not repeated);
    ``allowed`` bool [B, Sq, T]. Softmax over allowed keys of exp(scale * q.k);
    a row with no allowed key averages V uniformly over all T (the limit the
    reference's finfo.min mask gives). Returns [B, Sq, H, D] float64."""
    b, sq, h, d = q.shape
    t = k.shape[1]
    out = np.zeros((b, sq, h, d))
    for bi in range(b):
        for si in range(sq):
            keys = [ti for ti in range(t) if allowed[bi, si, ti]]
            for hi in range(h):
                g = hi // n_rep
                if not keys:
                    out[bi, si, hi] = v[bi, :, g].astype(np.float64).mean(axis=0)
                    continue
                s = []
                for ti in keys:
                    acc = 0.0
                    for di in range(d):
                        acc += float(q[bi, si, hi, di]) * float(k[bi, ti, g, di])
                    s.append(acc * scale)
                mx = max(s)
                w = [math.exp(x - mx) for x in s]
                z = sum(w)
                for ti, wi in zip(keys, w):
                    out[bi, si, hi] += (wi / z) * v[bi, ti, g].astype(np.float64)
    return out
