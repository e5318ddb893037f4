"""Oracle: decode attention over a KV cache, and causal self-attention.

Test infrastructure only (see ``oracle/__init__.py``).

``causal_attention_f64``: ``src/model/chassis.py:465`` without a cache,
F.scaled_dot_product_attention(q, k, v, is_causal=True): query t attends to
keys 0..t with scale 1/sqrt(head_dim).

``src/model/chassis.py:441-478`` with a cache (``:262-330``) at T == 1:
F.scaled_dot_product_attention(q, k, v) without a mask, i.e. for every
(sequence, head) o = softmax(q . k_j * scale over the L cached j) @ V with
scale = 1/sqrt(head_dim).
"""
import math

import numpy as np


def decode_attention_f64(q, k, v, scale=None) -> np.ndarray:
    """q [B, H, D], k / v [B, H, L, D] -> o [B, H, D] in float64."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    D = q.shape[-1]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    s = np.einsum('bhd,bhjd->bhj', q, k) * scale
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p = p / p.sum(axis=-1, keepdims=True)
    return np.einsum('bhj,bhjd->bhd', p, v)


def causal_attention_f64(q, k, v, scale=None) -> np.ndarray:
    """q, k, v [B, H, T, D] -> o [B, H, T, D] in float64."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    T, D = q.shape[-2], q.shape[-1]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    s = np.einsum('bhtd,bhjd->bhtj', q, k) * scale
    s = np.where(np.tril(np.ones((T, T), bool)), s, -np.inf)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p = p / p.sum(axis=-1, keepdims=True)
    return np.einsum('bhtj,bhjd->bhtd', p, v)
