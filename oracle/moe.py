"""Oracle: HadamardRouter, FastMoEExperts and HadamardMoE forward.

Test infrastructure only (see ``oracle/__init__.py``).

Expert e owns the contiguous 32-wide feature block x[..., 32e:32e+32]
(``src/model/moe.py:536-539``) and is a SwiGLU with hidden size
32*expansion whose three weight tensors are absmean-ternarised with the
gamma-scaled quantiser (``moe.py:268-303``).
"""
import numpy as np

from . import ternary


def silu(a):
    return a / (1.0 + np.exp(-a))


def router_logits(x, w1, w2) -> np.ndarray:
    """logits = W2 silu(W1 x), no biases (``moe.py:407-411, 431``).
    x [M, C], w1 [C/4, C], w2 [E, C/4]; float64."""
    x = np.asarray(x, np.float64)
    h = silu(x @ np.asarray(w1, np.float64).T)
    return h @ np.asarray(w2, np.float64).T


def softmax(logits) -> np.ndarray:
    z = np.asarray(logits, np.float64)
    z = z - z.max(axis=-1, keepdims=True)
    e = np.exp(z)
    return e / e.sum(axis=-1, keepdims=True)


def topk_indices(probs, k) -> np.ndarray:
    """Indices of the k largest entries per row, largest first; equal values
    are ordered by lower index first.  (``moe.py:434-436`` uses
    ``torch.topk``; with distinct values the selected set is identical.)"""
    p = np.asarray(probs)
    order = np.lexsort((np.broadcast_to(np.arange(p.shape[-1]), p.shape), -p), axis=-1)
    return order[..., :k]


def route_from_probs(probs, max_experts):
    """Top-k routing on given probabilities (``moe.py:434-447``).

    k = min(max_experts, E) for every token -- the reference stores
    ``threshold`` and ``min_experts`` but never reads them (``moe.py:400-403``).
    Returns (weights, mask, topk_idx): mask is 1.0 on the selected experts,
    weights = probs*mask / max(sum(probs*mask), 1e-8).
    """
    p = np.asarray(probs, np.float64)
    E = p.shape[-1]
    k = min(max_experts, E)
    idx = topk_indices(p, k)
    mask = np.zeros_like(p)
    np.put_along_axis(mask, idx, 1.0, axis=-1)
    masked = p * mask
    s = np.maximum(masked.sum(axis=-1, keepdims=True), 1e-8)
    return masked / s, mask, idx


def experts_forward(x_blocks, gate_c, up_c, down_c, g_gate, g_up, g_down, weights) -> np.ndarray:
    """All-expert SwiGLU (``moe.py:337-380``), float64.

    x_blocks [M, E, D]; gate/up codes [E, H, D], down codes [E, D, H];
    gammas are the per-tensor absmean scales (the quantiser returns
    code*gamma); weights [M, E] are the routing weights (0 for unselected
    experts, so those output blocks are exactly zero).
    """
    x = np.asarray(x_blocks, np.float64)
    gw = gate_c.astype(np.float64) * float(g_gate)
    uw = up_c.astype(np.float64) * float(g_up)
    dw = down_c.astype(np.float64) * float(g_down)
    g = np.einsum('med,ehd->meh', x, gw)
    u = np.einsum('med,ehd->meh', x, uw)
    h = silu(g) * u
    out = np.einsum('meh,edh->med', h, dw)
    return out * np.asarray(weights, np.float64)[..., None]


def aux_loss(probs, mask) -> float:
    """Switch-style balance loss E * sum_e mean(mask_e) * mean(p_e)
    (``moe.py:544-560``)."""
    p = np.asarray(probs, np.float64).reshape(-1, probs.shape[-1])
    m = np.asarray(mask, np.float64).reshape(-1, mask.shape[-1])
    return float((m.mean(0) * p.mean(0)).sum() * p.shape[-1])


def moe_forward(x, w1, w2, gate_w, up_w, down_w, max_experts):
    """HadamardMoE.forward (``moe.py:512-542``) from latent weights.

    x [M, C] float; returns dict(out [M, C], probs, mask, weights, idx, aux,
    gammas, codes).  Quantisation follows ``oracle.ternary.moe_quantized``.
    """
    x = np.asarray(x, np.float64)
    M, C = x.shape
    E = np.asarray(w2).shape[0]
    D = C // E
    probs = softmax(router_logits(x, w1, w2))
    weights, mask, idx = route_from_probs(probs, max_experts)
    gc, gg, _ = ternary.moe_quantized(gate_w)
    uc, gu, _ = ternary.moe_quantized(up_w)
    dc, gd, _ = ternary.moe_quantized(down_w)
    out = experts_forward(x.reshape(M, E, D), gc, uc, dc, gg, gu, gd, weights)
    return dict(out=out.reshape(M, C), probs=probs, mask=mask, weights=weights, idx=idx,
                aux=aux_loss(probs, mask), gammas=(gg, gu, gd), codes=(gc, uc, dc))
