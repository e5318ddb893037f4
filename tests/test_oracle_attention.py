"""Pins for oracle.attention: torch's float64 CPU scaled_dot_product_attention
and closed forms."""
import numpy as np
import torch
import torch.nn.functional as F

from oracle import attention


def test_matches_torch_sdpa_float64():
    rng = np.random.default_rng(0)
    for (B, H, L, D) in ((2, 3, 1, 16), (1, 4, 37, 64), (2, 2, 300, 128)):
        q = rng.normal(size=(B, H, D))
        k = rng.normal(size=(B, H, L, D))
        v = rng.normal(size=(B, H, L, D))
        ref = F.scaled_dot_product_attention(torch.tensor(q)[:, :, None], torch.tensor(k), torch.tensor(v))[:, :, 0]
        assert np.allclose(attention.decode_attention_f64(q, k, v), ref.numpy(), rtol=1e-12, atol=1e-12)


def test_closed_forms():
    rng = np.random.default_rng(1)
    v = rng.normal(size=(1, 2, 9, 16))
    # equal keys: uniform weights, the mean of V
    k = np.ones((1, 2, 9, 16))
    q = rng.normal(size=(1, 2, 16))
    assert np.allclose(attention.decode_attention_f64(q, k, v), v.mean(axis=2))
    # one key dominating: that key's value
    k = np.zeros((1, 2, 9, 16))
    k[:, :, 4] = 50 * q / np.linalg.norm(q, axis=-1, keepdims=True)
    assert np.allclose(attention.decode_attention_f64(q, k, v), v[:, :, 4], atol=1e-9)
    # L = 1: the single value
    assert np.allclose(attention.decode_attention_f64(q, k[:, :, :1], v[:, :, :1]), v[:, :, 0])
