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


def test_causal_matches_torch_sdpa_float64():
    rng = np.random.default_rng(2)
    for (B, H, T, D) in ((1, 2, 1, 16), (2, 3, 37, 16), (1, 2, 130, 64)):
        q, k, v = (rng.normal(size=(B, H, T, D)) for _ in range(3))
        ref = F.scaled_dot_product_attention(torch.tensor(q), torch.tensor(k), torch.tensor(v), is_causal=True)
        assert np.allclose(attention.causal_attention_f64(q, k, v), ref.numpy(), rtol=1e-12, atol=1e-12)


def test_causal_closed_forms():
    rng = np.random.default_rng(3)
    B, H, T, D = 1, 2, 11, 16
    v = rng.normal(size=(B, H, T, D))
    q = rng.normal(size=(B, H, T, D))
    # equal keys: query t gets the mean of v[0..t] (a prefix mean)
    k = np.ones((B, H, T, D))
    o = attention.causal_attention_f64(q, k, v)
    for t in range(T):
        assert np.allclose(o[:, :, t], v[:, :, :t + 1].mean(axis=2))
    # query 0 sees only key 0; the last query row equals the decode oracle over all keys
    k = rng.normal(size=(B, H, T, D))
    o = attention.causal_attention_f64(q, k, v)
    assert np.allclose(o[:, :, 0], v[:, :, 0])
    assert np.allclose(o[:, :, -1], attention.decode_attention_f64(q[:, :, -1], k, v))
