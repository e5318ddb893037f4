"""Pins of oracle/channel_mod.py (HadamardChannelModulation, moe.py:610-771)
by closed forms the reference's formulas fix, finite differences, the
streams' flat view, and agreement with the model oracle's torch restatement."""
import numpy as np
import pytest
import torch

from oracle import channel_mod as ocm
from oracle import ternary


def _silu(a):
    return a / (1 + np.exp(-a))


def test_zero_second_layer_is_identity():
    """W2 = 0 gives raw scale 0 and shift 0, so scale = 1 and out = x exactly,
    for the dense and the ternary MLP (codes of a zero tensor are 0)."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 7, 64))
    w1 = rng.standard_normal((16, 64))
    for use_ternary in (False, True):
        out, scale, shift = ocm.channel_mod(x, w1, np.zeros((4, 16)), 1.0, 2, 0.5, use_ternary)
        assert np.array_equal(scale, np.ones((3, 2))) and np.array_equal(shift, np.zeros((3, 2)))
        assert np.array_equal(out, x)


@pytest.mark.parametrize("temp,t_eff", [(0.01, 0.1), (0.3, 0.3), (2.0, 0.5)])
@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_saturated_scale_closed_form(temp, t_eff, sign):
    """Positive bulk, positive W1 and W2 scale rows of +-100: tanh saturates
    to +-1, so scale = 1 +- clamp(temp, 0.1, 0.5) and, with zero shift rows,
    out = x (1 + r (scale - 1))."""
    C, nb, r = 64, 4, 0.5
    x = np.full((2, 5, C), 0.7)
    w1 = np.full((C // 4, C), 0.05)
    w2 = np.zeros((2 * nb, C // 4))
    w2[:nb] = 100.0 * sign
    out, scale, shift = ocm.channel_mod(x, w1, w2, temp, nb, r, use_ternary=False)
    s = 1.0 + sign * t_eff
    assert np.allclose(scale, s, rtol=0, atol=1e-15)
    assert np.array_equal(shift, np.zeros((2, nb)))
    assert np.allclose(out, 0.7 * (1 + r * (s - 1)), rtol=1e-15, atol=0)


def test_shift_closed_form():
    """Constant input a, W1 = w everywhere: h_j = silu(C w a) for every j;
    zero scale rows and shift row b = v_b give shift_b = hidden v_b h and
    out = a + r 0.1 shift_b on block b."""
    C, nb, r, a, w = 32, 2, 0.5, 0.4, 0.03
    hidden = C // 4
    x = np.full((1, 3, C), a)
    w1 = np.full((hidden, C), w)
    w2 = np.zeros((2 * nb, hidden))
    v = np.array([0.2, -0.7])
    w2[nb:] = v[:, None]
    out, scale, shift = ocm.channel_mod(x, w1, w2, 1.0, nb, r, use_ternary=False)
    h = _silu(C * w * a)
    assert np.allclose(shift[0], hidden * v * h, rtol=1e-14)
    assert np.array_equal(scale, np.ones((1, nb)))
    expect = np.concatenate([np.full(C // nb, a + r * 0.1 * hidden * vb * h) for vb in v])
    assert np.allclose(out[0], expect[None, :], rtol=1e-14)


def test_bulk_is_mean_over_tokens_per_batch_row():
    """The bulk state averages over T only: a batch row whose tokens are all
    zero gets scale 1 and shift 0 (bulk 0), whatever the other row holds;
    permuting the tokens of a row changes nothing."""
    rng = np.random.default_rng(1)
    C, nb = 64, 2
    x = np.zeros((2, 6, C))
    x[0] = rng.standard_normal((6, C))
    w1 = rng.standard_normal((C // 4, C))
    w2 = rng.standard_normal((2 * nb, C // 4))
    _, scale, shift = ocm.channel_mod(x, w1, w2, 0.4, nb, use_ternary=False)
    assert np.array_equal(scale[1], np.ones(nb)) and np.array_equal(shift[1], np.zeros(nb))
    assert not np.allclose(scale[0], 1.0)
    _, scale_p, shift_p = ocm.channel_mod(x[:, ::-1], w1, w2, 0.4, nb, use_ternary=False)
    assert np.allclose(scale_p, scale, rtol=1e-14) and np.allclose(shift_p, shift, rtol=1e-14, atol=1e-16)


def test_blocks_are_contiguous_channel_ranges():
    """Block b covers channels [b C/nb, (b+1) C/nb): with distinct per-block
    scales and no shift, out / x on channel c is 1 + r (scale_{c // bd} - 1)."""
    C, nb, r = 48, 3, 0.5
    x = np.random.default_rng(2).uniform(0.5, 1.5, (2, 4, C))
    scale = np.array([[0.6, 1.0, 1.4], [1.2, 0.8, 1.1]])
    out = ocm.modulate(x, scale, np.zeros((2, nb)), r)
    bd = C // nb
    for g in range(2):
        ratio = out[g] / x[g]
        for c in range(C):
            assert np.allclose(ratio[:, c], 1 + r * (scale[g, c // bd] - 1), rtol=1e-14)


def test_modulate_matches_triton_algebraic_form():
    """The Triton kernel's rewritten form (moe.py:147-151):
    x (1 + r (scale - 1)) + r shift_scale shift."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 5, 64))
    scale = rng.uniform(0.5, 1.5, (2, 4))
    shift = rng.standard_normal((2, 4))
    r = 0.37
    out = ocm.modulate(x, scale, shift, r)
    s = np.repeat(scale, 16, axis=1)[:, None, :]
    h = np.repeat(shift, 16, axis=1)[:, None, :]
    assert np.allclose(out, x * (1 + r * (s - 1)) + r * 0.1 * h, rtol=1e-13, atol=1e-15)


def test_modulate_bwd_finite_differences():
    rng = np.random.default_rng(4)
    B, T, C, nb, r = 2, 3, 16, 2, 0.5
    x = rng.standard_normal((B, T, C))
    scale = rng.uniform(0.5, 1.5, (B, nb))
    shift = rng.standard_normal((B, nb))
    g = rng.standard_normal((B, T, C))
    gx, ds, dh = ocm.modulate_bwd(g, x, scale, r)

    def loss(x_, s_, h_):
        return float((ocm.modulate(x_, s_, h_, r) * g).sum())
    eps = 1e-6
    for (arr, grad) in ((x, gx), (scale, ds), (shift, dh)):
        num = np.zeros_like(arr)
        for i in np.ndindex(arr.shape):
            p = arr.copy()
            p[i] += eps
            m = arr.copy()
            m[i] -= eps
            args = [x, scale, shift]
            k = [x is arr, scale is arr, shift is arr].index(True)
            args_p, args_m = list(args), list(args)
            args_p[k], args_m[k] = p, m
            num[i] = (loss(*args_p) - loss(*args_m)) / (2 * eps)
        assert np.allclose(grad, num, rtol=1e-7, atol=1e-8)


def test_ternary_mlp_weights_are_moe_quantised():
    rng = np.random.default_rng(5)
    w1 = rng.standard_normal((8, 32)).astype(np.float32) * 0.02
    w2 = rng.standard_normal((4, 8)).astype(np.float32) * 0.01
    q1, q2 = ocm.mlp_weights(w1, w2, True)
    for w, q in ((w1, q1), (w2, q2)):
        c, g, _ = ternary.moe_quantized(w)
        assert set(np.unique(c)) <= {-1, 0, 1}
        assert np.array_equal(q, c.astype(np.float32).astype(np.float64) * np.float64(np.float32(g)))


def test_streams_flat_view_groups_tokens():
    """mHCLlamaBlock's x.view(B*n, T, C) of streams [B, T, n, C]: group
    b*n + j holds tokens j*T/n .. (j+1)*T/n - 1 of every stream, not stream j."""
    B, T, n, C = 2, 4, 2, 3
    x = np.zeros((B, T, n, C))
    for b, t, s in np.ndindex(B, T, n):
        x[b, t, s, :] = 100 * b + 10 * t + s
    f = ocm.streams_flat_view(x)
    assert f.shape == (B * n, T, C)
    for b, j, k in np.ndindex(B, n, T):
        tok, s = divmod(j * T + k, n)
        assert f[b * n + j, k, 0] == 100 * b + 10 * tok + s


def test_model_oracle_channel_mod_matches_numpy():
    """The model oracle's torch restatement (used for the whole-model checks)
    equals the pinned numpy one, forward and, through torch float64
    autograd, the modulation's backward."""
    from oracle.model import Oracle
    rng = np.random.default_rng(6)
    C, G, T = 64, 3, 5
    sd = {'cm.context_mlp.0.weight': torch.tensor(rng.standard_normal((C // 4, C)) * 0.02, dtype=torch.float32),
          'cm.context_mlp.2.weight': torch.tensor(rng.standard_normal((4, C // 4)) * 0.01, dtype=torch.float32),
          'cm.scale_temp': torch.tensor([0.3])}
    x = rng.standard_normal((G, T, C))
    o = Oracle(sd, C, 1, 0)
    got = o.channel_mod(torch.tensor(x, dtype=torch.float32), 'cm', n_blocks=2).numpy()
    ref, scale, _ = ocm.channel_mod(x, sd['cm.context_mlp.0.weight'].numpy(), sd['cm.context_mlp.2.weight'].numpy(),
                                    0.3, 2, 0.5, True)
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()
    og = Oracle(sd, C, 1, 0, grad=True)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    g = rng.standard_normal((G, T, C))
    (og.channel_mod(xt, 'cm', n_blocks=2) * torch.tensor(g)).sum().backward()
    # the modulation's gradient wrt x plus the path through the bulk state:
    # check the direct term by freezing scale / shift (their dependence on x
    # is through the mean only)
    gx_direct, _, _ = ocm.modulate_bwd(g, x, scale, 0.5)
    bulk_path = xt.grad.numpy() - gx_direct
    # the bulk path is the same for every token of a group (d mean / d x_t = 1/T);
    # the numpy scale used float32 gammas, the float64 oracle float64 ones
    assert np.abs(bulk_path - bulk_path[:, :1, :]).max() <= 1e-6 * np.abs(bulk_path).max()
