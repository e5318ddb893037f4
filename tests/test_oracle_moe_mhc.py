"""Pins for oracle.moe and oracle.mhc."""
import numpy as np
import torch

from oracle import mhc, moe


# ----------------------------------------------------------------- routing

def test_topk_brute_force_with_ties():
    rng = np.random.default_rng(0)
    p = rng.integers(0, 5, size=(200, 16)).astype(np.float64)   # many ties
    for k in (1, 3, 6, 16):
        idx = moe.topk_indices(p, k)
        for r in range(p.shape[0]):
            ref = sorted(range(16), key=lambda e: (-p[r, e], e))[:k]
            assert idx[r].tolist() == ref


def test_topk_selected_set_matches_torch_when_distinct():
    rng = np.random.default_rng(1)
    p = moe.softmax(rng.standard_normal((500, 16)))
    idx = moe.topk_indices(p, 6)
    _, ti = torch.from_numpy(p).topk(6, dim=-1)
    assert np.array_equal(np.sort(idx, -1), np.sort(ti.numpy(), -1))
    assert np.array_equal(idx, ti.numpy())      # both order largest first


def test_route_weights_and_mask():
    rng = np.random.default_rng(2)
    p = moe.softmax(rng.standard_normal((100, 16)))
    w, m, idx = moe.route_from_probs(p, max_experts=6)
    assert np.all(m.sum(-1) == 6)
    assert np.allclose(w.sum(-1), 1.0)
    assert np.all(w[m == 0] == 0)
    # k = min(max_experts, E)
    w2, m2, _ = moe.route_from_probs(p[:, :4], max_experts=6)
    assert np.all(m2 == 1)


def test_experts_per_block_brute_force():
    rng = np.random.default_rng(3)
    M, E, D, H = 5, 4, 32, 128
    x = rng.standard_normal((M, E, D))
    gc = rng.integers(-1, 2, (E, H, D)).astype(np.int8)
    uc = rng.integers(-1, 2, (E, H, D)).astype(np.int8)
    dc = rng.integers(-1, 2, (E, D, H)).astype(np.int8)
    wts = rng.uniform(0, 1, (M, E))
    wts[:, 1] = 0.0
    out = moe.experts_forward(x, gc, uc, dc, 0.5, 0.25, 0.125, wts)
    for t in range(M):
        for e in range(E):
            g = 0.5 * gc[e].astype(float) @ x[t, e]
            u = 0.25 * uc[e].astype(float) @ x[t, e]
            h = g / (1 + np.exp(-g)) * u
            ref = wts[t, e] * (0.125 * dc[e].astype(float) @ h)
            assert np.allclose(out[t, e], ref)
    assert np.all(out[:, 1] == 0)


def test_aux_loss_uniform_closed_form():
    # uniform probs, balanced mask with k of E chosen: aux = E * E*(k/E)*(1/E) = k
    E, k = 16, 6
    p = np.full((32, E), 1 / E)
    m = np.zeros((32, E))
    for r in range(32):
        m[r, [(r + j) % E for j in range(k)]] = 1
    assert np.isclose(moe.aux_loss(p, m), k)


def test_moe_forward_shapes_and_zero_blocks():
    rng = np.random.default_rng(4)
    C, E = 128, 4
    x = rng.standard_normal((9, C))
    r = moe.moe_forward(x, rng.normal(0, .02, (C // 4, C)), rng.normal(0, .02, (E, C // 4)),
                        rng.uniform(-1, 1, (E, 128, 32)), rng.uniform(-1, 1, (E, 128, 32)),
                        rng.uniform(-1, 1, (E, 32, 128)), max_experts=2)
    out = r['out'].reshape(9, E, 32)
    unsel = r['mask'] == 0
    assert np.all(out[unsel] == 0)
    assert abs(r['gammas'][0] - 0.5) < 0.02          # absmean of U(-1, 1)


# ----------------------------------------------------------------- sinkhorn

def test_sinkhorn_invariants():
    rng = np.random.default_rng(5)
    h = rng.standard_normal((100, 4, 4))
    m = mhc.sinkhorn(h)
    assert np.all(m > 0)
    assert np.max(np.abs(m.sum(-1) - 1.0)) < 2e-8     # last step normalised rows (eps 1e-8)
    assert np.max(np.abs(m.sum(-2) - 1.0)) < 1e-5     # columns converge
    assert np.allclose(mhc.sinkhorn(np.zeros((1, 1, 1))), 1.0)


def test_sinkhorn_first_step_closed_form():
    h = np.log(np.array([[[1.0, 2.0], [3.0, 4.0]]]))
    m = mhc.sinkhorn(h, n_iter=1, eps=0.0)
    c = np.array([[1 / 4, 2 / 6], [3 / 4, 4 / 6]])
    ref = c / c.sum(-1, keepdims=True)
    assert np.allclose(m[0], ref)


def test_sinkhorn_identity_bias_stays_diagonal():
    m = mhc.sinkhorn(2 * np.eye(4)[None])
    assert np.allclose(np.diag(m[0]), np.e ** 2 / (np.e ** 2 + 3), atol=1e-6)


def test_sinkhorn_float32_close_to_float64():
    rng = np.random.default_rng(6)
    h = rng.standard_normal((50, 4, 4))
    a = mhc.sinkhorn(h.astype(np.float32), dtype=np.float32)
    b = mhc.sinkhorn(h)
    assert np.max(np.abs(a - b)) < 1e-6


def test_sinkhorn_matches_torch_restatement():
    # the reference computes with torch.exp / sum / divide in float32
    rng = np.random.default_rng(7)
    h = rng.standard_normal((64, 4, 4)).astype(np.float32)
    t = torch.exp(torch.from_numpy(h))
    for _ in range(20):
        t = t / (t.sum(-2, keepdim=True) + 1e-8)
        t = t / (t.sum(-1, keepdim=True) + 1e-8)
    assert np.max(np.abs(t.numpy() - mhc.sinkhorn(h, dtype=np.float32))) < 1e-6


# ----------------------------------------------------------------- mapping / stream

def test_mapping_zero_phi_gives_bias_transforms():
    n, C, M = 4, 8, 3
    x = np.random.default_rng(8).standard_normal((M, n * C))
    bias = np.array([[0.0, 1.0, -1.0, 2.0]])
    pre = mhc.mapping(x, np.zeros((n, n * C)), 0.01, bias, 'pre', n, 1e-6)
    post = mhc.mapping(x, np.zeros((n, n * C)), 0.01, bias, 'post', n, 1e-6)
    assert np.allclose(pre[:, 0], mhc.sigmoid(bias[0]))
    assert np.allclose(post, 2 * pre)
    res = mhc.mapping(x, np.zeros((n * n, n * C)), 0.01, 2 * np.eye(n), 'res', n, 1e-6)
    assert np.allclose(res, mhc.sinkhorn(2 * np.eye(n)[None]))


def test_mapping_rms_scale_invariance():
    # phi(x / rms(x)) ignores the scale of x (eps -> 0)
    rng = np.random.default_rng(9)
    n, C = 4, 16
    x = rng.standard_normal((5, n * C))
    phi = rng.standard_normal((n, n * C))
    a = mhc.mapping(x, phi, 0.5, np.zeros((1, n)), 'pre', n, 0.0)
    b = mhc.mapping(7.5 * x, phi, 0.5, np.zeros((1, n)), 'pre', n, 0.0)
    assert np.allclose(a, b)


def test_stream_identity_layer_closed_form():
    rng = np.random.default_rng(10)
    n, C, M = 4, 8, 6
    x = rng.standard_normal((M, n, C))
    maps = dict(pre=(rng.standard_normal((n, n * C)), 0.3, np.zeros((1, n))),
                post=(rng.standard_normal((n, n * C)), 0.3, np.zeros((1, n))),
                res=(rng.standard_normal((n * n, n * C)), 0.3, 2 * np.eye(n)))
    x_new, hp, hq, hr, li = mhc.stream_forward(x, maps, lambda v: v, 1e-6)
    for t in range(M):
        l_in = sum(hp[t, 0, s] * x[t, s] for s in range(n))
        for r in range(n):
            ref = sum(hr[t, r, s] * x[t, s] for s in range(n)) + hq[t, 0, r] * l_in
            assert np.allclose(x_new[t, r], ref)
    # rows of H_res sum to one, so a constant stream stays constant when
    # sum(H_pre) * H_post adds nothing (zero layer)
    xc = np.ones((2, n, C))
    x_new, *_ = mhc.stream_forward(xc, maps, lambda v: 0 * v, 1e-6)
    assert np.allclose(x_new, 1.0, atol=1e-6)


def test_rms_eps_values():
    """F.rms_norm(x, shape) with eps=None, the mappings' normalisation
    (mhc.py:291): for float32 and bfloat16 inputs alike it equals
    x * rsqrt(mean(x.float()^2) + 2^-23) rounded to the input dtype, bit for
    bit -- torch normalises in float32 and takes float32's epsilon, not the
    bfloat16 epsilon 2^-7 (which would differ by up to a factor of 4 on
    rows of RMS ~0.02, the scale of the embedding-initialised streams)."""
    assert mhc.rms_eps(np.float32) == float(torch.finfo(torch.float32).eps)
    assert mhc.rms_eps('bfloat16') == float(torch.finfo(torch.float32).eps)
    gen = torch.Generator().manual_seed(0)
    for dtype in (torch.float32, torch.bfloat16):
        for scale in (1e-3, 0.02, 1.0, 30.0):
            x = (torch.randn(64, 512, generator=gen) * scale).to(dtype)
            eps = mhc.rms_eps(np.float32 if dtype == torch.float32 else 'bfloat16')
            xf = x.float()
            ref = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(dtype)
            assert torch.equal(torch.nn.functional.rms_norm(x, (512,)), ref), (dtype, scale)
            if dtype == torch.bfloat16 and scale <= 0.02:
                wrong = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 2.0 ** -7)).to(dtype)
                assert not torch.equal(torch.nn.functional.rms_norm(x, (512,)), wrong)


def test_sinkhorn_bwd_matches_torch_autograd_and_finite_differences():
    """oracle.mhc.sinkhorn_bwd against torch float64 autograd of the
    reference loop (mhc.py:214-229) and central differences."""
    import torch
    from oracle import mhc as omhc
    rng = np.random.default_rng(12)
    for n in (1, 2, 4, 7):
        h = rng.normal(0, 1.5, (5, n, n))
        g = rng.normal(0, 1, (5, n, n))
        ht = torch.tensor(h, requires_grad=True)
        M = torch.exp(ht)
        for _ in range(20):
            M = M / (M.sum(dim=-2, keepdim=True) + 1e-8)
            M = M / (M.sum(dim=-1, keepdim=True) + 1e-8)
        (M * torch.tensor(g)).sum().backward()
        dh = omhc.sinkhorn_bwd(h, g)
        assert np.allclose(dh, ht.grad.numpy(), rtol=1e-10, atol=1e-12)
        eps = 1e-6
        for idx in ((0, 0, 0), (3, n - 1, 0), (4, n // 2, n - 1)):
            e = np.zeros_like(h)
            e[idx] = eps
            fd = ((omhc.sinkhorn(h + e) * g).sum() - (omhc.sinkhorn(h - e) * g).sum()) / (2 * eps)
            assert abs(fd - dh[idx]) <= 1e-6 * max(1.0, abs(fd))
    # rows and columns of the output sum to ~1, so a constant gradient has
    # (almost) no effect: the gradient of sum(M) is ~0
    h = rng.normal(0, 1, (3, 4, 4))
    assert np.abs(omhc.sinkhorn_bwd(h, np.ones_like(h))).max() < 1e-6
