"""Oracle: Sylvester Hadamard matrix, FHT butterflies, HadamardLinear forward.

Test infrastructure only (see ``oracle/__init__.py``).

Layout (``src/model/fht_cuda.py:497-499``): a row of C = 32*in_o features is
viewed as [32 groups g, in_o columns i], element (g, i) at g*in_o + i.
"""
import math

import numpy as np
import torch

ALGEBRA_DIM = 32


def sylvester(n: int, normalize: bool = True) -> np.ndarray:
    """Sylvester construction H_2k = [[H, H], [H, -H]] (``fht_cuda.py:32-56``)."""
    assert n > 0 and (n & (n - 1)) == 0
    h = np.ones((1, 1), dtype=np.float64)
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    if normalize:
        h = h / math.sqrt(n)
    return h


def fht(x, normalize: bool = True) -> np.ndarray:
    """In-order butterfly FHT along the last axis (``fht_cuda.py:281-309``).

    Stage s pairs index k with k + 2^s inside blocks of 2^(s+1), (a, b) ->
    (a + b, a - b); the result is scaled by 1/sqrt(N) when ``normalize``.
    Vectorised over leading axes; computes in the dtype of ``x``.
    """
    y = np.array(x, copy=True)
    n = y.shape[-1]
    assert n > 0 and (n & (n - 1)) == 0
    lead = y.shape[:-1]
    h = 1
    while h < n:
        y = y.reshape(lead + (n // (2 * h), 2, h))
        a = y[..., 0, :].copy()
        b = y[..., 1, :].copy()
        y[..., 0, :] = a + b
        y[..., 1, :] = a - b
        h *= 2
    y = y.reshape(lead + (n,))
    if normalize:
        y = y * y.dtype.type(1.0 / math.sqrt(n))
    return y


def hadamard_linear_f64(x, codes, alpha, beta) -> np.ndarray:
    """Float64 HadamardLinear forward: y = beta * H W H (alpha * x).

    ``fht_cuda.py:489-519``: x viewed [M, 32, in_o]; alpha [32, in_o]
    scales before the group-axis transform with the normalised H; each group
    g applies its ternary matrix W[g] (out_o x in_o); a second group-axis
    transform with H; beta [32, out_o] scales the result.
    """
    x = np.asarray(x, dtype=np.float64)
    M = x.shape[0]
    G, out_o, in_o = codes.shape
    assert G == ALGEBRA_DIM and x.shape[1] == G * in_o
    H = sylvester(G)
    xs = x.reshape(M, G, in_o) * np.asarray(alpha, np.float64)
    xm = np.einsum('mgi,gh->mhi', xs, H)
    yp = np.einsum('mgi,goi->mgo', xm, codes.astype(np.float64))
    ym = np.einsum('mgo,gh->mho', yp, H)
    y = ym * np.asarray(beta, np.float64)
    return y.reshape(M, G * out_o)


def head_mixer_f64(x, W, beta) -> np.ndarray:
    """Float64 HadamardHeadMixerFused.forward (``fht_cuda.py:650-662``).

    x [B, 32, T, D] (32 attention heads); x_fht[g] = sum_h H[h, g] x[h]
    (``:655``), y[h] = x_fht[h] @ W[h] with W [32, D, D] dense (``:658``),
    y_fht[g] = sum_h H[h, g] y[h] (``:661``), times beta [D] broadcast over
    heads and tokens (``:662``); H the normalised Sylvester matrix.
    """
    x = np.asarray(x, dtype=np.float64)
    B, G, T, D = x.shape
    assert G == ALGEBRA_DIM
    H = sylvester(G)
    xf = np.einsum('bhti,hg->bgti', x, H)
    y = np.einsum('bhti,hio->bhto', xf, np.asarray(W, np.float64))
    yf = np.einsum('bhti,hg->bgti', y, H)
    return yf * np.asarray(beta, np.float64)


def rope_f64(y, freqs_cis, head_dim: int) -> np.ndarray:
    """apply_rotary_emb (``chassis.py:339-345``) on y [B, T, C] in float64:
    C is split into heads of head_dim features; pair (2i, 2i+1) of a head at
    token t turns by freqs_cis[t, i] = cos + i sin (complex [T, head_dim/2]):
    (a, b) -> (a cos - b sin, a sin + b cos).
    """
    y = np.asarray(y, dtype=np.float64)
    B, T, C = y.shape
    f = np.asarray(freqs_cis)[:T]
    c = np.real(f).astype(np.float64)[None, :, None, :]
    s = np.imag(f).astype(np.float64)[None, :, None, :]
    v = y.reshape(B, T, C // head_dim, head_dim // 2, 2)
    a, b = v[..., 0], v[..., 1]
    out = np.stack([a * c - b * s, a * s + b * c], axis=-1)
    return out.reshape(B, T, C)


def hadamard_linear_torch32(x, codes, alpha, beta) -> torch.Tensor:
    """The reference CPU float32 evaluation order (``fht_cuda.py:497-519``).

    Same math as ``hadamard_linear_f64`` with torch-CPU float32 einsums
    against the normalised H, exactly as the reference module runs on CPU.
    Used as the timed CPU baseline and as the float32 comparison point.
    """
    x = torch.as_tensor(x, dtype=torch.float32)
    lead = x.shape[:-1]
    G, out_o, in_o = codes.shape
    H = torch.as_tensor(sylvester(G), dtype=torch.float32)
    w = torch.as_tensor(np.asarray(codes), dtype=torch.float32)
    xs = x.reshape(*lead, G, in_o) * torch.as_tensor(alpha, dtype=torch.float32)
    xm = torch.einsum('...gi,gh->...hi', xs, H)
    yp = torch.einsum('...gi,goi->...go', xm, w)
    ym = torch.einsum('...go,gh->...ho', yp, H)
    y = ym * torch.as_tensor(beta, dtype=torch.float32)
    return y.reshape(*lead, G * out_o)


def dense_matrix(codes, alpha, beta) -> np.ndarray:
    """The layer as one dense [32*out_o, 32*in_o] float64 matrix.

    A = diag(beta) (H (x) I_out) blockdiag(W_0..W_31) (H (x) I_in) diag(alpha),
    built with Kronecker products, independently of the einsum path above.
    """
    G, out_o, in_o = codes.shape
    H = sylvester(G)
    blk = np.zeros((G * out_o, G * in_o))
    for g in range(G):
        blk[g * out_o:(g + 1) * out_o, g * in_o:(g + 1) * in_o] = codes[g]
    left = np.kron(H, np.eye(out_o))
    right = np.kron(H, np.eye(in_o))
    return (np.asarray(beta, np.float64).reshape(-1)[:, None]
            * (left @ blk @ right)
            * np.asarray(alpha, np.float64).reshape(-1)[None, :])


def init_weight(out_o: int, in_o: int, gen: torch.Generator) -> torch.Tensor:
    """Latent weight init of ``fht_cuda.py:459-466`` (each group scaled to
    Frobenius norm 0.02*sqrt(out_o*in_o))."""
    w = torch.randn(ALGEBRA_DIM, out_o, in_o, generator=gen) * 0.02
    n = w.view(ALGEBRA_DIM, -1).norm(dim=1, keepdim=True).unsqueeze(-1)
    return w / (n + 1e-8) * 0.02 * math.sqrt(out_o * in_o)


def beta_init(in_o: int) -> float:
    """Variance-preserving beta init sqrt(3 / (2 in_o)) (``fht_cuda.py:475-476``)."""
    return math.sqrt(3.0 / (2.0 * in_o))


def hadamard_linear_bwd_f64(x, codes, alpha, beta, gy, latent=None):
    """Float64 gradients of ``hadamard_linear_f64`` for the output gradient gy.

    The autograd the reference builds for ``fht_cuda.py:497-519``:
    FHTFunction.backward is the same normalised transform (``:328-332``, H
    symmetric), the einsum's gradients are the transposed contractions, and
    the weight gradient passes physics.quantize_ternary's STE, whose only
    differentiable path is ``w.clamp(-1.5, 1.5)`` (``physics.py:48-50``):
    dlatent = dW_q * [-1.5 <= latent <= 1.5] when ``latent`` is given.

    Returns (dx [M, 32*in_o], dalpha [32, in_o], dbeta [32, out_o],
    dW [32, out_o, in_o]).
    """
    x = np.asarray(x, dtype=np.float64)
    gy = np.asarray(gy, dtype=np.float64)
    M = x.shape[0]
    G, out_o, in_o = codes.shape
    W = codes.astype(np.float64)
    a = np.asarray(alpha, np.float64)
    b = np.asarray(beta, np.float64)
    H = sylvester(G)
    xs = x.reshape(M, G, in_o)
    g = gy.reshape(M, G, out_o)
    xm = np.einsum('mgi,gh->mhi', xs * a, H)
    ym = np.einsum('mgo,gh->mho', np.einsum('mgi,goi->mgo', xm, W), H)
    dbeta = (g * ym).sum(0)
    dyp = np.einsum('mgo,gh->mho', g * b, H)
    dW = np.einsum('mgo,mgi->goi', dyp, xm)
    dxs = np.einsum('mgi,gh->mhi', np.einsum('mgo,goi->mgi', dyp, W), H)
    dalpha = (dxs * xs).sum(0)
    dx = (dxs * a).reshape(M, G * in_o)
    if latent is not None:
        lat = np.asarray(latent, np.float64)
        dW = dW * ((lat >= -1.5) & (lat <= 1.5))
    return dx, dalpha, dbeta, dW
