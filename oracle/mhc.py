"""Oracle: Sinkhorn-Knopp projection, ResidualStreamMapping, mHCResidualStream.

Test infrastructure only (see ``oracle/__init__.py``).
"""
import numpy as np


def sinkhorn(h, n_iter: int = 20, eps: float = 1e-8, dtype=np.float64) -> np.ndarray:
    """M = exp(H); n_iter x {column normalise, then row normalise}.

    ``src/model/mhc.py:214-229``: each step divides by (sum + eps); columns
    first, no max subtraction.  ``dtype`` selects float64 (closed form) or
    float32 (the reference's arithmetic).
    """
    m = np.exp(np.asarray(h, dtype=dtype))
    e = dtype(eps)
    for _ in range(n_iter):
        m = m / (m.sum(axis=-2, keepdims=True) + e)
        m = m / (m.sum(axis=-1, keepdims=True) + e)
    return m


def sinkhorn_bwd(h, g, n_iter: int = 20, eps: float = 1e-8) -> np.ndarray:
    """Float64 reverse-mode gradient of ``sinkhorn`` wrt h for the output
    gradient g (the autograd torch derives for ``mhc.py:214-229``): the
    forward is taped, then each normalisation Y = X / (sum + eps) is undone
    with dX = (dY - sum(dY * Y)) / (sum + eps) along the normalised axis, and
    exp with dh = dM0 * M0."""
    m0 = np.exp(np.asarray(h, np.float64))
    tape = []
    m = m0
    for _ in range(n_iter):
        c = m.sum(axis=-2, keepdims=True) + eps
        t = m / c
        r = t.sum(axis=-1, keepdims=True) + eps
        u = t / r
        tape.append((t, c, u, r))
        m = u
    G = np.asarray(g, np.float64)
    for t, c, u, r in reversed(tape):
        dT = (G - (G * u).sum(axis=-1, keepdims=True)) / r
        G = (dT - (dT * t).sum(axis=-2, keepdims=True)) / c
    return G * m0


def sigmoid(a):
    return 1.0 / (1.0 + np.exp(-a))


def rms_eps(dtype) -> float:
    """The epsilon ``F.rms_norm(x, shape)`` adds when eps is None
    (``mhc.py:291``): torch normalises in the op-math type (float32 for a
    bfloat16 input) and uses that type's epsilon, so 2^-23 for float32 and
    bfloat16 inputs alike, 2^-52 for float64 (checked bit for bit against
    torch's own rms_norm in the oracle tests)."""
    return {np.float32: 2.0 ** -23, 'bfloat16': 2.0 ** -23, np.float64: 2.0 ** -52}[dtype]


def mapping(x_flat, phi, alpha, bias, kind: str, n: int, eps: float, n_iter: int = 20) -> np.ndarray:
    """ResidualStreamMapping.forward (``mhc.py:283-318``), float64.

    x_flat [M, n*C]; phi [out, n*C] (out = n*n for 'res', n otherwise);
    alpha scalar; bias [n, n] or [1, n].
    'res'  -> SK(alpha*phi(x_hat).view(n, n) + bias)       [M, n, n]
    'pre'  -> sigmoid(alpha*phi(x_hat) + bias)             [M, 1, n]
    'post' -> 2*sigmoid(alpha*phi(x_hat) + bias)           [M, 1, n]
    with x_hat = x / sqrt(mean(x^2) + eps) (no weight).
    """
    x = np.asarray(x_flat, np.float64)
    xh = x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + eps)
    dyn = xh @ np.asarray(phi, np.float64).T
    a = float(alpha)
    b = np.asarray(bias, np.float64)
    if kind == 'res':
        return sinkhorn(a * dyn.reshape(-1, n, n) + b, n_iter)
    t = a * dyn + b.reshape(-1)
    s = sigmoid(t)
    return (s if kind == 'pre' else 2.0 * s)[:, None, :]


def stream_forward(x, maps, layer_fn, eps: float):
    """mHCResidualStream.forward (``mhc.py:345-381``), float64.

    x [M, n, C]; maps = dict(pre=(phi, alpha, bias), post=..., res=...).
    x_new = H_res @ x + H_post^T (layer_fn(H_pre @ x)).
    Returns (x_new, H_pre, H_post, H_res, layer_input).
    """
    x = np.asarray(x, np.float64)
    M, n, C = x.shape
    xf = x.reshape(M, n * C)
    hp = mapping(xf, *maps['pre'], 'pre', n, eps)
    hq = mapping(xf, *maps['post'], 'post', n, eps)
    hr = mapping(xf, *maps['res'], 'res', n, eps)
    li = np.einsum('mos,msc->moc', hp, x)[:, 0, :]
    out = np.asarray(layer_fn(li), np.float64)
    x_new = np.einsum('mrs,msc->mrc', hr, x) + hq[:, 0, :, None] * out[:, None, :]
    return x_new, hp, hq, hr, li
