"""Oracle: HadamardChannelModulation (forward and the modulation's backward).

Test infrastructure only (see ``oracle/__init__.py``).  float64 numpy
restatement of ``src/model/moe.py``:

  forward           :676-727   bulk = mean over T, MLP, scale/shift, modulation
  _forward_ternary  :753-762   Linear weights through quantize_ternary (:297-303)
  _forward_pytorch  :729-744   x_mod = x*scale + 0.1*shift; x + r*(x_mod - x)
  _channel_mod_bwd  :155-199   gx = g*(1 + r*(scale - 1)), dscale = r*sum(g*x),
                               dshift = 0.1*r*sum(g) per (batch, block)

and of the block's use (``src/model/mhc.py:528-532``): x + cm(RMSNorm(x))
on the [B*n, T, C] view of the contiguous [B, T, n, C] streams.
"""
import numpy as np

from . import ternary


def silu(a):
    return a / (1.0 + np.exp(-a))


def mlp_weights(w1, w2, use_ternary: bool = True):
    """The float values the MLP multiplies by: code*gamma of the MoE
    quantiser (float32, as torch computes it) or the weights themselves."""
    if use_ternary:
        return (ternary.moe_quantized(np.asarray(w1, np.float32))[2].astype(np.float64),
                ternary.moe_quantized(np.asarray(w2, np.float32))[2].astype(np.float64))
    return np.asarray(w1, np.float64), np.asarray(w2, np.float64)


def scale_shift(x, w1q, w2q, scale_temp: float, n_blocks: int):
    """(scale, shift) [B, n_blocks] of x [B, T, C] (moe.py:693-709) for MLP
    weights already in their multiplied form."""
    x = np.asarray(x, np.float64)
    bulk = x.mean(axis=1)
    h = silu(bulk @ np.asarray(w1q, np.float64).T)
    mods = h @ np.asarray(w2q, np.float64).T
    raw, shift = mods[:, :n_blocks], mods[:, n_blocks:]
    t = min(max(float(scale_temp), 0.1), 0.5)
    return 1.0 + t * np.tanh(raw), shift


def modulate(x, scale, shift, residual_scale: float, shift_scale: float = 0.1):
    """Per-block modulation (moe.py:729-744): x [B, T, C], scale / shift
    [B, n_blocks]; block b = channels [b*C/n, (b+1)*C/n)."""
    x = np.asarray(x, np.float64)
    B, T, C = x.shape
    nb = scale.shape[-1]
    xb = x.reshape(B, T, nb, C // nb)
    s = np.asarray(scale, np.float64).reshape(B, 1, nb, 1)
    h = np.asarray(shift, np.float64).reshape(B, 1, nb, 1)
    xm = xb * s + h * shift_scale
    return (xb + residual_scale * (xm - xb)).reshape(B, T, C)


def channel_mod(x, w1, w2, scale_temp: float, n_blocks: int, residual_scale: float = 0.5,
                use_ternary: bool = True):
    """HadamardChannelModulation.forward: (out, scale, shift)."""
    w1q, w2q = mlp_weights(w1, w2, use_ternary)
    scale, shift = scale_shift(x, w1q, w2q, scale_temp, n_blocks)
    return modulate(x, scale, shift, residual_scale), scale, shift


def modulate_bwd(g, x, scale, residual_scale: float, shift_scale: float = 0.1):
    """Backward of ``modulate`` wrt x, scale, shift (moe.py:155-199)."""
    g = np.asarray(g, np.float64)
    x = np.asarray(x, np.float64)
    B, T, C = x.shape
    nb = scale.shape[-1]
    gb = g.reshape(B, T, nb, C // nb)
    xb = x.reshape(B, T, nb, C // nb)
    s = np.asarray(scale, np.float64).reshape(B, 1, nb, 1)
    gx = (gb * (1.0 + residual_scale * (s - 1.0))).reshape(B, T, C)
    dscale = residual_scale * (gb * xb).sum(axis=(1, 3))
    dshift = shift_scale * residual_scale * gb.sum(axis=(1, 3))
    return gx, dscale, dshift


def rmsnorm(x, w, eps: float = 1e-6):
    """RMSNorm over the last dim (chassis.py:96-106), float64."""
    x = np.asarray(x, np.float64)
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * np.asarray(w, np.float64)


def block_residual(x, norm_w, w1, w2, scale_temp: float, n_blocks: int, residual_scale: float = 0.5,
                   use_ternary: bool = True, eps: float = 1e-6):
    """x + cm(RMSNorm(x)) for x [G, T, C] (moe.py:796-798, mhc.py:531)."""
    out, scale, shift = channel_mod(rmsnorm(x, norm_w, eps), w1, w2, scale_temp, n_blocks, residual_scale,
                                    use_ternary)
    return np.asarray(x, np.float64) + out, scale, shift


def streams_flat_view(x):
    """The [B*n, T, C] view mHCLlamaBlock takes of streams [B, T, n, C]
    (mhc.py:530): a reinterpretation of the contiguous memory, so group
    b*n + j holds tokens j*T/n .. of every stream when n divides T."""
    x = np.ascontiguousarray(x)
    B, T, n, C = x.shape
    return x.reshape(B * n, T, C)
