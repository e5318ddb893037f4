"""Ternary quantisation and the octonion layer selection
(module surface of src/model/physics.py).

``quantize_ternary`` computes gamma and the codes with the HIP kernels
(walsh_ternary_gamma / walsh_ternary_quantize); the straight-through
gradient of the reference (physics.py:35-39) is kept for autograd users.
"""
import torch

from . import kernels
from .octonion import OctonionFusedLinear, OctonionTernaryLinearRef  # noqa: F401


class TernaryAbsmeanSTE(torch.autograd.Function):
    """BitNet-b1.58 absmean ternary STE (physics.py:13-39): forward returns
    clamp(round(W / gamma), -1, 1) with gamma = mean(|W|) + 1e-8."""

    @staticmethod
    def forward(ctx, w_latent, training=True):
        q = kernels.ternary_quantize(w_latent, codes=True, packed=False)
        return q["codes"].to(w_latent.dtype)

    @staticmethod
    def backward(ctx, grad_output):
        # clamp(grad, -2, 2) (physics.py:35-39) on the GPU
        return kernels.ternary_ste_bwd(grad_output, mode=1).to(grad_output.dtype), None


def quantize_ternary(w, training=True):
    """clamp(W, +-1.5) + (codes - clamp(W, +-1.5)).detach() (physics.py:42-51);
    its value equals the codes exactly."""
    w_quant = TernaryAbsmeanSTE.apply(w, training)
    w_clamped = w.clamp(-1.5, 1.5)
    return w_clamped + (w_quant - w_clamped).detach()


OctonionTernaryLinear = OctonionFusedLinear
