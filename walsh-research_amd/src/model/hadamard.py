"""Hadamard-32 ternary linear layers on the fused HIP kernel.

Module surface of src/model/fht_cuda.py (hadamard_matrix :32-56, packing
:65-117, fht :281-337, HadamardTernaryLinear :344-427, HadamardLinear
:436-519, HadamardTernaryLinearTuple :526-569, head mixers :576-670):
same class names, constructor signatures, parameter/buffer names, shapes
and initialisation; forward runs walsh_hadamard_linear_fwd.
"""
import math

import torch
import torch.nn as nn

from . import kernels
from ._common import WeightCache, act_dtype, adjacent_parts_view, tracked_dtype

ALGEBRA_DIM = 32


def hadamard_matrix(n: int, normalize: bool = True) -> torch.Tensor:
    """Sylvester Hadamard matrix H_n (fht_cuda.py:32-56), float32."""
    assert n > 0 and (n & (n - 1)) == 0, f"n must be power of 2, got {n}"
    idx = torch.arange(n)
    bits = (idx[:, None] & idx[None, :])
    parity = torch.zeros_like(bits)
    while bool(bits.any()):
        parity ^= bits & 1
        bits = bits >> 1
    H = (1 - 2 * parity).to(torch.float32)
    if normalize:
        H = H / math.sqrt(n)
    return H


def pack_ternary_weights(w: torch.Tensor) -> torch.Tensor:
    """Pack ternary values {-1,0,1} [.., K] -> uint8 [.., K/4] on the GPU
    (fht_cuda.py:65-93): byte = v0<<6 | v1<<4 | v2<<2 | v3, v = w + 1."""
    assert w.shape[-1] % 4 == 0, f"K dimension must be divisible by 4, got {w.shape[-1]}"
    # values are already ternary: gamma = 1 leaves them unchanged
    one = torch.ones(1, device=w.device, dtype=torch.float32)
    return kernels.ternary_quantize(w.float(), gamma=one, packed=True)["packed"]


def unpack_ternary_weights(packed: torch.Tensor, original_k: int) -> torch.Tensor:
    """Inverse of pack_ternary_weights, float32 (fht_cuda.py:96-117)."""
    return kernels.ternary_unpack(packed, original_k).float()


def _init_latent(out_o: int, in_o: int) -> torch.Tensor:
    # fht_cuda.py:459-466: N(0, 0.02), every group rescaled to Frobenius
    # norm 0.02*sqrt(out_o*in_o)
    w = torch.randn(ALGEBRA_DIM, out_o, in_o) * 0.02
    norms = w.view(ALGEBRA_DIM, -1).norm(dim=1, keepdim=True).unsqueeze(-1)
    return w / (norms + 1e-8) * 0.02 * math.sqrt(out_o * in_o)


class HadamardLinearFunction(torch.autograd.Function):
    """Autograd of the Hadamard linear on the HIP kernels: forward
    walsh_hadamard_linear_fwd, backward walsh_hadamard_linear_bwd (dx through
    the transposed layer, dalpha / dbeta / dW as fixed-order reductions, the
    weight gradient through physics.quantize_ternary's STE clamp,
    physics.py:48-50).  Replaces the graph the reference's einsum + FHTFunction
    (fht_cuda.py:316-337, :497-519) builds."""

    @staticmethod
    def forward(ctx, x, weight, alpha, beta, layer, gsx=None, gsy=None):
        _, _, kw = layer.ternary_state()
        y = kernels.hadamard_linear(x, layer.in_o, layer.out_o, kw, alpha, beta, gsx=gsx, gsy=gsy)
        ctx.layer, ctx.gs = layer, (gsx, gsy)
        ctx.save_for_backward(x, weight, alpha, beta)
        return y

    @staticmethod
    def backward(ctx, gy):
        x, weight, alpha, beta = ctx.saved_tensors
        layer = ctx.layer
        nx, nw, na, nb = ctx.needs_input_grad[:4]
        _, packed, kw = layer.ternary_state()
        kwt = layer.ternary_state_t() if (nx or na) else None
        gsx, gsy = ctx.gs
        gx, da, db, dw = kernels.hadamard_linear_bwd(x, gy.to(x.dtype).contiguous(), layer.in_o, layer.out_o, kw,
                                                      kwt, alpha, beta, latent=weight, need=(nx, na, nb, nw),
                                                      gsx=gsx, gsy=gsy)
        return gx, dw, da, db, None, None, None


class _HadamardBase(nn.Module):
    """Parameters and the HIP forward shared by the Hadamard linear classes."""

    ALGEBRA_DIM = ALGEBRA_DIM

    def _init_params(self, in_features: int, out_features: int):
        assert in_features % ALGEBRA_DIM == 0, f"in_features must be divisible by {ALGEBRA_DIM}"
        assert out_features % ALGEBRA_DIM == 0, f"out_features must be divisible by {ALGEBRA_DIM}"
        self.in_o = in_features // ALGEBRA_DIM
        self.out_o = out_features // ALGEBRA_DIM
        self.weight = nn.Parameter(_init_latent(self.out_o, self.in_o))
        self.alpha = nn.Parameter(torch.ones(ALGEBRA_DIM, self.in_o))
        self.beta = nn.Parameter(torch.ones(ALGEBRA_DIM, self.out_o) * math.sqrt(3.0 / (2.0 * self.in_o)))
        self._wcache = WeightCache()
        self._wcache_t = WeightCache()

    def ternary_state(self):
        """(gamma, packed codes, kernel layout) of the current weight, cached."""
        w = self.weight

        def build():
            q = kernels.ternary_quantize(w, packed=True)
            return q["gamma"], q["packed"], kernels.hadamard_prepare(q["packed"], self.in_o, self.out_o)

        return self._wcache.get([w], build)

    def ternary_state_t(self):
        """Kernel layout of the transposed codes (the input-gradient pass), cached."""
        w = self.weight

        def build():
            _, packed, _ = self.ternary_state()
            return kernels.hadamard_prepare_t(packed, self.in_o, self.out_o)

        return self._wcache_t.get([w], build)

    def _apply_2d(self, x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
        _, _, kw = self.ternary_state()
        return kernels.hadamard_linear(x if x.dtype == dtype else x.to(dtype), self.in_o, self.out_o, kw,
                                       self.alpha, self.beta)

    def _needs_grad(self, x: torch.Tensor) -> bool:
        return torch.is_grad_enabled() and (x.requires_grad or self.weight.requires_grad
                                            or self.alpha.requires_grad or self.beta.requires_grad)

    def apply_rows(self, x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
        """The layer on x [..., 32*in_o] in ``dtype``, differentiable when
        autograd needs it."""
        xin = x if x.dtype == dtype else x.to(dtype)
        if self._needs_grad(xin):
            return HadamardLinearFunction.apply(xin, self.weight, self.alpha, self.beta, self)
        return self._apply_2d(xin, dtype)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        assert x.shape[-1] == self.in_o * ALGEBRA_DIM, f"expected last dim {self.in_o * ALGEBRA_DIM}, got {x.shape[-1]}"
        y = self.apply_rows(x, act_dtype(x))
        return y.to(x.dtype)


class HadamardTernaryLinear(_HadamardBase):
    """y = beta * FHT(W_ternary * FHT(alpha * x)) (fht_cuda.py:344-427)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = False):
        super().__init__()
        self._init_params(in_features, out_features)

    def extra_repr(self) -> str:
        return f"in={self.in_o * ALGEBRA_DIM}, out={self.out_o * ALGEBRA_DIM}, algebra=hadamard32"


class HadamardLinear(_HadamardBase):
    """y = beta * H W_ternary H (alpha * x) (fht_cuda.py:436-519)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = False):
        super().__init__()
        self._init_params(in_features, out_features)
        self.in_features = in_features
        self.out_features = out_features
        self.register_buffer('H', hadamard_matrix(ALGEBRA_DIM, normalize=True))


class HadamardTernaryLinearTuple(nn.Module):
    """Tuple interface over HadamardLinear (fht_cuda.py:526-569): 32 parts
    [..., in_o] in, 32 views [..., out_o] out.  Parts that are adjacent
    slices of one tensor (``x.split``) are read in place, without the cat."""

    ALGEBRA_DIM = ALGEBRA_DIM

    def __init__(self, in_features: int, out_features: int, bias: bool = False):
        super().__init__()
        self.inner = HadamardLinear(in_features, out_features, bias)
        self.in_o = self.inner.in_o
        self.out_o = self.inner.out_o

    @property
    def weight(self):
        return self.inner.weight

    @property
    def beta(self):
        return self.inner.beta

    def forward_full(self, x: torch.Tensor) -> torch.Tensor:
        """Whole rows [..., 32*in_o] -> [..., 32*out_o] in the activation dtype
        (the same result as split -> forward -> cat, without the copies)."""
        return self.inner.apply_rows(x, act_dtype(x))

    def forward_full_rope(self, x: torch.Tensor, freqs_cis: torch.Tensor, head_dim: int):
        """forward_full on x [B, T, C] with apply_rotary_emb (chassis.py:339-345)
        fused into the store, or None when the shapes do not allow it or
        autograd needs the linear's own graph (the caller then applies the
        rotation separately)."""
        inner = self.inner
        if x.dim() != 3 or not kernels.rope_supported(x, inner.out_o, head_dim) or inner._needs_grad(x):
            return None
        dt = act_dtype(x)
        _, _, kw = inner.ternary_state()
        return kernels.hadamard_linear_rope(x if x.dtype == dt else x.to(dt), inner.in_o, inner.out_o, kw,
                                           inner.alpha, inner.beta, freqs_cis, head_dim)

    def forward(self, x_parts: tuple) -> tuple:
        assert len(x_parts) == ALGEBRA_DIM, f"Expected {ALGEBRA_DIM} parts, got {len(x_parts)}"
        x = adjacent_parts_view(x_parts, self.in_o)
        if x is None:
            x = torch.cat(x_parts, dim=-1)
        y = self.inner(x)
        return tuple(y.split(self.out_o, dim=-1))


class HadamardPackedLinear(nn.Module):
    """Inference Hadamard linear holding 2-bit packed codes (fht_cuda.py:751-840):
    buffer ``weight_packed`` [32, out_o, ceil(in_o/4)] uint8 in the
    pack_ternary_weights layout, ``H`` as there, and the trained layer's
    diagonals.  Two defects of the reference class are fixed: ``beta`` keeps
    the trained layer's [32, out_o] shape (the reference holds [out_o] and
    repeats it over the groups, :780, :838-840) and ``alpha`` [32, in_o] is
    applied (the reference drops it, :806, :826-835), so the result equals
    HadamardLinear.forward on the same codes.  Runs the forward kernel on a
    layout prepared once per weight_packed version."""

    ALGEBRA_DIM = ALGEBRA_DIM

    def __init__(self, in_features: int, out_features: int):
        super().__init__()
        assert in_features % ALGEBRA_DIM == 0 and out_features % ALGEBRA_DIM == 0
        self.in_o = in_features // ALGEBRA_DIM
        self.out_o = out_features // ALGEBRA_DIM
        self.in_features = in_features
        self.out_features = out_features
        self.register_buffer('weight_packed', torch.zeros(ALGEBRA_DIM, self.out_o, (self.in_o + 3) // 4,
                                                          dtype=torch.uint8))
        self.register_buffer('alpha', torch.ones(ALGEBRA_DIM, self.in_o))
        self.register_buffer('beta', torch.ones(ALGEBRA_DIM, self.out_o))
        self.register_buffer('H', hadamard_matrix(ALGEBRA_DIM, normalize=True))
        self._wcache = WeightCache()

    @classmethod
    def from_trained(cls, trained_layer) -> 'HadamardPackedLinear':
        """Packed copy of a trained HadamardLinear / HadamardTernaryLinear."""
        layer = getattr(trained_layer, 'inner', trained_layer)
        packed = cls(layer.in_o * ALGEBRA_DIM, layer.out_o * ALGEBRA_DIM).to(layer.weight.device)
        _, pk, _ = layer.ternary_state()
        packed.weight_packed.copy_(pk)
        packed.alpha.copy_(layer.alpha.detach())
        packed.beta.copy_(layer.beta.detach())
        return packed

    def ternary_state(self):
        """(None, packed codes, kernel layout): the HadamardLinear interface."""
        wp = self.weight_packed
        return self._wcache.get([wp], lambda: (None, wp, kernels.hadamard_prepare(wp, self.in_o, self.out_o)))

    def _needs_grad(self, x: torch.Tensor) -> bool:
        return False

    def _apply_2d(self, x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
        _, _, kw = self.ternary_state()
        return kernels.hadamard_linear(x if x.dtype == dtype else x.to(dtype), self.in_o, self.out_o, kw,
                                       self.alpha, self.beta)

    apply_rows = _apply_2d

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        assert x.shape[-1] == self.in_features, f"expected last dim {self.in_features}, got {x.shape[-1]}"
        return self._apply_2d(x, act_dtype(x)).to(x.dtype)


def optimize_for_inference(model: nn.Module) -> nn.Module:
    """Swap every HadamardLinear / HadamardTernaryLinear (also the inner layer
    of a HadamardTernaryLinearTuple) for a HadamardPackedLinear with the same
    codes and diagonals, in place (fht_cuda.py:843-866)."""
    def replace(module):
        for name, child in module.named_children():
            if isinstance(child, _HadamardBase):
                setattr(module, name, HadamardPackedLinear.from_trained(child))
            else:
                replace(child)
    replace(model)
    return model


def fht_butterfly(x: torch.Tensor) -> torch.Tensor:
    """Normalised fast Hadamard transform along the last dim (any power of
    two N <= 16384), fht_cuda.py:281-309, on the GPU."""
    return kernels.fht(x, normalize=True)


class FHTFunction(torch.autograd.Function):
    """Normalised FHT with its backward (fht_cuda.py:316-332): H is symmetric
    and orthonormal, so the gradient is the same transform of grad_y."""

    @staticmethod
    def forward(ctx, x: torch.Tensor) -> torch.Tensor:
        return kernels.fht(x, normalize=True)

    @staticmethod
    def backward(ctx, grad_y: torch.Tensor) -> torch.Tensor:
        return kernels.fht(grad_y, normalize=True)


def fht(x: torch.Tensor) -> torch.Tensor:
    """fht (fht_cuda.py:335-337): FHTFunction.apply."""
    return FHTFunction.apply(x)


def fht_reference(x: torch.Tensor) -> torch.Tensor:
    """fht_reference (fht_cuda.py:266-278) computes the same transform."""
    return kernels.fht(x, normalize=True)


class HadamardHeadMixerFused(nn.Module):
    """Hadamard head mixer (fht_cuda.py:627-662), same parameters.

    On the GPU with head_dim <= 32 (or <= 128 in bf16) it runs
    walsh_head_mixer_fwd: H over the 32 heads, the per-head dense W (bf16
    matrix cores under autocast, as the reference's einsums), H again and
    beta, in one kernel that writes the token-major rows the output
    projection reads.  Other shapes and CPU tensors run the reference's three
    products as torch matmuls."""

    ALGEBRA_DIM = ALGEBRA_DIM

    def __init__(self, head_dim: int):
        super().__init__()
        self.head_dim = head_dim
        self.W = nn.Parameter(torch.randn(ALGEBRA_DIM, head_dim, head_dim) * 0.02)
        self.beta = nn.Parameter(torch.ones(head_dim) * math.sqrt(3.0 / (2.0 * head_dim)))
        self.register_buffer('H', hadamard_matrix(ALGEBRA_DIM, normalize=True))
        self._wcache = WeightCache()

    def uses_kernel(self, x: torch.Tensor) -> bool:
        """The mixer kernel serves inference; when autograd tracks the call
        the torch products (differentiable) run instead."""
        dt = x.dtype if x.dtype in (torch.float32, torch.bfloat16) else torch.float32
        if torch.is_grad_enabled() and (x.requires_grad or self.W.requires_grad or self.beta.requires_grad):
            return False
        return x.is_cuda and kernels.head_mixer_supported(self.head_dim, dt)

    def _kweight(self, dt: torch.dtype) -> torch.Tensor:
        return self._wcache.get([self.W], lambda: kernels.head_mixer_prepare(self.W, dt), extra=(dt,))

    def forward_rows(self, x: torch.Tensor, out: torch.Tensor = None) -> torch.Tensor:
        """x [B, 32, T, D] -> the mixed heads as token-major rows [B, T, 32*D]
        (written into ``out`` when given, see kernels.head_mixer)."""
        B, Hh, T, D = x.shape
        assert Hh == ALGEBRA_DIM
        if self.uses_kernel(x):
            dt = x.dtype if x.dtype in (torch.float32, torch.bfloat16) else torch.float32
            return kernels.head_mixer(x.to(dt), self._kweight(dt), self.beta, out=out)
        r = self.forward(x).transpose(1, 2).reshape(B, T, Hh * D)
        if out is not None:
            out.copy_(r)
            return out
        return r

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        B, Hh, T, D = x.shape
        assert Hh == ALGEBRA_DIM
        if self.uses_kernel(x):
            # a [B, 32, T, D] view of the token-major result
            return self.forward_rows(x).view(B, T, Hh, D).transpose(1, 2)
        out_dt = x.dtype
        tracked = torch.is_grad_enabled()
        dt = tracked_dtype(out_dt) if tracked else out_dt
        x = x.to(dt)
        dev = x.device.type
        with torch.autocast(dev, dtype=torch.get_autocast_dtype(dev), enabled=torch.is_autocast_enabled(dev) and not tracked):
            H = self.H.to(dt).contiguous()          # symmetric: H^T x == H x
            xf = torch.matmul(H, x.reshape(B, Hh, T * D).contiguous()).view(B, Hh, T, D)
            y = torch.matmul(xf, self.W.to(dt).contiguous())
            yf = torch.matmul(H, y.reshape(B, Hh, T * D).contiguous()).view(B, Hh, T, D)
        return (yf * self.beta.to(dt)).to(out_dt)


HadamardHeadMixer = HadamardHeadMixerFused
