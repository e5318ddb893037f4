"""Octonion (Cayley-Dickson) ternary linear layers on the HIP GEMM kernel.

Module surface of src/model/cayley_dickson_cuda.py (packing :134-187,
cayley_dickson_fused :574-619, OctonionFusedLinear :622-668,
OctonionPackedLinear :702-772, optimize_for_inference :778-818,
OctonionHeadMixerFused :1011-1043) and physics.OctonionTernaryLinearRef
(src/model/physics.py:53-82).
"""
import math

import torch
import torch.nn as nn

from . import kernels
from ._common import WeightCache, act_dtype, adjacent_parts_view
from .constants import SIGN_TABLE, WEIGHT_IDX
from .hadamard import pack_ternary_weights, unpack_ternary_weights  # noqa: F401  (same 2-bit layout)


def _parts_to_rows(x_parts, in_o):
    assert len(x_parts) == 8, f"Expected 8 parts, got {len(x_parts)}"
    x = adjacent_parts_view(x_parts, in_o)
    return torch.cat(x_parts, dim=-1) if x is None else x


def _prepared(cache: WeightCache, w_ternary_src, packed_fn, in_o, out_o, dtype):
    """Expanded block matrix for ``dtype``, cached on the weight version."""
    def build():
        return {}
    store = cache.get([w_ternary_src], build)
    if dtype not in store:
        store[dtype] = kernels.octonion_prepare(packed_fn(), in_o, out_o, dtype)
    return store[dtype]


def cayley_dickson_fused(x_parts, weight: torch.Tensor) -> tuple:
    """y_i = sum_j S[i][j] x_j @ weight[i^j]^T for 8 parts [..., K] and a
    ternary-valued weight [8, N, K] (cayley_dickson_cuda.py:574-619).  Like the
    reference kernel it computes with bf16 operands and returns bf16."""
    K = x_parts[0].shape[-1]
    N = weight.shape[1]
    x = _parts_to_rows(x_parts, K).to(torch.bfloat16)
    one = torch.ones(1, device=weight.device, dtype=torch.float32)
    packed = kernels.ternary_quantize(weight.float(), gamma=one, packed=True)["packed"]
    B = kernels.octonion_prepare(packed, K, N, torch.bfloat16)
    y = kernels.octonion_linear(x, K, N, B, torch.ones(N, device=x.device))
    return tuple(y.split(N, dim=-1))


class OctonionLinearFunction(torch.autograd.Function):
    """Autograd of the octonion layer on the HIP kernels (the role of
    CayleyDicksonFunction, cayley_dickson_cuda.py:428-567): the exact
    transpose of the forward's signed-permutation block matrix for dx, and
    dW / dbeta folded from gy^T x; the weight gradient passes the STE clamp
    of physics.quantize_ternary (physics.py:48-50).  ``fused``: the forward
    is the reference GPU module's (bf16 operands, the product rounded to
    bf16, times beta in float32: a float32 result); the roundings pass the
    gradient straight through."""

    @staticmethod
    def forward(ctx, x, weight, beta, layer, fused):
        if fused:
            y = kernels.octonion_fused_linear(x, layer.in_o, layer.out_o, layer.block_matrix(torch.bfloat16), beta)
        else:
            y = kernels.octonion_linear(x, layer.in_o, layer.out_o, layer.block_matrix(x.dtype), beta)
        ctx.layer = layer
        ctx.save_for_backward(x, weight, beta)
        return y

    @staticmethod
    def backward(ctx, gy):
        x, weight, beta = ctx.saved_tensors
        layer = ctx.layer
        nx, nw, nb, _, _ = ctx.needs_input_grad
        packed = layer.ternary_state()[1]
        gx, dw, db = kernels.octonion_linear_bwd(x, gy.to(x.dtype).contiguous(), layer.in_o, layer.out_o, packed,
                                                 beta, latent=weight, need=(nx, nw, nb))
        return gx, dw, db, None, None


class _OctonionTernaryBase(nn.Module):
    """Parameters of the octonion ternary layers (physics.py:55-64,
    cayley_dickson_cuda.py:628-641): latent ``weight`` [8, out_o, in_o] drawn
    from U(-1, 1) and ``beta`` [out_o] = sqrt(3 / (2 in_o))."""

    def __init__(self, in_features, out_features, bias=False):
        super().__init__()
        assert in_features % 8 == 0 and out_features % 8 == 0
        self.in_o = in_features // 8
        self.out_o = out_features // 8
        self.weight = nn.Parameter(torch.rand(8, self.out_o, self.in_o) * 2 - 1)
        self.beta = nn.Parameter(torch.ones(self.out_o) * math.sqrt(3.0 / (2.0 * self.in_o)))
        self._wcache = WeightCache()
        self._pcache = WeightCache()

    def ternary_state(self):
        """(gamma, packed codes [8, out_o, ceil(in_o/4)]) of the current weight."""
        w = self.weight

        def build():
            q = kernels.ternary_quantize(w, packed=True)
            return q["gamma"], q["packed"]

        return self._pcache.get([w], build)

    def block_matrix(self, dtype: torch.dtype) -> torch.Tensor:
        return _prepared(self._wcache, self.weight, lambda: self.ternary_state()[1], self.in_o, self.out_o, dtype)

    def _tracked(self, x):
        return torch.is_grad_enabled() and (x.requires_grad or self.weight.requires_grad or self.beta.requires_grad)

    def forward(self, x_parts):
        y = self.forward_full(_parts_to_rows(x_parts, self.in_o))
        return tuple(y.split(self.out_o, dim=-1))


class OctonionFusedLinear(_OctonionTernaryBase):
    """Octonion ternary linear, the reference's GPU module
    (cayley_dickson_cuda.py:622-668): 8 parts [..., in_o] in, 8 parts
    [..., out_o] out.  As there, the input is rounded to bf16, the product
    accumulates in float32 and is rounded to bf16 (the fused kernel's output,
    :402, :411, :421), and the module multiplies it by the float32 beta
    (:668), so the result is float32 whatever the input dtype or autocast."""

    def forward_full(self, x: torch.Tensor) -> torch.Tensor:
        """Rows x [..., 8*in_o] (parts side by side) -> float32 [..., 8*out_o]."""
        xb = x if x.dtype == torch.bfloat16 else x.to(torch.bfloat16)
        if self._tracked(x):
            return OctonionLinearFunction.apply(xb, self.weight, self.beta, self, True)
        return kernels.octonion_fused_linear(xb, self.in_o, self.out_o, self.block_matrix(torch.bfloat16),
                                             self.beta)


class OctonionTernaryLinearRef(_OctonionTernaryBase):
    """physics.py:53-82, the reference's CPU module: the same parameters and
    math, computed in the activation dtype (float32 matrix cores for float32
    inputs, bf16 operands with float32 accumulation under bf16 autocast or
    for bf16 inputs).  The result has the dtype of y * beta in the
    reference: the input dtype promoted with beta's (float32)."""

    def forward_full(self, x: torch.Tensor) -> torch.Tensor:
        out_dt = torch.promote_types(x.dtype, self.beta.dtype)
        dt = act_dtype(x)
        x = x if x.dtype == dt else x.to(dt)
        if self._tracked(x):
            y = OctonionLinearFunction.apply(x, self.weight, self.beta, self, False)
        else:
            y = kernels.octonion_linear(x, self.in_o, self.out_o, self.block_matrix(dt), self.beta)
        return y if y.dtype == out_dt else y.to(out_dt)


OctonionTernaryLinear = OctonionFusedLinear


class OctonionPackedLinear(nn.Module):
    """Inference layer holding 2-bit packed codes (cayley_dickson_cuda.py:702-772):
    buffer ``weight_packed`` [8, out_o, in_o//4] uint8 and parameter ``beta``.
    Its forward is OctonionFusedLinear's (float32 = bf16 product times beta,
    :761-765)."""

    def __init__(self, in_features, out_features, bias=False):
        super().__init__()
        assert in_features % 8 == 0 and out_features % 8 == 0
        assert in_features % 32 == 0, "in_features must be divisible by 32 for packing"
        self.in_o = in_features // 8
        self.out_o = out_features // 8
        self.register_buffer('weight_packed', torch.zeros(8, self.out_o, self.in_o // 4, dtype=torch.uint8))
        self.beta = nn.Parameter(torch.ones(self.out_o) * math.sqrt(3.0 / (2.0 * self.in_o)))
        self._wcache = WeightCache()

    @classmethod
    def from_unpacked(cls, layer: OctonionFusedLinear) -> 'OctonionPackedLinear':
        packed = cls(layer.in_o * 8, layer.out_o * 8).to(layer.weight.device)
        packed.weight_packed.copy_(layer.ternary_state()[1])
        packed.beta.data = layer.beta.data.clone()
        return packed

    def forward_full(self, x):
        B = _prepared(self._wcache, self.weight_packed, lambda: self.weight_packed, self.in_o, self.out_o,
                      torch.bfloat16)
        return kernels.octonion_fused_linear(x, self.in_o, self.out_o, B, self.beta)

    def forward(self, x_parts):
        y = self.forward_full(_parts_to_rows(x_parts, self.in_o))
        return tuple(y.split(self.out_o, dim=-1))

    def clear_cache(self):
        self._wcache.clear()


def optimize_for_inference(model):
    """Swap every OctonionFusedLinear for an OctonionPackedLinear holding its
    2-bit codes (cayley_dickson_cuda.py:778-818 converts to the fused layer;
    here the fused layer already is the default, so the useful conversion is
    to packed storage)."""
    def replace(module):
        for name, child in module.named_children():
            if type(child) is OctonionFusedLinear:
                setattr(module, name, OctonionPackedLinear.from_unpacked(child))
            else:
                replace(child)
    replace(model)
    return model


class OctonionHeadMixerFused(nn.Module):
    """Octonion head mixer (cayley_dickson_cuda.py:1011-1043; math of
    chassis.py:375-399): y_i = beta * sum_j S[i][j] heads_j @ W[i^j].  Runs as
    one PyTorch matmul against the dense block matrix (outside the hot path
    of this build)."""

    SIGNS = SIGN_TABLE
    WIDX = WEIGHT_IDX

    def __init__(self, head_dim):
        super().__init__()
        self.head_dim = head_dim
        self.W = nn.Parameter(torch.randn(8, head_dim, head_dim) * 0.02)
        self.beta = nn.Parameter(torch.ones(head_dim) * math.sqrt(3.0 / (2.0 * head_dim)))
        self.register_buffer('signs', torch.tensor(SIGN_TABLE, dtype=torch.float32))
        self.register_buffer('widx', torch.tensor(WEIGHT_IDX, dtype=torch.long))

    def forward(self, x):
        B, H, T, D = x.shape
        assert H == 8, f"OctonionHeadMixer requires exactly 8 heads, got {H}"
        dt = x.dtype
        # dense [8D (j, d), 8D (i, e)] = S[i][j] W[i^j][d][e]
        Wd = self.W.to(dt)[self.widx]                     # [i, j, D, D]
        blocks = Wd * self.signs.to(dt)[:, :, None, None]
        dense = blocks.permute(1, 2, 0, 3).reshape(8 * D, 8 * D).contiguous()
        xr = x.permute(0, 2, 1, 3).reshape(B * T, 8 * D).contiguous()
        y = torch.matmul(xr, dense).view(B, T, 8, D).permute(0, 2, 1, 3)
        return y * self.beta.to(dt)
