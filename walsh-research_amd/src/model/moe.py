"""Hadamard mixture-of-experts FFN (module surface of src/model/moe.py).

``HadamardMoE`` keeps the reference's constructor, submodules and parameter
names (``router.gate.{0,2}.weight``, ``experts.{gate,up,down}_weights``) and
its side state (``_aux_loss``, ``_last_expert_mask``, ``_expert_counts``,
``_total_tokens``), but computes only the selected (token, expert) pairs
instead of a dense einsum over all experts (moe.py:363-374):

  * bf16 at n_embd 512 (16 experts): one launch, walsh_moe_ffn_fwd (router,
    routing and experts fused, the input tile read once into LDS);
  * otherwise three launches:
      1. walsh_moe_route_fwd   router MLP + softmax + top-k + weights +
                               per-expert counts, zero-filling the blocks of
                               unselected experts (for a wide router: torch
                               GEMMs for the two Linears + walsh_moe_topk_fwd);
      2. walsh_moe_scatter     per-expert pair lists;
      3. walsh_moe_experts_fwd ternary SwiGLU on the routed pairs, weighted
                               by the routing weight.

Routing semantics are the reference's: top-k with k = min(max_experts, E)
for every token (moe.py:434-436); ``threshold`` and ``min_experts`` are
stored and unused, as there.  Equal probabilities select the lower expert
index first.
"""
import types
from typing import Optional, Tuple

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F

from . import kernels
from ._common import WeightCache, act_dtype, tracked_dtype

# A fused router keeps W1 in each wavefront's working set; beyond this width
# the two Linears run as library GEMMs (plain dense products) instead.
_FUSED_ROUTER_MAX_C = 1024
_FUSED_ROUTER_MAX_E = 64


class TernaryAbsmeanSTE(torch.autograd.Function):
    """Absmean ternary quantiser of the MoE experts (moe.py:268-294): returns
    clamp(round(W / gamma), -1, 1) * gamma, gamma = mean(|W|) + 1e-8 over the
    whole tensor; backward passes the gradient clipped to [-2, 2]."""

    @staticmethod
    def forward(ctx, w_latent):
        q = kernels.ternary_quantize(w_latent, packed=False, scaled=True)
        return q["scaled"].to(w_latent.dtype)

    @staticmethod
    def backward(ctx, grad_output):
        return kernels.ternary_ste_bwd(grad_output, mode=1).to(grad_output.dtype)


def quantize_ternary(w: torch.Tensor) -> torch.Tensor:
    """W_ternary = clip(round(W / gamma), -1, 1) * gamma (moe.py:297-303)."""
    return TernaryAbsmeanSTE.apply(w)


def _output_dtype(x: torch.Tensor, weights_dtype: torch.dtype = torch.float32) -> torch.dtype:
    """dtype of ``expert_out * routing_weight`` in the reference: the routing
    weights come out of a float32 softmax under autocast, so the product is
    float32 there; without autocast it is the promotion of the two dtypes."""
    return torch.promote_types(act_dtype(x), weights_dtype)


class FastMoEExperts(nn.Module):
    """Ternary SwiGLU experts on 32-wide blocks (moe.py:306-380).

    gate_weights / up_weights [E, H, dim] and down_weights [E, dim, H]
    (H = dim * expansion) are float32 latents initialised U(-1, 1) in that
    order; the forward uses their gamma-scaled ternary codes."""

    def __init__(self, n_experts: int = 8, dim: int = 32, expansion: int = 4, use_ternary: bool = True):
        super().__init__()
        self.n_experts = n_experts
        self.dim = dim
        self.hidden = dim * expansion
        self.use_ternary = use_ternary
        self.gate_weights = nn.Parameter(torch.empty(n_experts, self.hidden, dim))
        self.up_weights = nn.Parameter(torch.empty(n_experts, self.hidden, dim))
        self.down_weights = nn.Parameter(torch.empty(n_experts, dim, self.hidden))
        nn.init.uniform_(self.gate_weights, -1, 1)
        nn.init.uniform_(self.up_weights, -1, 1)
        nn.init.uniform_(self.down_weights, -1, 1)
        self._q = WeightCache()
        self._prep = WeightCache()

    def _check(self):
        if not self.use_ternary:
            raise NotImplementedError("FastMoEExperts(use_ternary=False) is outside this build's scope")
        if self.dim != 32 or self.hidden not in (64, 128, 256):
            raise NotImplementedError(f"experts need dim 32 and expansion 2, 4 or 8 (dim={self.dim}, "
                                      f"hidden={self.hidden})")

    def quantized(self):
        """(gammas float32 [3], packed codes (gate, up, down)) of the three
        weight tensors (2-bit pack_ternary_weights layout)."""
        self._check()
        ws = (self.gate_weights, self.up_weights, self.down_weights)

        def build():
            qs = [kernels.ternary_quantize(w, packed=True) for w in ws]
            return torch.cat([q["gamma"] for q in qs]), tuple(q["packed"] for q in qs)

        return self._q.get(ws, build)

    @staticmethod
    def operand_gammas(gammas: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
        """Under bf16 autocast the einsum operand code * gamma is a bf16
        tensor, i.e. code * bf16(gamma)."""
        return gammas.to(torch.bfloat16).float() if dtype == torch.bfloat16 else gammas

    def ternary_state(self, dtype: torch.dtype):
        """(operand gammas [3], fragments for walsh_moe_experts_fwd)."""
        ws = (self.gate_weights, self.up_weights, self.down_weights)

        def build():
            g, packed = self.quantized()
            return self.operand_gammas(g, dtype), kernels.moe_expert_fragments(*packed)

        return self._prep.get(ws, build, extra=(dtype,))

    def routed(self, x2d: torch.Tensor, route: "kernels.MoERoute", y2d: torch.Tensor) -> None:
        """Write w * expert_e(x_e) into y2d for every routed (token, e)."""
        gammas, frags = self.ternary_state(x2d.dtype)
        lists = kernels.moe_scatter(route)
        kernels.moe_experts(x2d, y2d, route, lists, frags, gammas, self.hidden)

    def forward_autograd(self, x: torch.Tensor, expert_weights: torch.Tensor, mask: torch.Tensor = None,
                         k: int = None) -> torch.Tensor:
        """The experts as differentiable products for training (moe.py:337-380),
        float32 result.  Given the routing selection (``mask`` [B, T, E] with
        ``k`` ones per token) on the GPU with hidden size <= 128: forward and
        backward on the HIP kernels over the routed pairs only (the others have
        weight zero and add nothing; their routing-weight gradient is returned
        as zero, which the routing's mask multiplies away).  Otherwise
        quantize_ternary (straight-through gradient clipped to [-2, 2]) and
        per-expert matrix products in float32 (see tracked_dtype), times the
        routing weights."""
        self._check()
        B, T, E, D = x.shape
        if mask is not None and k is not None and x.is_cuda and self.hidden <= 128:
            return _RoutedExperts.apply(x, expert_weights, mask, k, self.gate_weights, self.up_weights,
                                        self.down_weights, self)
        gw, uw, dw = (quantize_ternary(w) for w in (self.gate_weights, self.up_weights, self.down_weights))
        dt = tracked_dtype(act_dtype(x))
        dev = x.device.type
        with torch.autocast(dev, dtype=torch.get_autocast_dtype(dev), enabled=False):
            xe = x.to(dt).reshape(B * T, E, D).transpose(0, 1).contiguous()            # [E, M, D]
            g = torch.matmul(xe, gw.to(dt).transpose(1, 2).contiguous())               # [E, M, H]
            u = torch.matmul(xe, uw.to(dt).transpose(1, 2).contiguous())
            o = torch.matmul(F.silu(g) * u, dw.to(dt).transpose(1, 2).contiguous())     # [E, M, D]
            out = o.transpose(0, 1).reshape(B, T, E, D) * expert_weights.to(dt).unsqueeze(-1)
        return out

    def forward(self, x: torch.Tensor, expert_weights: torch.Tensor) -> torch.Tensor:
        """x [B, T, E, dim], expert_weights [B, T, E] -> [B, T, E, dim]: every
        expert on its block, times its weight (moe.py:337-380)."""
        B, T, E, D = x.shape
        assert E == self.n_experts and D == self.dim, f"expert input shape {tuple(x.shape)}"
        assert tuple(expert_weights.shape) == (B, T, E), "expert_weights shape"
        if torch.is_grad_enabled() and (x.requires_grad or expert_weights.requires_grad
                                        or any(p.requires_grad for p in self.parameters())):
            return self.forward_autograd(x, expert_weights)
        dt = act_dtype(x)
        M = B * T
        x2d = x.to(dt).reshape(M, E * D)
        y = torch.empty(M, E * D, device=x.device, dtype=_output_dtype(x, expert_weights.dtype))
        if M:
            # every (token, expert) pair, weighted by the given weights
            r = kernels.MoERoute(M, E, E, x.device, dense=False, parts=1)
            r.topk_idx.copy_(torch.arange(E, device=x.device, dtype=torch.int32).expand(M, E))
            r.topk_w.copy_(expert_weights.reshape(M, E))
            r.count_part.fill_(M)
            r.probsum_part.zero_()
            self.routed(x2d, r, y)
        return y.view(B, T, E, D)


class _RoutedExperts(torch.autograd.Function):
    """FastMoEExperts on the routed pairs, forward and backward on HIP
    (walsh_moe_experts_fwd / walsh_moe_experts_bwd), float32 arithmetic.
    Inputs: x [B, T, E, 32], expert_weights [B, T, E], mask [B, T, E] (k
    ones per token), k, the three latent weight tensors and the module.

    A token's k experts are taken in ascending expert order (a stable sort
    of its mask row), so a recomputed forward (activation checkpointing)
    lists the pairs exactly as the first one did.  Everything the backward
    reads (inputs, pair order and weights, the per-expert pair lists) goes
    through save_for_backward: under non-reentrant checkpointing those are
    the recomputation's tensors, consistent with each other, and nothing
    outlives the forward outside the saved set."""

    @staticmethod
    def forward(ctx, x, expert_weights, mask, k, gate_w, up_w, down_w, mod):
        B, T, E, D = x.shape
        M = B * T
        dev = x.device
        m2 = mask.detach().reshape(M, E)
        idx = torch.sort(m2, dim=-1, descending=True, stable=True).indices[:, :k]
        w = expert_weights.detach().reshape(M, E).float().gather(-1, idx).contiguous()
        r = kernels.MoERoute(M, E, k, dev, dense=False, parts=1)
        r.topk_idx.copy_(idx)
        r.topk_w.copy_(w)
        r.count_part.copy_(m2.sum(0).to(torch.int32).view(1, E))
        r.probsum_part.zero_()
        lists = kernels.moe_scatter(r)
        gammas, packed = mod.quantized()
        frags = kernels.moe_expert_fragments(*packed)
        x2d = x.detach().reshape(M, E * D).float().contiguous()
        y = torch.zeros(M, E * D, device=dev, dtype=torch.float32)
        if M:
            kernels.moe_experts(x2d, y, r, lists, frags, gammas, mod.hidden)
        ctx.save_for_backward(x2d, idx, r.topk_w, *lists, gammas, *packed)
        ctx.shape, ctx.k, ctx.H, ctx.x_dtype = (B, T, E, D), k, mod.hidden, x.dtype
        return y.view(B, T, E, D)

    @staticmethod
    def backward(ctx, gy):
        x2d, idx, topk_w, lst, offset, toff, gammas, pg, pu, pd = ctx.saved_tensors
        B, T, E, D = ctx.shape
        M = B * T
        need_x, need_w_route = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        need_w = any(ctx.needs_input_grad[4:7])
        route = types.SimpleNamespace(M=M, E=E, k=ctx.k, topk_w=topk_w)
        gy2d = gy.reshape(M, E * D).float().contiguous()
        dx, dpair, grads = kernels.moe_experts_bwd(x2d, gy2d, route, (lst, offset, toff), (pg, pu, pd), gammas,
                                                   ctx.H, need_w=need_w)
        d_ew = None
        if need_w_route:
            # dpair[t, j] belongs to expert idx[t, j]: the same saved order the pair lists were built from
            d_ew = torch.zeros(M, E, device=gy.device, dtype=torch.float32).scatter_(1, idx, dpair).view(B, T, E)
        gx = dx.view(B, T, E, D).to(ctx.x_dtype) if need_x else None
        gg, gu, gd = grads if grads is not None else (None, None, None)
        return gx, d_ew, None, None, gg, gu, gd, None


class HadamardRouter(nn.Module):
    """Router MLP Linear(C, C/4) -> SiLU -> Linear(C/4, E), no biases,
    weights N(0, 0.01) (moe.py:383-416); forward is moe.py:418-447."""

    def __init__(self, n_embd: int, n_experts: int = 8, threshold: float = 0.1, min_experts: int = 1,
                 max_experts: int = 4):
        super().__init__()
        self.n_experts = n_experts
        self.threshold = threshold
        self.min_experts = min_experts
        self.max_experts = max_experts
        hidden = n_embd // 4
        self.gate = nn.Sequential(
            nn.Linear(n_embd, hidden, bias=False),
            nn.SiLU(),
            nn.Linear(hidden, n_experts, bias=False),
        )
        for m in self.gate:
            if isinstance(m, nn.Linear):
                nn.init.normal_(m.weight, std=0.01)
        self._frag = WeightCache()

    @property
    def top_k(self) -> int:
        return min(self.max_experts, self.n_experts)

    def _fused(self, C: int) -> bool:
        return C <= _FUSED_ROUTER_MAX_C and self.n_experts <= _FUSED_ROUTER_MAX_E and C % 64 == 0

    def route(self, x2d: torch.Tensor, dense: bool = False, y2d: torch.Tensor = None) -> "kernels.MoERoute":
        """Routing of x2d [M, C] (activation dtype); see kernels.moe_route."""
        w1, w2 = self.gate[0].weight, self.gate[2].weight
        C = x2d.shape[-1]
        if self._fused(C):
            f1, f2 = self._frag.get((w1, w2), lambda: kernels.moe_router_fragments(w1, w2, x2d.dtype),
                                    extra=(x2d.dtype,))
            return kernels.moe_route(x2d, f1, f2, w1.shape[0], self.n_experts, self.top_k, dense=dense, y=y2d)
        # wide router: weights cast to the activation dtype once per weight
        # version; in bf16 both products, SiLU and the routing run on the
        # matrix-core router, in float32 the Linears are library GEMMs
        w1c, w2c = self._frag.get((w1, w2), lambda: (w1.detach().to(x2d.dtype).contiguous(),
                                                     w2.detach().to(x2d.dtype).contiguous()),
                                  extra=(x2d.dtype, "gemm"))
        if kernels.moe_router_wide_supported(x2d, w1.shape[0], self.n_experts, self.top_k):
            return kernels.moe_router_wide(x2d, w1c, w2c, self.n_experts, self.top_k, dense=dense, y=y2d)
        logits = F.linear(F.silu(F.linear(x2d, w1c)), w2c)
        r = kernels.moe_topk(logits, self.top_k, dense=dense)
        if y2d is not None:
            _zero_unselected(y2d, r)
        return r

    def route_autograd(self, x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """moe.py:418-447 as differentiable operations (training): the router
        MLP, softmax, top-k mask and the renormalised weights; the gradient
        reaches the router through the probabilities of the selected experts."""
        logits = self.gate(x)
        probs = F.softmax(logits, dim=-1)
        _, idx = probs.topk(self.top_k, dim=-1)
        mask = torch.zeros_like(probs).scatter_(-1, idx, 1.0)
        mp = probs * mask
        return mp / mp.sum(dim=-1, keepdim=True).clamp(min=1e-8), mask, probs

    def forward(self, x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """x [B, T, C] -> (expert_weights, expert_mask, router_probs), each
        [B, T, E] float32."""
        B, T, C = x.shape
        if torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters())):
            return self.route_autograd(x)
        dt = act_dtype(x)
        r = self.route(x.to(dt).reshape(B * T, C), dense=True)
        E = self.n_experts
        return r.weights.view(B, T, E), r.mask.view(B, T, E), r.probs.view(B, T, E)


def _zero_unselected(y2d: torch.Tensor, r: "kernels.MoERoute") -> None:
    """Zero the output blocks of unselected experts when the router ran as
    GEMMs + walsh_moe_topk_fwd (the fused router does this itself)."""
    keep = torch.zeros(r.M, r.E, device=y2d.device, dtype=torch.bool)
    keep.scatter_(1, r.topk_idx.long(), True)
    y2d.view(r.M, r.E, 32).masked_fill_(~keep.unsqueeze(-1), 0)


class HadamardMoE(nn.Module):
    """Sparse FFN over the 32-wide Hadamard blocks (moe.py:450-598)."""
    BLOCK_DIM = 32

    def __init__(self, config, n_experts: int = None, expansion: int = 4, threshold: float = 0.1,
                 min_experts: int = 1, max_experts: int = 4, aux_loss_weight: float = 0.01):
        super().__init__()
        self.n_embd = config.n_embd
        if n_experts is None:
            n_experts = config.n_embd // self.BLOCK_DIM
        self.n_experts = n_experts
        self.block_dim = config.n_embd // n_experts
        self.aux_loss_weight = aux_loss_weight
        assert config.n_embd % n_experts == 0, \
            f"n_embd ({config.n_embd}) must be divisible by n_experts ({n_experts})"
        assert self.block_dim == self.BLOCK_DIM, \
            f"block_dim ({self.block_dim}) should be {self.BLOCK_DIM} for Hadamard structure"
        self.router = HadamardRouter(n_embd=config.n_embd, n_experts=n_experts, threshold=threshold,
                                     min_experts=min_experts, max_experts=max_experts)
        self.experts = FastMoEExperts(n_experts=n_experts, dim=self.block_dim, expansion=expansion)
        self.register_buffer('_expert_counts', torch.zeros(n_experts), persistent=False)
        self.register_buffer('_total_tokens', torch.zeros(1), persistent=False)
        self._ffn = WeightCache()   # single-launch operand layouts
        self._route = None          # routing of the last forward (device tensors)
        self._route_shape = None
        self._aux_value = None
        self._mask_value = None

    # Side state of the last forward, materialised on first access: the
    # balance loss E * sum_e mean(mask_e) * mean(p_e) (moe.py:544-560) from
    # the per-expert counts and probability sums, and the dense selection mask.
    @property
    def _aux_loss(self):
        if self._aux_value is None and self._route is not None:
            r = self._route
            self._aux_value = (r.count.float() / r.M * (r.probsum / r.M)).sum() * self.n_experts
        return self._aux_value

    @_aux_loss.setter
    def _aux_loss(self, v):
        self._aux_value = v

    @property
    def _last_expert_mask(self):
        if self._mask_value is None and self._route is not None:
            r = self._route
            m = torch.zeros(r.M, r.E, device=r.topk_idx.device, dtype=torch.float32)
            m.scatter_(1, r.topk_idx.long(), 1.0)
            self._mask_value = m.view(*self._route_shape, r.E)
        return self._mask_value

    @_last_expert_mask.setter
    def _last_expert_mask(self, v):
        self._mask_value = v

    def forward(self, x: torch.Tensor, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        """x [B, T, C] -> [B, T, C].  The result dtype is the reference's
        (float32 under autocast, where the routing weights are float32);
        ``out_dtype`` overrides it for callers that round the result anyway."""
        B, T, C = x.shape
        assert C == self.n_embd, f"expected n_embd {self.n_embd}, got {C}"
        if torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters())):
            return self._forward_autograd(x, out_dtype)
        dt = act_dtype(x)
        M = B * T
        x2d = x.to(dt).reshape(M, C)
        ydt = _output_dtype(x) if out_dtype is None else out_dtype
        if dt == torch.float32:
            ydt = torch.float32
        y = torch.empty(M, C, device=x.device, dtype=ydt)
        ex = self.experts
        if kernels.moe_ffn_supported(x2d, self.n_experts, ex.hidden, self.router.top_k) and self.use_fused:
            # router, routing and experts in one launch
            g, frags = self._ffn_state()
            r = kernels.moe_ffn(x2d, y, frags, g, self.n_experts, self.router.top_k, ex.hidden)
        else:
            r = self._decode(x2d, y) if self.use_fused else None
            if r is None:
                r = self.router.route(x2d, y2d=y)
                if M:
                    ex.routed(x2d, r, y)
        self._route, self._route_shape = r, (B, T)
        self._aux_value = self._mask_value = None
        if self.training:
            with torch.no_grad():
                self._expert_counts += r.count.float()
                self._total_tokens += M
        return y.view(B, T, C)

    use_fused = True   # single-launch kernels where supported (tests switch it off to compare paths)

    def _decode(self, x2d: torch.Tensor, y: torch.Tensor) -> Optional["kernels.MoERoute"]:
        """A few tokens of a wide bf16 model (decode): router, routing and the
        routed experts in one launch (walsh_moe_decode_fwd); None where that
        kernel does not apply."""
        rt, ex = self.router, self.experts
        w1, w2 = rt.gate[0].weight, rt.gate[2].weight
        if not kernels.moe_decode_supported(x2d, w1.shape[0], self.n_experts, rt.top_k, ex.hidden, y):
            return None
        w1c, w2c = rt._frag.get((w1, w2), lambda: (w1.detach().to(x2d.dtype).contiguous(),
                                                   w2.detach().to(x2d.dtype).contiguous()),
                                extra=(x2d.dtype, "gemm"))
        gammas, frags = ex.ternary_state(x2d.dtype)
        sync = self._decode_sync
        if sync is None or sync.device != x2d.device:
            # the kernel's completion counter: zero once, left at zero by every call
            sync = self._decode_sync = torch.zeros(1, device=x2d.device, dtype=torch.int32)
        return kernels.moe_decode(x2d, y, w1c, w2c, self.n_experts, rt.top_k, frags, gammas, ex.hidden, sync)

    _decode_sync = None

    def _forward_autograd(self, x: torch.Tensor, out_dtype: Optional[torch.dtype]) -> torch.Tensor:
        """Training form (moe.py:512-542): differentiable routing, the
        balance loss kept as a differentiable tensor, and every expert on its
        block (FastMoEExperts.forward_autograd)."""
        B, T, C = x.shape
        E = self.n_experts
        dt = act_dtype(x)
        xr = x.to(dt)
        weights, mask, probs = self.router.route_autograd(xr)
        self._route, self._route_shape = None, (B, T)
        self._aux_value = (mask.reshape(-1, E).mean(0) * probs.reshape(-1, E).mean(0)).sum() * E
        self._mask_value = mask.detach()
        if self.training:
            with torch.no_grad():
                self._expert_counts += mask.reshape(-1, E).sum(0)
                self._total_tokens += B * T
        out = self.experts.forward_autograd(xr.reshape(B, T, E, self.block_dim), weights, mask=mask.detach(),
                                            k=self.router.top_k).reshape(B, T, C)
        ydt = _output_dtype(x) if out_dtype is None else out_dtype
        return out.to(torch.float32 if dt == torch.float32 else ydt)

    def _ffn_state(self):
        ex, w1, w2 = self.experts, self.router.gate[0].weight, self.router.gate[2].weight
        ws = (w1, w2, ex.gate_weights, ex.up_weights, ex.down_weights)

        def build():
            g, packed = ex.quantized()
            return (ex.operand_gammas(g, torch.bfloat16), kernels.moe_ffn_fragments(w1, w2, *packed))

        return self._ffn.get(ws, build)

    def get_aux_loss(self) -> Optional[torch.Tensor]:
        a = self._aux_loss
        return a if a is not None else torch.tensor(0.0)

    def get_expert_stats(self) -> dict:
        """Expert load, mean experts per token and 1 - |Gini| of the load
        (moe.py:566-589)."""
        total = self._total_tokens.item()
        if total == 0:
            return {'expert_load': [0.0] * self.n_experts, 'avg_experts': 0.0, 'load_balance': 0.0}
        load = self._expert_counts.cpu().numpy() / total
        s = np.sort(load)
        n = len(s)
        csum = np.cumsum(s)
        gini = (2 * np.sum(np.arange(1, n + 1) * s) - (n + 1) * csum[-1]) / (n * csum[-1] + 1e-8)
        return {'expert_load': load.tolist(), 'avg_experts': float(load.sum()),
                'load_balance': float(1 - abs(gini))}

    def reset_stats(self):
        self._expert_counts.zero_()
        self._total_tokens.zero_()

    def get_expert_usage(self) -> dict:
        return self.get_expert_stats()


def should_use_moe(config) -> bool:
    return getattr(config, 'use_moe', False)


def should_use_channel_mod(config) -> bool:
    return getattr(config, 'use_channel_mod', False)


class ChannelModFunction(torch.autograd.Function):
    """Per-block modulation out = x + r*(x*scale + shift_scale*shift - x)
    with its backward (moe.py:202-256), both on HIP kernels
    (walsh_chanmod_apply / walsh_chanmod_bwd)."""

    @staticmethod
    def forward(ctx, x, scale, shift, n_blocks, block_dim, residual_scale, shift_scale):
        if x.dim() != 3:
            raise ValueError(f"Expected 3D input, got {x.shape}")
        assert scale.shape[-1] == n_blocks and n_blocks * block_dim == x.shape[-1], "block layout"
        y = kernels.chanmod_apply(x, scale, shift, residual_scale, shift_scale)
        ctx.save_for_backward(x, scale)
        ctx.residual_scale = residual_scale
        ctx.shift_scale = shift_scale
        ctx.shift_dtype = shift.dtype
        return y

    @staticmethod
    def backward(ctx, grad_out):
        x, scale = ctx.saved_tensors
        gx, ds, dh = kernels.chanmod_bwd(grad_out, x, scale, ctx.residual_scale, ctx.shift_scale)
        return gx, ds.to(scale.dtype), dh.to(ctx.shift_dtype), None, None, None, None


class HadamardChannelModulation(nn.Module):
    """Bulk-state channel modulation (moe.py:610-771): per group (batch row)
    the mean over T of the input drives a two-layer MLP whose outputs give a
    scale in [1 - t, 1 + t] (t = clamp(scale_temp, 0.1, 0.5)) and a shift for
    each block of C / n_blocks channels:
        out = x + residual_scale * (x * scale + 0.1 * shift - x).
    Parameter names are the reference's (``context_mlp.{0,2}.weight``,
    ``scale_temp``).

    Inference runs walsh_chanmod_fwd: a column-sum kernel for the bulk state,
    the MLP kernel and the apply kernel (the input is read twice and the
    output written once).  ``fused_residual(x, norm)`` computes
    x + self(norm(x)) in the same three kernels with the RMSNorm folded into
    both passes over x.  With autograd on, the MLP runs as float32 torch
    operations (the ternary weights through TernaryAbsmeanSTE) and the
    modulation through ChannelModFunction.

    The MLP runs in float32 also under bfloat16 autocast, where the
    reference's F.linear rounds its inputs to bfloat16 (moe.py:753-762)."""

    BLOCK_DIM = 32

    def __init__(self, n_embd: int = 256, n_blocks: int = None, use_ternary: bool = True,
                 residual_scale: float = 0.5):
        super().__init__()
        if n_blocks is None:
            n_blocks = n_embd // self.BLOCK_DIM
        self.n_blocks = n_blocks
        self.block_dim = n_embd // n_blocks
        self.residual_scale = residual_scale
        self.use_ternary = use_ternary
        hidden = n_embd // 4
        self.context_mlp = nn.Sequential(
            nn.Linear(n_embd, hidden, bias=False),
            nn.SiLU(),
            nn.Linear(hidden, n_blocks * 2, bias=False),
        )
        nn.init.normal_(self.context_mlp[0].weight, std=0.02)
        nn.init.normal_(self.context_mlp[-1].weight, std=0.01)
        self.scale_temp = nn.Parameter(torch.ones(1) * 1.0)
        self._wcache = WeightCache()
        self._last_ss = None   # float32 [G, 2*n_blocks]: scale then shift of the last forward

    # statistics of the last forward (moe.py:711-715), computed when read
    def _stat(self, which):
        ss = self._last_ss
        if ss is None:
            return 0.0
        nb = self.n_blocks
        if which == 'scale_mean':
            return ss[:, :nb].mean().item()
        if which == 'scale_std':
            return ss[:, :nb].std().item()
        return ss[:, nb:].abs().mean().item()

    @property
    def _last_scale_mean(self):
        return self._stat('scale_mean')

    @property
    def _last_scale_std(self):
        return self._stat('scale_std')

    @property
    def _last_shift_mean(self):
        return self._stat('shift_mean')

    def get_modulation_stats(self) -> dict:
        return {
            'scale_mean': self._last_scale_mean,
            'scale_std': self._last_scale_std,
            'shift_mean': self._last_shift_mean,
            'scale_temp': self.scale_temp.item(),
        }

    def _tracked(self, x) -> bool:
        return torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters()))

    def _mlp_weights(self):
        """(w1, w2) float32 as the MLP uses them: code * gamma (moe.py:288)
        for the ternary module, the weights themselves otherwise."""
        l1, l2 = self.context_mlp[0].weight, self.context_mlp[2].weight

        def build():
            if not self.use_ternary:
                return l1.detach().float().contiguous(), l2.detach().float().contiguous()
            return (kernels.ternary_quantize(l1, packed=False, scaled=True)["scaled"],
                    kernels.ternary_quantize(l2, packed=False, scaled=True)["scaled"])
        return self._wcache.get((l1, l2), build, extra=(self.use_ternary,))

    def _forward_autograd(self, x):
        with torch.autocast("cuda", enabled=False):
            h = x.float().mean(dim=1)
            for layer in self.context_mlp:
                if isinstance(layer, nn.Linear):
                    w = quantize_ternary(layer.weight) if self.use_ternary else layer.weight
                    h = F.linear(h, w.float())
                else:
                    h = layer(h)
            raw_scale, shift = h.chunk(2, dim=-1)
            scale = 1.0 + torch.clamp(self.scale_temp, 0.1, 0.5) * torch.tanh(raw_scale)
        self._last_ss = torch.cat([scale, shift], -1).detach()
        return ChannelModFunction.apply(x, scale, shift.contiguous(), self.n_blocks, self.block_dim,
                                        self.residual_scale, 0.1)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """x [B, T, n_embd] -> modulated x, same shape and dtype."""
        if self._tracked(x):
            return self._forward_autograd(x)
        w1, w2 = self._mlp_weights()
        y, self._last_ss = kernels.chanmod_fwd(x, w1, w2, self.scale_temp, self.n_blocks, self.residual_scale, 0.1)
        return y

    def fused_residual(self, x: torch.Tensor, norm) -> torch.Tensor:
        """x + self(norm(x)) for an RMSNorm module ``norm`` (mhc.py:531,
        moe.py:796-798), in x's dtype."""
        if self._tracked(x):
            return (x + self(norm(x))).to(x.dtype)
        w1, w2 = self._mlp_weights()
        y, self._last_ss = kernels.chanmod_fwd(x, w1, w2, self.scale_temp, self.n_blocks, self.residual_scale, 0.1,
                                               norm_w=norm.weight, eps=norm.eps, add_input=True)
        return y


class HadamardChannelModulationBlock(nn.Module):
    """x + channel_mod(norm(x)) (moe.py:774-798): n_blocks 8 and residual
    scale 0.1 by default, as there."""

    def __init__(self, config, n_blocks: int = 8):
        super().__init__()
        from .chassis import RMSNorm
        self.norm = RMSNorm(config.n_embd)
        self.channel_mod = HadamardChannelModulation(
            n_embd=config.n_embd,
            n_blocks=n_blocks,
            use_ternary=getattr(config, 'use_ternary', True),
            residual_scale=0.1,
        )

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.channel_mod.fused_residual(x, self.norm)
