"""Walsh configuration, layer factories and the transformer harness around
the hot path (module surface of src/model/chassis.py).

The hot-path layers (Hadamard / octonion ternary linears, Hadamard MoE) run
on HIP kernels; attention (SDPA), RoPE, RMSNorm, embeddings and the head
mixers stay PyTorch operations on the GPU.  Class names, constructor
signatures, parameter names, shapes and the order in which parameters are
created (hence the RNG stream consumed by seeded initialisation) follow the
reference.
"""
import math
from dataclasses import dataclass
from typing import List, Optional, Tuple

import torch
import torch.utils.checkpoint
import torch.nn as nn
from torch.nn import functional as F

from .hadamard import HadamardLinear, HadamardTernaryLinear, HadamardTernaryLinearTuple  # noqa: F401
from .hadamard import HadamardLinearFunction
from .hadamard import HadamardHeadMixer, HadamardHeadMixerFused
from .octonion import OctonionHeadMixerFused, OctonionTernaryLinear
from . import kernels
from ._common import WeightCache, act_dtype, cached_linear

_HADAMARD_AVAILABLE = True
_HADAMARD_HEAD_MIXER_AVAILABLE = True


@dataclass
class WalshConfig:
    """chassis.py:33-51 (fields and defaults unchanged)."""
    block_size: int = 256
    vocab_size: int = 65
    n_layer: int = 6
    n_head: int = 6
    n_embd: int = 768
    dropout: float = 0.0
    bias: bool = False
    head_mixing: bool = False
    algebra: str = "octonion"
    hash_embeddings: bool = False
    use_moe: bool = False
    moe_threshold: float = 0.1
    moe_min_experts: int = 1
    moe_max_experts: int = 4
    use_channel_mod: bool = False


def get_linear_layer(config: WalshConfig):
    """(LayerClass, algebra_dim) for the configured algebra (chassis.py:54-65)."""
    if config.algebra == "hadamard":
        return HadamardTernaryLinearTuple, 32
    return OctonionTernaryLinear, 8


def get_head_mixer(config: WalshConfig, head_dim: int):
    """Head mixer for the configured algebra, or None (chassis.py:68-94)."""
    if not config.head_mixing:
        return None
    if config.algebra == "hadamard":
        if config.n_head % 32 != 0:
            raise ValueError(f"Hadamard head_mixing requires n_head % 32 == 0, got {config.n_head}")
        return HadamardHeadMixerFused(head_dim)
    if config.n_head % 8 != 0:
        raise ValueError(f"Octonion head_mixing requires n_head % 8 == 0, got {config.n_head}")
    return OctonionHeadMixerFused(head_dim)


class RMSNorm(nn.Module):
    """x * rsqrt(mean(x^2) + eps) * weight, computed in float32 (chassis.py:96-106)."""

    def __init__(self, dim, eps=1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def _norm(self, x):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps)

    def forward(self, x):
        return self._norm(x.float()).type_as(x) * self.weight


class KVCache:
    """Per-layer K/V cache (chassis.py:262-330), extended to a batch
    dimension.  Storage is [batch, n_head, max_seq_len, head_dim] so that the
    attention reads each head's keys contiguously; ``update`` returns the
    reference's [batch, total_len, n_head, head_dim] view of it."""

    def __init__(self, n_layers: int, max_seq_len: int, n_head: int, head_dim: int,
                 device: torch.device, dtype: torch.dtype = torch.bfloat16, batch: int = 1):
        self.n_layers = n_layers
        self.max_seq_len = max_seq_len
        self.n_head = n_head
        self.head_dim = head_dim
        self.batch = batch
        self.k_cache: List[torch.Tensor] = [
            torch.zeros(batch, n_head, max_seq_len, head_dim, device=device, dtype=dtype) for _ in range(n_layers)]
        self.v_cache: List[torch.Tensor] = [
            torch.zeros(batch, n_head, max_seq_len, head_dim, device=device, dtype=dtype) for _ in range(n_layers)]
        self.cached_len = 0

    def update(self, layer_idx: int, k: torch.Tensor, v: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        b, new_len = k.shape[0], k.shape[1]
        assert b <= self.batch, f"batch {b} exceeds cache batch {self.batch}"
        s, e = self.cached_len, self.cached_len + new_len
        assert e <= self.max_seq_len, "KV cache overflow"
        kc = self.k_cache[layer_idx].transpose(1, 2)   # [batch, max_seq_len, n_head, head_dim] view
        vc = self.v_cache[layer_idx].transpose(1, 2)
        kc[:b, s:e] = k.to(kc.dtype)
        vc[:b, s:e] = v.to(vc.dtype)
        return kc[:b, :e], vc[:b, :e]

    def slot(self, layer_idx: int, b: int, new_len: int = 1) -> Tuple[torch.Tensor, torch.Tensor]:
        """Views [b, new_len, n_head, head_dim] of the positions the next
        ``update`` of this layer would write, for producers that store there
        directly (then ``filled`` replaces ``update``)."""
        s = self.cached_len
        assert b <= self.batch and s + new_len <= self.max_seq_len, "KV cache overflow"
        return (self.k_cache[layer_idx].transpose(1, 2)[:b, s:s + new_len],
                self.v_cache[layer_idx].transpose(1, 2)[:b, s:s + new_len])

    def filled(self, layer_idx: int, b: int, new_len: int = 1) -> Tuple[torch.Tensor, torch.Tensor]:
        """What ``update`` returns, once the new positions hold their k and v."""
        e = self.cached_len + new_len
        return self.k_cache[layer_idx].transpose(1, 2)[:b, :e], self.v_cache[layer_idx].transpose(1, 2)[:b, :e]

    def increment(self, n: int = 1):
        self.cached_len += n

    def reset(self):
        self.cached_len = 0


def precompute_freqs_cis(dim: int, end: int, theta: float = 10000.0):
    """RoPE table (chassis.py:332-337)."""
    freqs = 1.0 / (theta ** (torch.arange(0, dim, 2)[: (dim // 2)].float() / dim))
    t = torch.arange(end, device=freqs.device)
    freqs = torch.outer(t, freqs).float()
    return torch.polar(torch.ones_like(freqs), freqs)


def apply_rotary_emb(xq, xk, freqs_cis):
    """Complex rotation of (q, k) pairs (chassis.py:339-345)."""
    xq_ = torch.view_as_complex(xq.float().reshape(*xq.shape[:-1], -1, 2))
    xk_ = torch.view_as_complex(xk.float().reshape(*xk.shape[:-1], -1, 2))
    freqs_cis = freqs_cis[:xq.shape[1]].unsqueeze(0).unsqueeze(2)
    xq_out = torch.view_as_real(xq_ * freqs_cis).flatten(3)
    xk_out = torch.view_as_real(xk_ * freqs_cis).flatten(3)
    return xq_out.type_as(xq), xk_out.type_as(xk)


class OctonionHeadMixer(OctonionHeadMixerFused):
    """chassis.py:347-399: same parameters and result as the fused mixer."""


def _qkv_layers(attn):
    """The inner Hadamard layers of wq, wk, wv when all three are Hadamard
    tuples of one shape (else None)."""
    inner = [getattr(m, "inner", None) for m in (attn.wq, attn.wk, attn.wv)]
    if any(i is None or not hasattr(i, "ternary_state") for i in inner):
        return None
    if len({(i.in_o, i.out_o) for i in inner}) != 1:
        return None
    return inner


def _attention_backends(tracked: bool):
    """Under autograd with 16-bit operands, scaled_dot_product_attention may
    use only the fused flash / memory-efficient kernels: the math
    fallback's backward makes bf16 batched products with transposed right
    operands (see _common.tracked_dtype), so a case those kernels cannot
    take raises instead."""
    import contextlib
    if not tracked:
        return contextlib.nullcontext()
    from torch.nn.attention import SDPBackend, sdpa_kernel
    return sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION])


def _full(layer, x):
    """Apply a tuple-interface ternary linear to a full [.., C] tensor."""
    return layer.forward_full(x)


class CausalSelfAttention(nn.Module):
    """chassis.py:401-483.  q/k/v/o are the algebra's ternary linears applied
    to whole rows (identical to split -> layer -> cat)."""

    def __init__(self, config):
        super().__init__()
        self.n_head = config.n_head
        self.n_embd = config.n_embd
        self.head_dim = config.n_embd // config.n_head
        self.head_mixing = config.head_mixing
        LinearLayer, self.algebra_dim = get_linear_layer(config)
        self.mixer_dim = 32 if config.algebra == "hadamard" else 8
        self.wq = LinearLayer(config.n_embd, config.n_embd)
        self.wk = LinearLayer(config.n_embd, config.n_embd)
        self.wv = LinearLayer(config.n_embd, config.n_embd)
        self.wo = LinearLayer(config.n_embd, config.n_embd)
        self.dropout = config.dropout
        self.head_mixer = get_head_mixer(config, self.head_dim)

    def _qkv_multi(self, x, freqs_cis, T, outs=None):
        """q (roped), k (roped), v in one launch (walsh_hadamard_linear_multi_fwd),
        or None when the layers, shapes or autograd do not allow it.  ``outs``:
        optional tensors to write (kernels.hadamard_linear_multi)."""
        inner = _qkv_layers(self)
        if inner is None or x.dim() != 3 or freqs_cis.shape[0] < T:
            return None
        if any(i._needs_grad(x) for i in inner) or not kernels.rope_supported(x, inner[0].out_o, self.head_dim):
            return None
        layers = [(i.ternary_state()[2], i.alpha, i.beta, r) for i, r in zip(inner, (True, True, False))]
        return kernels.hadamard_linear_multi(x, inner[0].in_o, inner[0].out_o, layers, freqs_cis, self.head_dim,
                                             outs=outs)

    def _mixer_proj(self, yg, B, T):
        """The head mixer and the output projection in one launch
        (kernels.head_mixer_proj, bitwise the two launches): inference in
        bf16 with head_dim 16, one group of 32 heads and a 16x16 Hadamard
        output projection; None where that does not hold."""
        wo = getattr(self.wo, "inner", self.wo)
        if (yg.shape[1] != 1 or self.head_dim != 16 or getattr(wo, "in_o", 0) != 16 or getattr(wo, "out_o", 0) != 16
                or not hasattr(wo, "ternary_state") or not hasattr(self.head_mixer, "_kweight")):
            return None
        x = yg[:, 0]
        if act_dtype(x) != torch.bfloat16 or not kernels.head_mixer_proj_supported(x, B * T) or wo._needs_grad(x):
            return None
        _, _, kw = wo.ternary_state()
        return kernels.head_mixer_proj(x, self.head_mixer._kweight(torch.bfloat16), self.head_mixer.beta, kw,
                                       wo.alpha, wo.beta)

    def forward(self, x, freqs_cis, kv_cache: Optional[KVCache] = None, layer_idx: int = 0):
        B, T, C = x.size()
        dt = act_dtype(x)
        x = x.to(dt)
        q = k = None
        fused, in_cache = None, False
        if (kv_cache is not None and T == 1 and B <= kv_cache.batch and self.n_head == 32
                and kv_cache.cached_len < kv_cache.max_seq_len and kv_cache.k_cache[layer_idx].dtype == dt):
            # decode: k and v go straight into the cache slot (no copy kernels)
            fused = self._qkv_multi(x, freqs_cis, T, outs=(None,) + kv_cache.slot(layer_idx, B))
            in_cache = fused is not None
        if fused is None:
            fused = self._qkv_multi(x, freqs_cis, T)
        if fused is not None:
            q, k, v = (t.view(B, T, self.n_head, self.head_dim) for t in fused)
        elif hasattr(self.wq, "forward_full_rope") and freqs_cis.shape[0] >= T:
            # the rotary embedding rides on the q and k projections' stores
            q = self.wq.forward_full_rope(x, freqs_cis, self.head_dim)
            k = self.wk.forward_full_rope(x, freqs_cis, self.head_dim) if q is not None else None
        if fused is not None:
            pass
        elif q is not None and k is not None:
            q = q.view(B, T, self.n_head, self.head_dim)
            k = k.view(B, T, self.n_head, self.head_dim)
            v = _full(self.wv, x).view(B, T, self.n_head, self.head_dim)
        else:
            q = _full(self.wq, x).view(B, T, self.n_head, self.head_dim)
            k = _full(self.wk, x).view(B, T, self.n_head, self.head_dim)
            v = _full(self.wv, x).view(B, T, self.n_head, self.head_dim)
            q, k = apply_rotary_emb(q, k, freqs_cis)
        if kv_cache is not None:
            k, v = kv_cache.filled(layer_idx, B) if in_cache else kv_cache.update(layer_idx, k, v)
        q = q.transpose(1, 2)
        k = k.transpose(1, 2).to(q.dtype)
        v = v.transpose(1, 2).to(q.dtype)
        att_dt = q.dtype
        tracked = torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad)
        drop = self.dropout if self.training else 0
        with _attention_backends(tracked and q.is_cuda and q.dtype != torch.float32):
            if kv_cache is not None and kv_cache.cached_len > 0 and T == 1:
                # one new position attends to every cached one: no mask needed;
                # the split-K decode kernel reads the cache in place
                if not tracked and drop == 0 and kernels.decode_attention_supported(q, k, v):
                    y = kernels.decode_attention(q, k, v)
                else:
                    y = F.scaled_dot_product_attention(q, k, v, dropout_p=drop)
            elif kv_cache is not None and kv_cache.cached_len > 0:
                total = k.size(2)
                mask = torch.ones(T, total, dtype=torch.bool, device=q.device).tril(diagonal=total - T)
                y = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, dropout_p=drop)
            elif (not tracked and drop == 0 and kernels.prefill_attention_preferred(q)
                  and kernels.prefill_attention_supported(q, k, v)):
                # causal prefill on the matrix cores, q / k / v read in place
                y = kernels.prefill_attention(q, k, v)
            else:
                y = F.scaled_dot_product_attention(q, k, v, is_causal=True, dropout_p=drop)
        y = y.to(att_dt)
        if self.head_mixer is not None:
            n_groups = self.n_head // self.mixer_dim
            yg = y.view(B, n_groups, self.mixer_dim, T, self.head_dim)
            if hasattr(self.head_mixer, "forward_rows") and self.head_mixer.uses_kernel(y):
                fused = self._mixer_proj(yg, B, T)
                if fused is not None:
                    return fused
                # the mixer kernel writes each group's heads straight into
                # the token-major rows: no cat and no transpose copy
                gw = self.mixer_dim * self.head_dim
                yr = torch.empty(B, T, C, device=y.device, dtype=y.dtype)
                for g in range(n_groups):
                    self.head_mixer.forward_rows(yg[:, g], out=yr[:, :, g * gw:(g + 1) * gw])
                return _full(self.wo, yr.to(dt))
            y = torch.cat([self.head_mixer(yg[:, g]) for g in range(n_groups)], dim=1)
        y = y.transpose(1, 2).contiguous().view(B, T, C).to(dt)
        return _full(self.wo, y)


class SwiGLUMLP(nn.Module):
    """down(silu(gate(x)) * up(x)) with ternary algebra linears (chassis.py:485-507)."""

    def __init__(self, config):
        super().__init__()
        LinearLayer, self.algebra_dim = get_linear_layer(config)
        hidden_dim = 4 * config.n_embd
        hidden_dim = int(2 * hidden_dim / 3)
        hidden_dim = math.ceil(hidden_dim / self.algebra_dim) * self.algebra_dim
        self.gate_proj = LinearLayer(config.n_embd, hidden_dim)
        self.up_proj = LinearLayer(config.n_embd, hidden_dim)
        self.down_proj = LinearLayer(hidden_dim, config.n_embd)

    def forward(self, x):
        x = x.to(act_dtype(x))
        if isinstance(self.gate_proj, HadamardTernaryLinearTuple) and not (
                torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters()))):
            # fused gate/up/silu*mul (inference; under autograd the three
            # differentiable linears below run); the hidden activation stays in
            # a group-padded layout (stride roundup(hid_o, 4)) read in place by down_proj
            g, u, d = self.gate_proj.inner, self.up_proj.inner, self.down_proj.inner
            hid_o = g.out_o
            if d.in_o == hid_o and kernels.hadamard_mlp_supported(x, g.in_o, hid_o, d.out_o):
                # the whole MLP in one launch, the hidden activation on chip
                return kernels.hadamard_mlp(x, g.in_o, hid_o, d.out_o, (g.ternary_state()[2], g.alpha, g.beta),
                                            (u.ternary_state()[2], u.alpha, u.beta),
                                            (d.ternary_state()[2], d.alpha, d.beta))
            h = kernels.hadamard_swiglu(x, g.in_o, hid_o, (g.ternary_state()[2], g.alpha, g.beta),
                                        (u.ternary_state()[2], u.alpha, u.beta))
            return kernels.hadamard_linear(h, d.in_o, d.out_o, d.ternary_state()[2], d.alpha, d.beta,
                                           gsx=h.shape[-1] // 32)
        if isinstance(self.gate_proj, HadamardTernaryLinearTuple):
            # training: the three linears with their backward kernels, the
            # hidden activation in the same group-padded layout (stride
            # roundup(hid_o, 4); pad slots are zeros and stay zero)
            g, u, d = self.gate_proj.inner, self.up_proj.inner, self.down_proj.inner
            gsh = (g.out_o + 3) // 4 * 4
            hg = HadamardLinearFunction.apply(x, g.weight, g.alpha, g.beta, g, None, gsh)
            hu = HadamardLinearFunction.apply(x, u.weight, u.alpha, u.beta, u, None, gsh)
            return HadamardLinearFunction.apply(F.silu(hg) * hu, d.weight, d.alpha, d.beta, d, gsh, None)
        h = F.silu(_full(self.gate_proj, x)) * _full(self.up_proj, x)
        return _full(self.down_proj, h)


class LlamaBlock(nn.Module):
    """Pre-norm residual block (chassis.py:509-531)."""

    def __init__(self, config):
        super().__init__()
        self.attention_norm = RMSNorm(config.n_embd)
        self.attention = CausalSelfAttention(config)
        self.ffn_norm = RMSNorm(config.n_embd)
        if getattr(config, 'use_moe', False):
            from .moe import HadamardMoE
            self.feed_forward = HadamardMoE(
                config,
                threshold=getattr(config, 'moe_threshold', 0.1),
                min_experts=getattr(config, 'moe_min_experts', 1),
                max_experts=getattr(config, 'moe_max_experts', 4),
            )
        else:
            self.feed_forward = SwiGLUMLP(config)

    def forward(self, x, freqs_cis, kv_cache: Optional[KVCache] = None, layer_idx: int = 0):
        dt = act_dtype(x)
        h = x + self.attention(self.attention_norm(x).to(dt), freqs_cis, kv_cache=kv_cache, layer_idx=layer_idx)
        return h + self.feed_forward(self.ffn_norm(h).to(dt))


class Walsh(nn.Module):
    """Single-stream Walsh model (chassis.py:533-668)."""

    def __init__(self, config):
        super().__init__()
        if config.hash_embeddings:
            raise NotImplementedError("hash embeddings are outside this build's scope")
        self.config = config
        self.tok_embeddings = nn.Embedding(config.vocab_size, config.n_embd)
        self.output = nn.Linear(config.n_embd, config.vocab_size, bias=False)
        self.tok_embeddings.weight = self.output.weight
        self.layers = nn.ModuleList([LlamaBlock(config) for _ in range(config.n_layer)])
        self.norm = RMSNorm(config.n_embd)
        self._output_cast = WeightCache()
        self.register_buffer("freqs_cis", precompute_freqs_cis(config.n_embd // config.n_head, config.block_size * 2))
        self.apply(self._init_weights)
        for pn, p in self.named_parameters():
            if pn.endswith('.beta'):
                torch.nn.init.constant_(p, 0.1)

    def _init_weights(self, module):
        if isinstance(module, (nn.Linear, nn.Embedding)):
            torch.nn.init.normal_(module.weight, mean=0.0, std=0.02)

    def forward(self, idx, targets=None, kv_cache: Optional[KVCache] = None, start_pos: int = 0,
                return_hidden: bool = False):
        B, T = idx.shape
        h = self.tok_embeddings(idx)
        freqs_cis = self.freqs_cis[start_pos:start_pos + T]
        for layer_idx, layer in enumerate(self.layers):
            if self.training and torch.is_grad_enabled():
                # every layer checkpointed in training (chassis.py:570-572)
                h = torch.utils.checkpoint.checkpoint(layer, h, freqs_cis, use_reentrant=False)
            else:
                h = layer(h, freqs_cis, kv_cache=kv_cache, layer_idx=layer_idx)
        h = self.norm(h)
        if targets is not None:
            logits = cached_linear(self.output, h, self._output_cast)
            loss = F.cross_entropy(logits.view(-1, logits.size(-1)), targets.view(-1))
        else:
            logits = cached_linear(self.output, h[:, [-1], :], self._output_cast)
            loss = None
        if return_hidden:
            return logits, loss, h
        return logits, loss
