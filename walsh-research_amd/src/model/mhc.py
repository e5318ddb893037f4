"""Manifold-constrained hyper-connections (module surface of src/model/mhc.py).

SinkhornKnopp / sinkhorn_knopp_fused -> walsh_sinkhorn_fwd;
mHCResidualStream.forward -> walsh_mhc_pre_fwd (RMS scale, the three phi
projections, sigmoid / 2*sigmoid / Sinkhorn and H_pre @ x in one pass), the
layer function, then walsh_mhc_post_fwd (H_res @ x + H_post^T (x) out).
"""
import math

import torch
import torch.utils.checkpoint
import torch.nn as nn
import torch.nn.functional as F

from . import kernels
from ._common import WeightCache, act_dtype, cached_linear, invalidate_weight_caches

_MAX_STREAMS = 4


class StreamAggregateFunction(torch.autograd.Function):
    """layer_in = H_pre @ x (mhc.py:366) with its backward on the GPU
    (walsh_mhc_aggregate_fwd / _bwd)."""

    @staticmethod
    def forward(ctx, x, h_pre):
        ctx.save_for_backward(x, h_pre)
        return kernels.mhc_aggregate(x, h_pre)

    @staticmethod
    def backward(ctx, g):
        x, h_pre = ctx.saved_tensors
        dx, dh = kernels.mhc_aggregate_bwd(x, h_pre, g)
        return dx, dh.to(h_pre.dtype)


class StreamUpdateFunction(torch.autograd.Function):
    """x_new = H_res @ x + H_post^T (x) out (mhc.py:366-381) with its
    backward on the GPU (walsh_mhc_post_fwd / walsh_mhc_post_bwd)."""

    @staticmethod
    def forward(ctx, x, out, h_res, h_post):
        ctx.save_for_backward(x, out, h_res, h_post)
        return kernels.mhc_post(x, out, h_res, h_post)

    @staticmethod
    def backward(ctx, g):
        x, out, h_res, h_post = ctx.saved_tensors
        dx, dout, dhr, dhq = kernels.mhc_post_bwd(x, out, h_res, h_post, g)
        return dx, dout.to(out.dtype), dhr.to(h_res.dtype), dhq.to(h_post.dtype)


class SinkhornFunction(torch.autograd.Function):
    """Sinkhorn projection with its backward on the GPU (walsh_sinkhorn_fwd /
    walsh_sinkhorn_bwd); the reference differentiates its torch loop
    (mhc.py:214-229) with autograd."""

    @staticmethod
    def forward(ctx, H, n_iter, eps):
        ctx.save_for_backward(H)
        ctx.n_iter, ctx.eps = n_iter, eps
        return kernels.sinkhorn(H, n_iter=n_iter, eps=eps)

    @staticmethod
    def backward(ctx, g):
        (H,) = ctx.saved_tensors
        return kernels.sinkhorn_bwd(H, g, n_iter=ctx.n_iter, eps=ctx.eps).to(H.dtype), None, None


def _sinkhorn(H, n_iter, eps):
    if torch.is_grad_enabled() and H.requires_grad:
        return SinkhornFunction.apply(H, n_iter, eps)
    return kernels.sinkhorn(H, n_iter=n_iter, eps=eps)


def sinkhorn_knopp_fused(H_tilde, n_iter=20):
    """Doubly-stochastic projection of [..., n, n] (mhc.py:152-195), float32."""
    return _sinkhorn(H_tilde, n_iter, 1e-8)


class SinkhornKnopp(nn.Module):
    """M = exp(H); n_iter x {column-normalise, row-normalise} (mhc.py:198-229)."""

    def __init__(self, n_iter=20, eps=1e-8):
        super().__init__()
        self.n_iter = n_iter
        self.eps = eps

    def forward(self, H):
        return _sinkhorn(H, self.n_iter, self.eps)


def _rms_eps(dtype: torch.dtype) -> float:
    # F.rms_norm(x, ...) with eps=None (mhc.py:291) normalises in the op-math
    # type (float32 for bf16 / fp16 inputs) and takes that type's epsilon:
    # 2^-23 for bf16 and fp32 activations, bit for bit the same as
    # rsqrt(mean(x.float()^2) + 2^-23) rounded back to the input dtype.
    # rms_norm has no autocast rule, so x keeps the activation dtype.
    return float(torch.finfo(torch.float64 if dtype == torch.float64 else torch.float32).eps)


def _phi_block(n: int, C: int, parts, dtype, device):
    """[32, n*C] projection in the activation dtype: rows pre|post|res, zero padded."""
    out = torch.zeros(32, n * C, device=device, dtype=dtype)
    r = 0
    for w, rows in parts:
        if w is not None:
            out[r:r + rows] = w.detach().to(dtype)
        r += rows
    return out


class ResidualStreamMapping(nn.Module):
    """H = P(alpha * phi(rms_norm(x)) + bias) with P = sigmoid ('pre'),
    2*sigmoid ('post') or Sinkhorn ('res') (mhc.py:232-318)."""

    def __init__(self, n_embd, n_streams, mapping_type='res'):
        super().__init__()
        self.n_embd = n_embd
        self.n_streams = n_streams
        self.mapping_type = mapping_type
        self.alpha = nn.Parameter(torch.tensor(0.01))
        if mapping_type == 'res':
            self.phi = nn.Linear(n_streams * n_embd, n_streams * n_streams, bias=False)
            self.bias = nn.Parameter(torch.zeros(n_streams, n_streams))
            self.sinkhorn = SinkhornKnopp(n_iter=20)
            with torch.no_grad():
                self.bias.copy_(torch.eye(n_streams) * 2.0)
        elif mapping_type == 'pre':
            self.phi = nn.Linear(n_streams * n_embd, n_streams, bias=False)
            self.bias = nn.Parameter(torch.zeros(1, n_streams))
        elif mapping_type == 'post':
            self.phi = nn.Linear(n_streams * n_embd, n_streams, bias=False)
            self.bias = nn.Parameter(torch.zeros(1, n_streams))
        nn.init.normal_(self.phi.weight, std=0.01)
        self._cache = WeightCache()

    def forward(self, x):
        """x [B, T, n*C] -> [B, T, n, n] ('res') or [B, T, 1, n]."""
        n, C = self.n_streams, self.n_embd
        if n > _MAX_STREAMS:
            raise NotImplementedError(f"n_streams={n} > {_MAX_STREAMS} is not supported by this build")
        B, T, _ = x.shape
        if torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters())):
            # differentiable form for training (the fused kernel has no backward)
            xn = F.rms_norm(x, (x.size(-1),))
            dyn = F.linear(xn, self.phi.weight.to(xn.dtype))
            if self.mapping_type == 'res':
                h = (self.alpha * dyn.view(B, T, n, n) + self.bias).float()
                return _sinkhorn(h, self.sinkhorn.n_iter, self.sinkhorn.eps)
            s = torch.sigmoid(self.alpha * dyn + self.bias).unsqueeze(2)
            return s if self.mapping_type == 'pre' else 2.0 * s
        dt = act_dtype(x)
        slot = {'pre': 0, 'post': 1, 'res': 2}[self.mapping_type]

        def build():
            ws = [None, None, None]
            ws[slot] = self.phi.weight
            phi = _phi_block(n, C, [(ws[0], n), (ws[1], n), (ws[2], n * n)], dt, x.device)
            coef = torch.zeros(3, device=x.device)
            coef[slot] = self.alpha.detach().float()
            bias = torch.zeros(2 * n + n * n, device=x.device)
            off = [0, n, 2 * n][slot]
            bias[off:off + self.bias.numel()] = self.bias.detach().float().reshape(-1)
            return phi, coef, bias

        phi, coef, bias = self._cache.get([self.phi.weight, self.alpha, self.bias], build, extra=(dt, x.device))
        xs = x.to(dt).reshape(B, T, n, C)
        _, hp, hq, hr = kernels.mhc_pre(xs, phi, coef, bias, _rms_eps(dt))
        if self.mapping_type == 'res':
            return hr
        return (hp if self.mapping_type == 'pre' else hq).unsqueeze(2)


class PendingUpdate:
    """A stream update x_new = H_res @ x + H_post^T (x) out (mhc.py:366-381)
    that has not been applied yet.  The next stream's mapping kernel forms it
    while loading its tile (walsh_mhc_post_pre_norm_fwd; for rows too long for
    an LDS tile, its projection launch, walsh_mhc_post_pre_wide_fwd), which
    saves one pass over the streams; ``materialize`` applies it on its own."""
    __slots__ = ('x', 'out', 'h_res', 'h_post')

    def __init__(self, x, out, h_res, h_post):
        self.x, self.out, self.h_res, self.h_post = x, out, h_res, h_post

    @property
    def shape(self):
        return self.x.shape

    def materialize(self) -> torch.Tensor:
        return kernels.mhc_post(self.x, self.out, self.h_res, self.h_post)


def materialize(x):
    return x.materialize() if isinstance(x, PendingUpdate) else x


class mHCResidualStream(nn.Module):
    """x_{l+1} = H_res @ x_l + H_post^T F(H_pre @ x_l) (mhc.py:321-381)."""

    def __init__(self, n_embd, n_streams=4):
        super().__init__()
        self.n_embd = n_embd
        self.n_streams = n_streams
        self.H_pre = ResidualStreamMapping(n_embd, n_streams, 'pre')
        self.H_post = ResidualStreamMapping(n_embd, n_streams, 'post')
        self.H_res = ResidualStreamMapping(n_embd, n_streams, 'res')
        self._cache = WeightCache()

    def fused_params(self, dtype, device):
        """(phi [32, n*C], coef [3], bias [2n + n*n]) for the fused kernel."""
        n, C = self.n_streams, self.n_embd
        maps = (self.H_pre, self.H_post, self.H_res)

        def build():
            phi = _phi_block(n, C, [(self.H_pre.phi.weight, n), (self.H_post.phi.weight, n),
                                    (self.H_res.phi.weight, n * n)], dtype, device)
            coef = torch.stack([m.alpha.detach().float() for m in maps]).to(device)
            bias = torch.cat([m.bias.detach().float().reshape(-1) for m in maps]).to(device)
            if kernels.mhc_pre_supported(n, C, dtype) and (n * C) % 16 == 0:
                frag = kernels.phi_fragments(phi)
            elif kernels.mhc_pre_wide_supported(n, C):
                frag = kernels.phi_fragments32(phi)
            else:
                frag = None
            return phi, coef, bias, frag

        tensors = [t for m in maps for t in (m.phi.weight, m.alpha, m.bias)]
        return self._cache.get(tensors, build, extra=(dtype, device))

    def _pre(self, x, dt, norm=None):
        n, C = self.n_streams, self.n_embd
        if n > _MAX_STREAMS:
            raise NotImplementedError(f"n_streams={n} > {_MAX_STREAMS} is not supported by this build")
        phi, coef, bias, frag = self.fused_params(dt, x.device)
        nw = None if norm is None else norm.weight
        neps = 1e-6 if norm is None else norm.eps
        if frag is not None and kernels.mhc_pre_supported(n, C, dt):
            return kernels.mhc_pre_norm(x, frag, coef, bias, _rms_eps(dt), norm_w=nw, norm_eps=neps)
        if frag is not None and kernels.mhc_pre_wide_supported(n, C):
            return kernels.mhc_pre_wide(x, frag, coef, bias, _rms_eps(dt), norm_w=nw, norm_eps=neps)
        li, hp, hq, hr = kernels.mhc_pre(x, phi, coef, bias, _rms_eps(dt))
        if norm is not None:
            li = norm(li).to(dt)
        return li, hp, hq, hr

    def _tracked(self, x) -> bool:
        return torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters()))

    def _forward_autograd(self, x, norm, layer_fn):
        """The stream update as differentiable operations, for training
        (mhc.py:345-381 with the mappings of :283-318): one projection for
        the three mappings' phi rows, sigmoid / 2*sigmoid, the Sinkhorn
        projection as SinkhornFunction (its backward on the GPU), then
        H_pre @ x, the layer, H_res @ x + H_post^T out.  The fused inference
        kernels (walsh_mhc_pre_fwd / walsh_mhc_post_fwd) have no backward."""
        B, T, n, C = x.shape
        xn = F.rms_norm(x.reshape(B, T, n * C), (n * C,))
        phi = torch.cat([self.H_pre.phi.weight, self.H_post.phi.weight, self.H_res.phi.weight], 0)
        d_pre, d_post, d_res = F.linear(xn, phi.to(xn.dtype)).split([n, n, n * n], dim=-1)
        h_pre = torch.sigmoid(self.H_pre.alpha * d_pre + self.H_pre.bias).unsqueeze(2)
        h_post = 2.0 * torch.sigmoid(self.H_post.alpha * d_post + self.H_post.bias).unsqueeze(2)
        sk = self.H_res.sinkhorn
        h_res = _sinkhorn((self.H_res.alpha * d_res.reshape(B, T, n, n) + self.H_res.bias).float(), sk.n_iter,
                          sk.eps)
        # the n x n mixing on the GPU kernels (float32 sums, results in the
        # stream dtype, as the reference's autocast matmuls give)
        layer_in = StreamAggregateFunction.apply(x, h_pre)
        out = layer_fn(layer_in if norm is None else norm(layer_in))
        return StreamUpdateFunction.apply(x, out, h_res, h_post)

    def forward(self, x, layer_fn):
        """x [B, T, n, C]; layer_fn maps [B, T, C] -> [B, T, C]."""
        if self._tracked(x):
            return self._forward_autograd(x, None, layer_fn)
        dt = act_dtype(x)
        x = x.to(dt)
        layer_in, _, h_post, h_res = self._pre(x, dt)
        out = layer_fn(layer_in)
        return kernels.mhc_post(x, out, h_res, h_post)

    def _post_pre(self, p: PendingUpdate, dt, norm):
        """The pending update of the previous stream fused with this stream's
        mappings, or None when the fused kernel does not take the shape."""
        n, C = self.n_streams, self.n_embd
        if p.x.dtype != dt or n > _MAX_STREAMS:
            return None
        nw = None if norm is None else norm.weight
        neps = 1e-6 if norm is None else norm.eps
        if kernels.mhc_post_pre_supported(n, C, dt):
            _, coef, bias, frag = self.fused_params(dt, p.x.device)
            if frag is not None:
                return kernels.mhc_post_pre_norm(p.x, p.out, p.h_res, p.h_post, frag, coef, bias, _rms_eps(dt),
                                                 norm_w=nw, norm_eps=neps)
        elif kernels.mhc_pre_wide_supported(n, C) and kernels.mhc_post_pre_wide_supported(n, C, dt):
            _, coef, bias, frag = self.fused_params(dt, p.x.device)
            if frag is not None:
                return kernels.mhc_post_pre_wide(p.x, p.out, p.h_res, p.h_post, frag, coef, bias, _rms_eps(dt),
                                                 norm_w=nw, norm_eps=neps)
        return None

    def forward_normed(self, x, norm, layer_fn, defer: bool = False):
        """forward(x, lambda v: layer_fn(norm(v))) with the RMSNorm ``norm``
        (chassis.RMSNorm) fused into the mapping kernel.  ``x`` may be a
        PendingUpdate of the previous stream; with ``defer`` the result is
        returned as one (inference only)."""
        if isinstance(x, PendingUpdate) and self._tracked(x.x):
            x = x.materialize()
        if not isinstance(x, PendingUpdate) and self._tracked(x):
            return self._forward_autograd(x, norm, layer_fn)
        fused = None
        if isinstance(x, PendingUpdate):
            dt = act_dtype(x.x)
            fused = self._post_pre(x, dt, norm)
            if fused is None:
                x = x.materialize()
        if fused is not None:
            x, layer_in, _, h_post, h_res = fused
        else:
            dt = act_dtype(x)
            x = x.to(dt)
            layer_in, _, h_post, h_res = self._pre(x, dt, norm=norm)
        out = layer_fn(layer_in)
        if defer:
            return PendingUpdate(x, out, h_res, h_post)
        return kernels.mhc_post(x, out, h_res, h_post)


class mHCBlock(nn.Module):
    """Attention and FFN each wrapped in an mHC stream (mhc.py:384-423)."""

    def __init__(self, attention_module, ffn_module, n_embd, n_streams=4):
        super().__init__()
        self.n_streams = n_streams
        self.attention = attention_module
        self.ffn = ffn_module
        self.attn_stream = mHCResidualStream(n_embd, n_streams)
        self.ffn_stream = mHCResidualStream(n_embd, n_streams)

    def forward(self, x, freqs_cis, kv_cache=None, layer_idx=0):
        x = self.attn_stream(x, lambda v: self.attention(v, freqs_cis, kv_cache=kv_cache, layer_idx=layer_idx))
        return self.ffn_stream(x, lambda v: self.ffn(v))


def wrap_with_mhc(model_class, n_streams=4):
    """As in the reference (mhc.py:426-445): use mHCBlock directly."""
    raise NotImplementedError("Use mHCBlock directly in your model architecture. See mHCWalsh for an example.")


class mHCLlamaBlock(nn.Module):
    """Llama block with mHC streams around attention and FFN (mhc.py:451-534)."""

    def __init__(self, config, n_streams=4):
        super().__init__()
        self.n_streams = n_streams
        self.n_embd = config.n_embd
        from .chassis import CausalSelfAttention, RMSNorm, SwiGLUMLP
        self.attention_norm = RMSNorm(config.n_embd)
        self.ffn_norm = RMSNorm(config.n_embd)
        self.attention = CausalSelfAttention(config)
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
        self._moe = getattr(config, 'use_moe', False)
        self.use_channel_mod = getattr(config, 'use_channel_mod', False)
        if self.use_channel_mod:
            from .moe import HadamardChannelModulation
            self.channel_mod = HadamardChannelModulation(n_embd=config.n_embd, n_blocks=None, use_ternary=True,
                                                         residual_scale=0.5)
            self.channel_mod_norm = RMSNorm(config.n_embd)
        self.attn_stream = mHCResidualStream(config.n_embd, n_streams)
        self.ffn_stream = mHCResidualStream(config.n_embd, n_streams)

    def forward(self, x, freqs_cis, kv_cache=None, layer_idx=0):
        return materialize(self.forward_deferred(x, freqs_cis, kv_cache=kv_cache, layer_idx=layer_idx))

    def forward_deferred(self, x, freqs_cis, kv_cache=None, layer_idx=0):
        """forward() for x a tensor or a PendingUpdate; the FFN stream's
        update may come back pending (applied by the next block's first
        mapping kernel)."""
        # attn_stream(x, attention(attention_norm(.))) then
        # ffn_stream(x, feed_forward(ffn_norm(.))) (mhc.py:507-534), with each
        # RMSNorm fused into its stream's mapping kernel and each stream
        # update fused into the next stream's mapping kernel
        x = self.attn_stream.forward_normed(
            x, self.attention_norm,
            lambda v: self.attention(v, freqs_cis, kv_cache=kv_cache, layer_idx=layer_idx), defer=True)
        ff = self.feed_forward
        defer = not self.use_channel_mod
        if self._moe:
            # the stream update rounds the FFN output to the stream dtype
            # (autocast matmul, mhc.py:374-377), so produce it in that dtype
            x = self.ffn_stream.forward_normed(x, self.ffn_norm, lambda v: ff(v, out_dtype=v.dtype), defer=defer)
        else:
            x = self.ffn_stream.forward_normed(x, self.ffn_norm, ff, defer=defer)
        if self.use_channel_mod:
            # x + channel_mod(norm(x)) on the [B*n, T, C] view of the
            # contiguous [B, T, n, C] streams (mhc.py:528-532): a "group" of T
            # rows is that view's, as there, not one stream's.  The result
            # stays in the stream dtype.
            B, T, n, C = x.shape
            x = self.channel_mod.fused_residual(x.contiguous().view(B * n, T, C), self.channel_mod_norm)
            x = x.view(B, T, n, C)
        return x


class mHCWalsh(nn.Module):
    """Walsh model with n parallel residual streams (mhc.py:537-789)."""

    def __init__(self, config, n_streams=4, gradient_checkpointing=False):
        super().__init__()
        self.config = config
        self.n_streams = n_streams
        self.gradient_checkpointing = gradient_checkpointing
        from .chassis import RMSNorm, precompute_freqs_cis
        if getattr(config, 'hash_embeddings', False):
            raise NotImplementedError("hash embeddings are outside this build's scope")
        self.tok_embeddings = nn.Embedding(config.vocab_size, config.n_embd)
        self.output = nn.Linear(config.n_embd, config.vocab_size, bias=False)
        self.tok_embeddings.weight = self.output.weight
        self.stream_proj = nn.Linear(config.n_embd, n_streams * config.n_embd)
        self.layers = nn.ModuleList([mHCLlamaBlock(config, n_streams) for _ in range(config.n_layer)])
        self.stream_merge = nn.Linear(n_streams * config.n_embd, config.n_embd)
        self.norm = RMSNorm(config.n_embd)
        self._casts = {"proj": WeightCache(), "merge": WeightCache(), "output": WeightCache()}
        self.register_buffer("freqs_cis", precompute_freqs_cis(config.n_embd // config.n_head,
                                                               config.block_size * 2))
        self.apply(self._init_weights)
        with torch.no_grad():
            eye = torch.eye(config.n_embd).repeat(n_streams, 1) / math.sqrt(n_streams)
            self.stream_proj.weight.copy_(eye)
            if self.stream_proj.bias is not None:
                self.stream_proj.bias.zero_()
            avg = torch.eye(config.n_embd).repeat(1, n_streams) / n_streams
            self.stream_merge.weight.copy_(avg)
            if self.stream_merge.bias is not None:
                self.stream_merge.bias.zero_()

    def _init_weights(self, module):
        if isinstance(module, nn.Linear):
            torch.nn.init.normal_(module.weight, mean=0.0, std=0.02)
            if module.bias is not None:
                torch.nn.init.zeros_(module.bias)
        elif isinstance(module, nn.Embedding):
            torch.nn.init.normal_(module.weight, mean=0.0, std=0.02)

    def forward(self, idx, targets=None, kv_cache=None, start_pos=0, return_hidden=False):
        B, T = idx.shape
        h = self.tok_embeddings(idx)
        h = cached_linear(self.stream_proj, h, self._casts["proj"])
        dt = act_dtype(h)
        h = h.to(dt).view(B, T, self.n_streams, self.config.n_embd)
        freqs_cis = self.freqs_cis[start_pos:start_pos + T]
        checkpointed = self.gradient_checkpointing and self.training and torch.is_grad_enabled()
        for layer_idx, layer in enumerate(self.layers):
            if checkpointed:
                # activation checkpointing per layer (mhc.py:647-649): the
                # layer's forward is recomputed in the backward; it takes and
                # returns plain tensors (no pending stream update crosses it)
                h = torch.utils.checkpoint.checkpoint(layer.forward, materialize(h), freqs_cis, kv_cache, layer_idx,
                                                      use_reentrant=False)
            else:
                h = layer.forward_deferred(h, freqs_cis, kv_cache=kv_cache, layer_idx=layer_idx)
        h = materialize(h)
        h_flat = h.reshape(B, T, self.n_streams * self.config.n_embd)
        h_out = self.norm(cached_linear(self.stream_merge, h_flat, self._casts["merge"]))
        if targets is not None:
            logits = cached_linear(self.output, h_out, self._casts["output"])
            loss = F.cross_entropy(logits.view(-1, logits.size(-1)), targets.view(-1), ignore_index=-1)
        else:
            logits = cached_linear(self.output, h_out[:, -1:, :], self._casts["output"])
            loss = None
        if return_hidden:
            return logits, loss, h_out
        return logits, loss

    def invalidate_weight_caches(self) -> None:
        """Rebuild the ternary codes and kernel layouts on the next forward:
        call after writing parameters through ``.data`` (which autograd's
        version counter, the caches' change detector, does not see)."""
        invalidate_weight_caches()

    @property
    def num_parameters(self):
        total = sum(p.numel() for p in self.parameters())
        trainable = sum(p.numel() for p in self.parameters() if p.requires_grad)
        return total, trainable

    def get_aux_loss(self):
        aux = 0.0
        for layer in self.layers:
            if hasattr(layer.feed_forward, 'get_aux_loss'):
                aux = aux + layer.feed_forward.get_aux_loss()
        return aux

    def get_moe_stats(self) -> dict:
        stats = [l.feed_forward.get_expert_stats() for l in self.layers if hasattr(l.feed_forward, 'get_expert_stats')]
        if not stats:
            return {}
        E = len(stats[0]['expert_load'])
        load = [sum(s['expert_load'][i] for s in stats) / len(stats) for i in range(E)]
        return {'expert_load': load,
                'avg_experts': sum(s['avg_experts'] for s in stats) / len(stats),
                'load_balance': sum(s['load_balance'] for s in stats) / len(stats)}

    def reset_moe_stats(self):
        for layer in self.layers:
            if hasattr(layer.feed_forward, 'reset_stats'):
                layer.feed_forward.reset_stats()

    def get_channel_mod_stats(self) -> dict:
        """Channel-modulation statistics averaged over the layers (mhc.py:733-751)."""
        stats = [l.channel_mod.get_modulation_stats() for l in self.layers if hasattr(l, 'channel_mod')]
        if not stats:
            return {}
        return {k: sum(s[k] for s in stats) / len(stats) for k in ('scale_mean', 'scale_std', 'shift_mean')}

    @torch.no_grad()
    def generate(self, idx, max_new_tokens, temperature=1.0, top_k=None):
        """Sampling loop without a cache, as in the reference (mhc.py:754-772)."""
        for _ in range(max_new_tokens):
            idx_cond = idx if idx.size(1) <= self.config.block_size else idx[:, -self.config.block_size:]
            logits, _ = self(idx_cond)
            logits = logits[:, -1, :].float() / temperature
            if top_k is not None and top_k > 0:
                v, _ = torch.topk(logits, min(top_k, logits.size(-1)))
                logits[logits < v[:, [-1]]] = -float('Inf')
            probs = F.softmax(logits, dim=-1)
            idx = torch.cat((idx, torch.multinomial(probs, num_samples=1)), dim=1)
        return idx
