"""Oracle: functional float32 CPU forward of mHCWalsh from a state dict.

Test infrastructure only (see ``oracle/__init__.py``).  This is the
reference's CPU path restated with torch-CPU float32 operations in the
reference's order (generate.py:134 runs the CPU path without autocast):

  mHCWalsh.forward             src/model/mhc.py:617-681
  mHCLlamaBlock.forward        mhc.py:507-534
  mHCResidualStream.forward    mhc.py:345-381 (mappings :283-318, Sinkhorn :214-229)
  CausalSelfAttention.forward  src/model/chassis.py:424-483 (RoPE :332-345)
  SwiGLUMLP.forward            chassis.py:498-507
  RMSNorm                      chassis.py:96-106
  HadamardLinear.forward       src/model/fht_cuda.py:489-519 (quantiser physics.py:13-51)
  HadamardHeadMixerFused       fht_cuda.py:652-670
  OctonionTernaryLinearRef     src/model/physics.py:66-82 (algebra "octonion": the CPU
                               module chassis.get_linear_layer picks without a GPU,
                               chassis.py:54-65, physics.py:84-91)
  OctonionHeadMixer            chassis.py:347-399
  HadamardMoE.forward          src/model/moe.py:512-542 (router :418-447, experts :337-380)
  HadamardChannelModulation    src/model/moe.py:676-762 (its use in the block: mhc.py:528-532)

It also serves as the timed CPU baseline of the full forward.
"""
import math

import torch
import torch.nn.functional as F


# src/model/constants.py:13-31, rows = output part i, columns = input part j
# (the Cayley-Dickson signs; oracle/octonion.py re-derives them)
OCT_SIGN = (
    (+1, -1, -1, -1, -1, -1, -1, -1),
    (+1, +1, +1, -1, +1, -1, -1, +1),
    (+1, -1, +1, +1, +1, +1, -1, -1),
    (+1, +1, -1, +1, +1, -1, +1, -1),
    (+1, -1, -1, -1, +1, +1, +1, +1),
    (+1, +1, -1, +1, -1, +1, -1, +1),
    (+1, +1, +1, -1, -1, +1, +1, -1),
    (+1, -1, +1, +1, -1, -1, +1, +1),
)


def ternary_codes(w: torch.Tensor) -> torch.Tensor:
    """clamp(round(W / (mean|W| + 1e-8)), -1, 1) in float32 (physics.py:24-29)."""
    g = w.abs().mean() + 1e-8
    return torch.clamp(torch.round(w / g), -1, 1)


def sylvester(n=32):
    H = torch.ones(1, 1)
    while H.shape[0] < n:
        H = torch.cat([torch.cat([H, H], 1), torch.cat([H, -H], 1)], 0)
    return H / math.sqrt(n)


class _MoESTE(torch.autograd.Function):
    """moe.TernaryAbsmeanSTE (moe.py:276-294): value clamp(round(w/g), -1, 1)*g
    with g = mean|w| + 1e-8; gradient clamp(grad, -2, 2)."""

    @staticmethod
    def forward(ctx, w):
        g = w.abs().mean() + 1e-8
        return torch.clamp(torch.round(w / g), -1, 1) * g

    @staticmethod
    def backward(ctx, grad):
        return torch.clamp(grad, -2.0, 2.0)


class Oracle:
    """``grad=True`` turns the oracle into the gradient reference: every
    floating entry of the state dict becomes a ``grad_dtype`` (float64) leaf (tensors that
    share storage in the model, like the tied embedding / output weight,
    share one leaf), the Hadamard weights go through the STE of
    physics.quantize_ternary (physics.py:43-50) instead of fixed codes, and
    ``loss`` gives the cross-entropy whose backward fills ``leaf.grad``."""

    def __init__(self, sd, n_embd, n_head, n_layer, n_streams=4, head_mixing=True, block_size=256,
                 use_moe=False, moe_max_experts=4, grad=False, grad_dtype=torch.float64, use_channel_mod=False,
                 algebra="hadamard", octonion_gpu=False):
        self.grad = grad
        self.dt = grad_dtype if grad else torch.float32
        if grad:
            leaves, by_ptr = {}, {}
            for k, v in sd.items():
                if v.is_complex():
                    leaves[k] = v.detach().cpu()
                    continue
                key = (v.data_ptr(), v.dtype, tuple(v.shape))
                if key not in by_ptr:
                    by_ptr[key] = v.detach().to(self.dt).cpu().requires_grad_(v.is_floating_point())
                leaves[k] = by_ptr[key]
            self.sd = leaves
        else:
            self.sd = {k: (v.detach().cpu() if v.is_complex() else v.detach().float().cpu()) for k, v in sd.items()}
        self.C = n_embd
        self.n_head = n_head
        self.n_layer = n_layer
        self.n = n_streams
        self.head_mixing = head_mixing
        self.use_moe = use_moe
        self.use_channel_mod = use_channel_mod
        self.moe_k = moe_max_experts
        self.algebra = algebra
        # octonion_gpu: the octonion layers as the reference's GPU module
        # computes them (OctonionFusedLinear, cayley_dickson_cuda.py:650-668):
        # input rounded to bf16, the float32 sum rounded to bf16, then * beta
        self.octonion_gpu = octonion_gpu
        self.H = sylvester(32).to(self.dt)
        self._codes = {}

    def codes(self, key):
        if self.grad:
            w = self.sd[key]
            wc = w.clamp(-1.5, 1.5)
            return wc + (ternary_codes(w.detach()) - wc).detach()
        if key not in self._codes:
            self._codes[key] = ternary_codes(self.sd[key])
        return self._codes[key]

    # ---------------------------------------------------------------- hot path
    def hadamard_linear(self, x, p):
        """fht_cuda.py:497-519 (x.float(), einsum H, einsum W, einsum H, * beta)."""
        w = self.codes(p + '.weight')
        G, out_o, in_o = w.shape
        lead = x.shape[:-1]
        xs = x.reshape(*lead, G, in_o) * self.sd[p + '.alpha']
        xm = torch.einsum('...gi,gh->...hi', xs.to(self.dt), self.H)
        yp = torch.einsum('...gi,goi->...go', xm, w)
        ym = torch.einsum('...go,gh->...ho', yp, self.H)
        return (ym * self.sd[p + '.beta']).reshape(*lead, G * out_o)

    def octonion_linear(self, x, p):
        """physics.py:66-82: parts x_j = x[..., j in_o:(j+1) in_o],
        y_i = (sum_j S[i][j] x_j @ Wq[i^j]^T) * beta, the sum in the
        reference's term order (S[i][0] = +1, the terms added left to right)."""
        w = self.codes(p + '.weight')
        out_o, in_o = w.shape[1], w.shape[2]
        xs = x.to(self.dt)
        if self.octonion_gpu:
            xs = xs.to(torch.bfloat16).to(self.dt)
        parts = xs.split(in_o, dim=-1)
        ys = []
        for i in range(8):
            acc = None
            for j in range(8):
                t = parts[j] @ w[i ^ j].t()
                acc = t if acc is None else (acc + t if OCT_SIGN[i][j] > 0 else acc - t)
            if self.octonion_gpu:
                acc = acc.to(torch.bfloat16).to(self.dt)
            ys.append(acc * self.sd[p + '.beta'])
        return torch.cat(ys, dim=-1)

    def linear(self, x, p):
        """The algebra's ternary linear of module ``p`` (chassis.py:54-65)."""
        if self.algebra == "hadamard":
            return self.hadamard_linear(x, p + '.inner')
        return self.octonion_linear(x, p)

    def mapping(self, x_flat, p, kind):
        """mhc.py:283-318."""
        n = self.n
        xn = F.rms_norm(x_flat, (x_flat.size(-1),))
        dyn = xn @ self.sd[p + '.phi.weight'].t()
        a = self.sd[p + '.alpha']
        b = self.sd[p + '.bias']
        if kind == 'res':
            h = a * dyn.view(*dyn.shape[:-1], n, n) + b
            M = torch.exp(h)
            for _ in range(20):
                M = M / (M.sum(dim=-2, keepdim=True) + 1e-8)
                M = M / (M.sum(dim=-1, keepdim=True) + 1e-8)
            return M
        s = torch.sigmoid(a * dyn + b).unsqueeze(-2)
        return s if kind == 'pre' else 2.0 * s

    def stream(self, x, p, layer_fn):
        """mhc.py:345-381; x [B, T, n, C]."""
        B, T, n, C = x.shape
        xf = x.reshape(B, T, n * C)
        hp = self.mapping(xf, p + '.H_pre', 'pre')
        hq = self.mapping(xf, p + '.H_post', 'post')
        hr = self.mapping(xf, p + '.H_res', 'res')
        li = torch.matmul(hp, x).squeeze(2)
        out = layer_fn(li)
        return torch.matmul(hr, x) + torch.matmul(hq.transpose(-2, -1), out.unsqueeze(2))

    def moe(self, x, p):
        """moe.py:418-447, 337-380, 512-542 (top-k routing, all-expert einsum)."""
        B, T, C = x.shape
        h = F.silu(x @ self.sd[p + '.router.gate.0.weight'].t())
        logits = h @ self.sd[p + '.router.gate.2.weight'].t()
        probs = F.softmax(logits, dim=-1)
        E = probs.shape[-1]
        k = min(self.moe_k, E)
        _, idx = probs.topk(k, dim=-1)
        mask = torch.zeros_like(probs).scatter_(-1, idx, 1.0)
        mp = probs * mask
        wts = mp / mp.sum(-1, keepdim=True).clamp(min=1e-8)

        q = self.moe_quantized
        xb = x.view(B, T, E, C // E)
        g = torch.einsum('bted,ehd->bteh', xb, q(p + '.experts.gate_weights'))
        u = torch.einsum('bted,ehd->bteh', xb, q(p + '.experts.up_weights'))
        out = torch.einsum('bteh,edh->bted', F.silu(g) * u, q(p + '.experts.down_weights'))
        return (out * wts.unsqueeze(-1)).reshape(B, T, C), dict(probs=probs, mask=mask, weights=wts, idx=idx)

    def moe_quantized(self, key):
        """quantize_ternary of moe.py:276-303: clamp(round(w/g), -1, 1)*g."""
        w = self.sd[key]
        if self.grad:
            return _MoESTE.apply(w)
        g = w.abs().mean() + 1e-8
        return torch.clamp(torch.round(w / g), -1, 1) * g

    def channel_mod(self, x, p, n_blocks=None, residual_scale=0.5):
        """HadamardChannelModulation.forward with the ternary MLP
        (moe.py:676-727, :753-762) and the per-block modulation of
        _forward_pytorch (:729-744); x [G, T, C]."""
        G, T, C = x.shape
        nb = n_blocks or C // 32
        q = self.moe_quantized
        bulk = x.mean(dim=1)
        h = F.silu(bulk @ q(p + '.context_mlp.0.weight').t())
        mods = h @ q(p + '.context_mlp.2.weight').t()
        raw, shift = mods.chunk(2, dim=-1)
        scale = 1.0 + torch.clamp(self.sd[p + '.scale_temp'], 0.1, 0.5) * torch.tanh(raw)
        xb = x.view(G, T, nb, C // nb)
        xm = xb * scale.view(G, 1, nb, 1) + shift.view(G, 1, nb, 1) * 0.1
        return (xb + residual_scale * (xm - xb)).view(G, T, C)

    # ---------------------------------------------------------------- harness
    def rmsnorm(self, x, w, eps=1e-6):
        xf = x.to(self.dt)
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)) * w

    def rope(self, xq, xk, freqs):
        xq_ = torch.view_as_complex(xq.to(self.dt).reshape(*xq.shape[:-1], -1, 2))
        xk_ = torch.view_as_complex(xk.to(self.dt).reshape(*xk.shape[:-1], -1, 2))
        f = freqs[:xq.shape[1]].unsqueeze(0).unsqueeze(2)
        return torch.view_as_real(xq_ * f).flatten(3), torch.view_as_real(xk_ * f).flatten(3)

    def head_mixer(self, y, p):
        if self.algebra != "hadamard":
            # OctonionHeadMixer (chassis.py:375-399): y_i = beta *
            # sum_j S[i][j] heads_j @ W[i^j] (W not transposed)
            W = self.sd[p + '.W']
            out = []
            for i in range(8):
                acc = torch.zeros_like(y[:, 0])
                for j in range(8):
                    acc = acc + OCT_SIGN[i][j] * (y[:, j] @ W[i ^ j])
                out.append(acc * self.sd[p + '.beta'])
            return torch.stack(out, dim=1)
        xf = torch.einsum('bhti,hg->bgti', y, self.H)
        z = torch.einsum('bhti,hio->bhto', xf, self.sd[p + '.W'])
        zf = torch.einsum('bhti,hg->bgti', z, self.H)
        return zf * self.sd[p + '.beta']

    def attention(self, x, p, freqs):
        B, T, C = x.shape
        hd = C // self.n_head
        q = self.linear(x, p + '.wq').view(B, T, self.n_head, hd)
        k = self.linear(x, p + '.wk').view(B, T, self.n_head, hd)
        v = self.linear(x, p + '.wv').view(B, T, self.n_head, hd)
        q, k = self.rope(q, k, freqs)
        y = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), is_causal=True)
        if self.head_mixing:
            gsz = 32 if self.algebra == "hadamard" else 8
            ng = self.n_head // gsz
            yg = y.view(B, ng, gsz, T, hd)
            y = torch.cat([self.head_mixer(yg[:, g], p + '.head_mixer') for g in range(ng)], dim=1)
        y = y.transpose(1, 2).contiguous().view(B, T, C)
        return self.linear(y, p + '.wo')

    def swiglu(self, x, p):
        g = self.linear(x, p + '.gate_proj')
        u = self.linear(x, p + '.up_proj')
        return self.linear(F.silu(g) * u, p + '.down_proj')

    def block(self, h, l, freqs):
        """mHCLlamaBlock.forward (mhc.py:507-534) of layer l on the streams
        h [B, T, n, C] with the RoPE rows freqs [T, head_dim/2]."""
        sd = self.sd
        B, T = h.shape[0], h.shape[1]
        p = f'layers.{l}'
        h = self.stream(h, p + '.attn_stream',
                        lambda v: self.attention(self.rmsnorm(v, sd[p + '.attention_norm.weight']),
                                                 p + '.attention', freqs))
        if self.use_moe:
            ffn = lambda v: self.moe(self.rmsnorm(v, sd[p + '.ffn_norm.weight']), p + '.feed_forward')[0]  # noqa: E731
        else:
            ffn = lambda v: self.swiglu(self.rmsnorm(v, sd[p + '.ffn_norm.weight']), p + '.feed_forward')  # noqa: E731
        h = self.stream(h, p + '.ffn_stream', ffn)
        if self.use_channel_mod:
            # the [B*n, T, C] view of the streams (mhc.py:528-532)
            hf = h.reshape(B * self.n, T, self.C)
            hn = self.rmsnorm(hf, sd[p + '.channel_mod_norm.weight'])
            h = (hf + self.channel_mod(hn, p + '.channel_mod')).view(B, T, self.n, self.C)
        return h

    def loss(self, idx, targets):
        """mHCWalsh.forward's loss with targets (mhc.py:668-672): logits of
        every position, cross-entropy with ignore_index -1."""
        _, ho = self.forward(idx, return_hidden=True)
        logits = ho @ self.sd['output.weight'].t()
        return F.cross_entropy(logits.view(-1, logits.size(-1)), targets.view(-1), ignore_index=-1)

    def forward(self, idx, return_hidden=False):
        """Logits of the last position [B, 1, V] (mhc.py:617-681, targets=None)."""
        sd = self.sd
        B, T = idx.shape
        h = F.embedding(idx, sd['tok_embeddings.weight'])
        h = h @ sd['stream_proj.weight'].t() + sd['stream_proj.bias']
        h = h.view(B, T, self.n, self.C)
        freqs = sd['freqs_cis'][:T]
        for l in range(self.n_layer):
            h = self.block(h, l, freqs)
        hm = h.reshape(B, T, self.n * self.C) @ sd['stream_merge.weight'].t() + sd['stream_merge.bias']
        ho = self.rmsnorm(hm, sd['norm.weight'])
        logits = ho[:, [-1], :] @ sd['output.weight'].t()
        return (logits, ho) if return_hidden else logits
