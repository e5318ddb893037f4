"""bf16 parity at n_embd 4096 (config 5) and the reference's own model outputs.

* The reference fixtures of tests/golden (written from the reference's
  mHCWalsh on the CPU) loaded into the GPU model: float32 logits, hidden
  states and loss within 1e-5, MoE expert masks equal.
* The wide stream mapping (walsh_mhc_pre_wide_fwd: split-K projection, then
  per-token constraints, H_pre x and the RMSNorm) at n_embd 4096 in float32
  and bf16 with the row count straddling its chunk split, against the
  float64 mapping oracle on the rows at each chunk edge (mhc.py:283-318).
* Two config-5 layers (n_embd 4096, 32 heads of 128, MoE with 128 experts,
  k = 6, 4 streams) under bf16 autocast, and a cached bf16 decode at
  n_embd 4096, against the oracle in float32 and under CPU bf16 autocast.

bf16 bars.  A single kernel meets 1e-2 relative against float64 (the kernel
tests).  Through whole layers bf16 storage of the streams compounds; the
reference's own bf16 autocast path (the oracle run under CPU autocast)
drifts from float32 by d.  The GPU bf16 result must lie within
max(1e-2, 1.25 d) of float32 and within max(1e-2, 2 d) of the reference's
bf16 result (two independent bf16 roundings of the same computation).
With MoE layers a bf16 run may pick another expert set for a token whose
k-th and (k+1)-th router probabilities are near-equal; such a token's
hidden state then differs wholesale.  Those tokens are counted and each
must be a near tie in the float32 probabilities (relative gap < 2^-4 at
the layer where the runs first part); the hidden-state bars apply to the
tokens routed alike in every layer.
"""
import os

import numpy as np
import pytest
import torch

from oracle import mhc as omhc
from oracle.model import Oracle

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)), \
        float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def load(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _bf16_bars(d_ref):
    return max(1e-2, 1.25 * d_ref), max(1e-2, 2.0 * d_ref)


NEAR_TIE = 2.0 ** -4


def _routing_split(masks_a, masks_b, probs_ref, k):
    """Tokens routed to the same experts in every layer by runs a and b, and
    the tokens where they first part: for each such token the relative gap
    (p_k - p_k+1) / p_k of the reference probabilities at that layer (a
    bf16 run can only choose differently where that gap is within bf16's
    rounding of the router logits)."""
    n_tok = masks_a[0].shape[0]
    same = np.ones(n_tok, bool)
    gaps = []
    for ma, mb, p in zip(masks_a, masks_b, probs_ref):
        differ = (ma != mb).any(-1)
        first = differ & same
        ps = -np.sort(-np.asarray(p, np.float64), axis=-1)
        gap = (ps[:, k - 1] - ps[:, k]) / ps[:, k - 1]
        gaps += list(gap[first])
        same &= ~differ
    return same, np.array(gaps)


# --------------------------------------------------------------- reference fixtures
@pytest.mark.parametrize("name", ["model_c64.npz", "model_c96_moe.npz"])
def test_reference_fixture_model_on_gpu(name):
    """The reference's state dict (a drop-in load) and tokens give the
    reference's logits on the GPU: float32 within 1e-5 (last position, every
    position's hidden state, the loss), equal expert masks; bf16 autocast
    within the bf16 bars of the reference's own bf16 drift."""
    from src.model import WalshConfig, mHCWalsh
    fx = load(name)
    c = {k[4:]: (str(v) if v.dtype.kind == "U" else int(v)) for k, v in fx.items() if k.startswith("cfg/")}
    cfg = WalshConfig(block_size=c["block_size"], vocab_size=c["vocab"], n_layer=c["n_layer"], n_head=c["n_head"],
                      n_embd=c["n_embd"], algebra="hadamard", head_mixing=bool(c["head_mixing"]),
                      use_moe=bool(c["use_moe"]), moe_max_experts=c["max_experts"],
                      use_channel_mod=bool(c["use_channel_mod"]))
    model = mHCWalsh(cfg, n_streams=4)
    sd = {k[3:]: torch.from_numpy(v.copy()) for k, v in fx.items() if k.startswith("sd/")}
    model.load_state_dict(sd, strict=True)
    model = model.cuda().eval()
    idx = torch.from_numpy(fx["in/idx"]).cuda()
    targets = torch.from_numpy(fx["in/targets"]).cuda()
    with torch.no_grad():
        logits, _, h = model(idx, return_hidden=True)
        masks = [layer.feed_forward._last_expert_mask.cpu().numpy() for layer in model.layers] if c["use_moe"] else []
        _, loss = model(idx, targets=targets)
    rl, rh = rel(logits.cpu(), fx["out/logits_last"]), rel(h.cpu(), fx["out/h_out"])
    print(f"{name} fp32: logits {rl}, hidden {rh}, loss {float(loss):.7f} vs {float(fx['out/loss']):.7f}")
    assert max(rl) <= 1e-5 and max(rh) <= 1e-5
    assert abs(float(loss) - float(fx["out/loss"])) <= 1e-5 * abs(float(fx["out/loss"]))
    for l, m in enumerate(masks):
        assert np.array_equal(m, fx[f"out/moe_mask_{l}"]), f"layer {l} expert mask"

    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        lb, _, hb = model(idx, return_hidden=True)
        gmasks = [layer.feed_forward._last_expert_mask.cpu().numpy().reshape(-1, c["n_embd"] // 32)
                  for layer in model.layers] if c["use_moe"] else []
    orc = Oracle({k: v for k, v in sd.items()}, c["n_embd"], c["n_head"], c["n_layer"],
                 head_mixing=bool(c["head_mixing"]), use_moe=bool(c["use_moe"]), moe_max_experts=c["max_experts"],
                 use_channel_mod=bool(c["use_channel_mod"]))
    rmasks, rprobs = {"fp32": [], "bf16": []}, {"fp32": [], "bf16": []}
    if c["use_moe"]:
        moe = orc.moe

        def traced(x, p, key):
            out, info = moe(x, p)
            rmasks[key].append(info["mask"].float().numpy().reshape(x.shape[0] * x.shape[1], -1))
            rprobs[key].append(info["probs"].float().numpy().reshape(x.shape[0] * x.shape[1], -1))
            return out, info
        orc.moe = lambda x, p: traced(x, p, "fp32")
        with torch.no_grad():
            orc.forward(idx.cpu())
        orc.moe = lambda x, p: traced(x, p, "bf16")
    with torch.no_grad(), torch.autocast("cpu", dtype=torch.bfloat16):
        rb_l, rb_h = orc.forward(idx.cpu(), return_hidden=True)
    h32 = fx["out/h_out"].reshape(-1, c["n_embd"])
    hg = hb.float().cpu().numpy().reshape(h32.shape)
    hr = rb_h.float().numpy().reshape(h32.shape)
    keep = np.ones(h32.shape[0], bool)
    if c["use_moe"]:
        k = min(c["max_experts"], c["n_embd"] // 32)
        same_g, gaps_g = _routing_split(gmasks, rmasks["fp32"], rprobs["fp32"], k)
        same_r, gaps_r = _routing_split(rmasks["bf16"], rmasks["fp32"], rprobs["fp32"], k)
        keep = same_g & same_r
        print(f"{name} routing vs float32: GPU bf16 parts on {len(gaps_g)}/{len(keep)} tokens (max relative gap "
              f"{gaps_g.max(initial=0):.2e}), reference bf16 on {len(gaps_r)} (max {gaps_r.max(initial=0):.2e})")
        assert np.all(gaps_g < NEAR_TIE), gaps_g
        assert keep.sum() >= len(keep) // 2
    d_ref = rel(hr[keep], h32[keep])[0]
    d_gpu = rel(hg[keep], h32[keep])[0]
    d_pair = rel(hg[keep], hr[keep])[0]
    bar32, bar_pair = _bf16_bars(d_ref)
    print(f"{name} bf16 hidden over {int(keep.sum())}/{len(keep)} tokens: GPU vs reference fp32 {d_gpu:.3e} "
          f"(bar {bar32:.3e}); reference bf16 vs fp32 {d_ref:.3e}; GPU bf16 vs reference-style bf16 {d_pair:.3e} "
          f"(bar {bar_pair:.3e})")
    assert d_gpu <= bar32 and d_pair <= bar_pair


# --------------------------------------------------------------- wide mapping
def _chunk_rows(M, ld_bytes, align=16):
    """Rows per launch of walsh_mhc_pre_wide_fwd: buffers stay below 2^31
    bytes, split into equal multiples of 16 rows."""
    rows_max = (0x7FFFFFFF // ld_bytes) // align * align
    if M <= rows_max:
        return rows_max
    n = -(-M // rows_max)
    r = -(-(-(-M // n)) // align) * align
    return min(r, rows_max)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_mhc_pre_wide_vs_oracle_across_chunks(dtype):
    from src.model import kernels
    from src.model.chassis import RMSNorm
    from src.model.mhc import mHCResidualStream, _rms_eps
    n, C = 4, 4096
    esz = 4 if dtype == torch.float32 else 2
    rows_max = (0x7FFFFFFF // (n * C * esz)) // 16 * 16
    M = rows_max + 48                       # two chunks
    chunk = _chunk_rows(M, n * C * esz)
    assert M > chunk
    torch.manual_seed(4)
    stream = mHCResidualStream(C, n).cuda()
    norm = RMSNorm(C).cuda()
    g = torch.Generator().manual_seed(9)
    with torch.no_grad():
        for m in (stream.H_pre, stream.H_post, stream.H_res):
            m.alpha.fill_(0.5)
            m.bias.add_(0.5 * torch.randn(m.bias.shape, generator=g).cuda())
            m.phi.weight.copy_(0.02 * torch.randn(m.phi.weight.shape, generator=g))
        norm.weight.mul_(1 + 0.2 * torch.randn(C, generator=g).cuda())
    gdev = torch.Generator(device="cuda").manual_seed(11)
    x = torch.randn(M, n, C, device="cuda", generator=gdev).to(dtype)
    _, coef, bias, frag = stream.fused_params(dtype, x.device)
    with torch.no_grad():
        li, hp, hq, hr = kernels.mhc_pre_wide(x, frag, coef, bias, _rms_eps(dtype), norm_w=norm.weight, norm_eps=1e-6)
    torch.cuda.synchronize()
    rows = sorted(set(list(range(0, 16)) + list(range(chunk - 16, chunk + 16)) + list(range(M - 16, M))))
    ri = torch.tensor(rows, device="cuda")
    xs = x.index_select(0, ri).float().cpu().numpy().astype(np.float64)
    maps = {k: (getattr(stream, f"H_{k}").phi.weight.detach().cpu().numpy(),
                float(getattr(stream, f"H_{k}").alpha), getattr(stream, f"H_{k}").bias.detach().cpu().numpy())
            for k in ("pre", "post", "res")}
    eps = omhc.rms_eps(np.float32 if dtype == torch.float32 else "bfloat16")
    _, o_hp, o_hq, o_hr, o_li = omhc.stream_forward(xs, maps, lambda v: v, eps)
    w = norm.weight.detach().cpu().numpy().astype(np.float64)
    o_li = o_li / np.sqrt((o_li * o_li).mean(-1, keepdims=True) + 1e-6) * w
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    got = dict(pre=hp.index_select(0, ri).cpu().numpy().reshape(o_hp.shape),
               post=hq.index_select(0, ri).cpu().numpy().reshape(o_hq.shape),
               res=hr.index_select(0, ri).cpu().numpy(),
               layer_in=li.index_select(0, ri).float().cpu().numpy())
    ref = dict(pre=o_hp, post=o_hq, res=o_hr, layer_in=o_li)
    for k in got:
        r = rel(got[k], ref[k])
        print(f"{dtype} M={M} (chunks of {chunk}) {k}: rel {r}")
        assert r[0] <= tol and r[1] <= 10 * tol, k
    # the chunk edge itself: rows chunk-1 and chunk are checked row by row
    for j in (rows.index(chunk - 1), rows.index(chunk)):
        assert rel(got["layer_in"][j], ref["layer_in"][j])[0] <= tol


@pytest.mark.parametrize("M,n,C", [(1, 4, 4096), (100, 4, 4096), (2051, 4, 4096), (40, 3, 96), (7, 2, 64),
                                   (65568, 4, 4096)])
def test_mhc_post_pre_wide_equals_separate_kernels(M, n, C):
    """The stream update fused into the wide mapping's projection launch
    (walsh_mhc_post_pre_wide_fwd, bf16): x_new bitwise walsh_mhc_post_fwd's
    result; the mappings and layer input those of walsh_mhc_pre_wide_fwd on
    that x_new (pinned against the oracle above) up to the projection's
    float32 summation order (it runs column-major over the streams).
    M=1 and 100 take many column splits, 2051 a ragged last tile, 65568 two
    row chunks (x_new rows of 32 KiB)."""
    from src.model import kernels
    from src.model.chassis import RMSNorm
    from src.model.mhc import mHCResidualStream, _rms_eps
    dtype = torch.bfloat16
    print(f"post+pre wide M={M} n={n} C={C}", flush=True)
    torch.manual_seed(M + n + C)
    stream = mHCResidualStream(C, n).cuda()
    norm = RMSNorm(C).cuda()
    g = torch.Generator().manual_seed(M * 3 + C)
    with torch.no_grad():
        for m in (stream.H_pre, stream.H_post, stream.H_res):
            m.alpha.fill_(0.5)
            m.bias.add_(0.5 * torch.randn(m.bias.shape, generator=g).cuda())
            m.phi.weight.copy_(0.02 * torch.randn(m.phi.weight.shape, generator=g))
        norm.weight.mul_(1 + 0.2 * torch.randn(C, generator=g).cuda())
    gdev = torch.Generator(device="cuda").manual_seed(M + 7)
    x_old = torch.randn(M, n, C, device="cuda", generator=gdev).to(dtype)
    out = torch.randn(M, C, device="cuda", generator=gdev).to(dtype)
    h_res_prev = torch.rand(M, n, n, device="cuda", generator=gdev) * 0.5
    h_post_prev = torch.rand(M, n, device="cuda", generator=gdev) * 2
    _, coef, bias, frag = stream.fused_params(dtype, x_old.device)
    assert frag.numel() == 32 * n * C and kernels.mhc_pre_wide_supported(n, C)
    eps = _rms_eps(dtype)
    with torch.no_grad():
        x_new, li, hp, hq, hr = kernels.mhc_post_pre_wide(x_old, out, h_res_prev, h_post_prev, frag, coef, bias, eps,
                                                          norm_w=norm.weight, norm_eps=1e-6)
        x_ref = kernels.mhc_post(x_old, out, h_res_prev, h_post_prev)
        li_r, hp_r, hq_r, hr_r = kernels.mhc_pre_wide(x_ref, frag, coef, bias, eps, norm_w=norm.weight,
                                                       norm_eps=1e-6)
    torch.cuda.synchronize()
    assert torch.equal(x_new, x_ref)
    for name, a, b in (("h_pre", hp, hp_r), ("h_post", hq, hq_r), ("h_res", hr, hr_r)):
        d = (a - b).abs().max().item()
        assert d <= 2e-5, f"{name}: max |diff| {d:.3e}"
    # layer_in: bf16 values, a last-place difference where the float32 sums
    # straddle a rounding boundary (2^-7 relative covers one bf16 ulp)
    lf, lr = li.float(), li_r.float()
    d = ((lf - lr).abs() / lr.abs().clamp_min(1e-3)).max().item()
    assert d <= 2 ** -7, f"layer_in: max rel diff {d:.3e}"


# --------------------------------------------------------------- config-5 layers
def _make5(n_layer, block=64, seed=5, vocab=1000):
    from src.model import WalshConfig, mHCWalsh
    torch.manual_seed(seed)
    cfg = WalshConfig(block_size=block, vocab_size=vocab, n_layer=n_layer, n_head=32, n_embd=4096,
                      algebra="hadamard", head_mixing=True, use_moe=True, moe_max_experts=6, use_channel_mod=False)
    model = mHCWalsh(cfg, n_streams=4)
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith(('.alpha', '.beta', 'norm.weight')) and p.dim() > 0:
                p.mul_(1 + 0.2 * torch.randn(p.shape, generator=g))
            elif name.endswith('.alpha'):   # mapping gains
                p.fill_(0.3)
    return cfg, model.cuda().eval()


def test_config5_layers_bf16_vs_oracle():
    """Two config-5 layers under bf16 autocast (48 tokens) against the oracle
    in float32 and under CPU bf16 autocast.  Expert selections are compared
    token by token: a token whose selection first differs from float32's
    must be a near tie there (relative gap of the k-th and (k+1)-th
    probabilities below 2^-4); the hidden states are compared over the
    tokens routed alike in every layer by all three runs, with the bf16
    bars; the last-position logits with the same bars."""
    cfg, model = _make5(2)
    idx = torch.randint(0, cfg.vocab_size, (1, 48), generator=torch.Generator().manual_seed(3))
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        lg, _, h = model(idx.cuda(), return_hidden=True)
        gpu_masks = [layer.feed_forward._last_expert_mask.cpu().numpy().reshape(-1, 128) for layer in model.layers]
    sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    orc = Oracle(sd, 4096, 32, 2, n_streams=4, use_moe=True, moe_max_experts=6)
    masks = {"fp32": [], "bf16": []}
    probs = {"fp32": [], "bf16": []}
    moe = orc.moe

    def traced(x, p, key):
        out, info = moe(x, p)
        masks[key].append(info["mask"].float().numpy().reshape(-1, 128))
        probs[key].append(info["probs"].float().numpy().reshape(-1, 128))
        return out, info
    with torch.no_grad():
        orc.moe = lambda x, p: traced(x, p, "fp32")
        ref_l, ref_h = orc.forward(idx, return_hidden=True)
        orc.moe = lambda x, p: traced(x, p, "bf16")
        with torch.autocast("cpu", dtype=torch.bfloat16):
            rb_l, rb_h = orc.forward(idx, return_hidden=True)
    same_g, gaps_g = _routing_split(gpu_masks, masks["fp32"], probs["fp32"], 6)
    same_r, gaps_r = _routing_split(masks["bf16"], masks["fp32"], probs["fp32"], 6)
    keep = same_g & same_r
    hg, h32, hb = (t.float().cpu().numpy().reshape(48, -1) for t in (h, ref_h, rb_h))
    d_ref = rel(hb[keep], h32[keep])[0]
    d_gpu = rel(hg[keep], h32[keep])[0]
    d_pair = rel(hg[keep], hb[keep])[0]
    dl_gpu = rel(lg.float().cpu(), ref_l)[0]
    dl_ref = rel(rb_l.float(), ref_l)[0]
    bar32, bar_pair = _bf16_bars(d_ref)
    print(f"routing vs float32: GPU bf16 parts on {len(gaps_g)}/48 tokens (max relative gap {gaps_g.max(initial=0):.2e}), "
          f"reference bf16 on {len(gaps_r)}/48 (max gap {gaps_r.max(initial=0):.2e}); band {NEAR_TIE:.2e}")
    print(f"config-5 x2 bf16 hidden over the {int(keep.sum())} tokens routed alike: GPU vs fp32 {d_gpu:.3e} "
          f"(bar {bar32:.3e}); reference bf16 vs fp32 {d_ref:.3e}; GPU vs reference bf16 {d_pair:.3e} "
          f"(bar {bar_pair:.3e}); last-position logits GPU {dl_gpu:.3e}, reference bf16 {dl_ref:.3e}")
    assert np.all(gaps_g < NEAR_TIE), gaps_g
    assert keep.sum() >= 24
    assert d_gpu <= bar32 and d_pair <= bar_pair
    assert dl_gpu <= max(1e-2, 1.25 * dl_ref)


def test_config5_cached_decode_bf16_vs_oracle():
    """Prefill 8 tokens into the bf16 KV cache, then 3 single-token steps at
    batch 2 (n_embd 4096, MoE 128 experts): each step's logits against the
    oracle's uncached last-position logits in float32 and under CPU bf16
    autocast."""
    from src.model import KVCache
    cfg, model = _make5(1, seed=8)
    B, T0, steps = 2, 8, 3
    idx = torch.randint(0, cfg.vocab_size, (B, T0 + steps), generator=torch.Generator().manual_seed(7))
    kv = KVCache(1, cfg.block_size, 32, 128, torch.device("cuda"), dtype=torch.bfloat16, batch=B)
    sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    orc = Oracle(sd, 4096, 32, 1, n_streams=4, use_moe=True, moe_max_experts=6)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        model(idx[:, :T0].cuda(), kv_cache=kv, start_pos=0)
        kv.increment(T0)
        for s in range(steps):
            pos = T0 + s
            lg, _ = model(idx[:, pos:pos + 1].cuda(), kv_cache=kv, start_pos=pos)
            kv.increment(1)
            with torch.autocast("cuda", enabled=False):
                ref = orc.forward(idx[:, :pos + 1])
                with torch.autocast("cpu", dtype=torch.bfloat16):
                    refb = orc.forward(idx[:, :pos + 1])
            d_gpu = rel(lg[:, -1].float().cpu(), ref[:, -1])[0]
            d_ref = rel(refb[:, -1].float(), ref[:, -1])[0]
            d_pair = rel(lg[:, -1].float().cpu(), refb[:, -1].float())[0]
            bar32, bar_pair = _bf16_bars(d_ref)
            print(f"step {s} (KV {pos + 1}): GPU cached bf16 vs fp32 {d_gpu:.3e} (bar {bar32:.3e}); reference bf16 "
                  f"vs fp32 {d_ref:.3e}; GPU vs reference bf16 {d_pair:.3e} (bar {bar_pair:.3e})")
            assert d_gpu <= bar32 and d_pair <= bar_pair
