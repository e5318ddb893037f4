"""GPU parity of channel modulation (walsh_chanmod_fwd / _apply / _bwd and
the modules built on them) against oracle/channel_mod.py and the model
oracle.  Bars: max|d| / max|ref| and ||d|| / ||ref|| <= 1e-5 in float32,
1e-2 in bfloat16 (bf16 inputs rounded before the oracle runs)."""
import numpy as np
import pytest
import torch

from oracle import channel_mod as ocm

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2}


def assert_close(y, ref, tol, what=""):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    d = y - ref
    n, m = np.linalg.norm(ref), np.abs(ref).max()
    r_norm = np.linalg.norm(d) / n if n > 0 else np.linalg.norm(d)
    r_max = np.abs(d).max() / m if m > 0 else np.abs(d).max()
    print(f"{what} rel_norm={r_norm:.3e} rel_max={r_max:.3e} tol={tol}", flush=True)
    assert r_norm <= tol and r_max <= tol, (what, r_norm, r_max)


@pytest.fixture(scope="module")
def K():
    from src.model import kernels
    return kernels


def _np(t):
    return t.detach().double().cpu().numpy()


# (G, T, C, n_blocks): block dims 32, 64, 16, 128; T = 1 is the decode shape
SHAPES = [(2, 5, 64, 2), (4, 1, 512, 16), (3, 100, 512, 8), (2, 37, 96, 6), (1, 300, 4096, 32), (32, 256, 512, 16)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("G,T,C,nb", SHAPES)
@pytest.mark.parametrize("fused", [False, True])
def test_chanmod_fwd_vs_oracle(K, G, T, C, nb, dtype, fused):
    print(f"chanmod fwd G={G} T={T} C={C} nb={nb} {dtype} fused={fused}", flush=True)
    g = torch.Generator().manual_seed(G * 1000 + T + C)
    x = torch.randn(G, T, C, generator=g)
    if not fused:
        x = x * 0.5
    w1 = torch.randn(C // 4, C, generator=g) * 0.05
    w2 = torch.randn(2 * nb, C // 4, generator=g) * 0.3
    nw = 1 + 0.2 * torch.randn(C, generator=g)
    temp = torch.tensor([0.35])
    xd = x.to(dtype).cuda()
    w1q, w2q = ocm.mlp_weights(w1.numpy(), w2.numpy(), True)
    w1d = torch.tensor(w1q, dtype=torch.float32).cuda()
    w2d = torch.tensor(w2q, dtype=torch.float32).cuda()
    if fused:
        y, ss = K.chanmod_fwd(xd, w1d, w2d, temp.cuda(), nb, 0.5, norm_w=nw.cuda(), eps=1e-6, add_input=True)
        ref, scale, shift = ocm.block_residual(_np(xd), nw.numpy(), w1q, w2q, 0.35, nb, 0.5, use_ternary=False)
    else:
        y, ss = K.chanmod_fwd(xd, w1d, w2d, temp.cuda(), nb, 0.5)
        ref, scale, shift = ocm.channel_mod(_np(xd), w1q, w2q, 0.35, nb, 0.5, use_ternary=False)
    torch.cuda.synchronize()
    assert y.dtype == dtype and y.shape == (G, T, C)
    ssn = _np(ss)
    assert_close(ssn[:, :nb], scale, 1e-5, "scale")
    assert_close(ssn[:, nb:], shift, 1e-5, "shift")
    assert_close(_np(y), ref, TOL[dtype], "y")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_chanmod_fwd_strided_rows_and_determinism(K, dtype):
    """Rows with a padded stride read the same as the packed rows; two calls
    give identical bits (fixed-order sums)."""
    G, T, C, nb = 3, 70, 256, 8
    g = torch.Generator().manual_seed(7)
    base = torch.randn(G, T, C + 12, generator=g).to(dtype).cuda()
    x = base[..., :C]
    w1 = (torch.randn(C // 4, C, generator=g) * 0.05).cuda()
    w2 = (torch.randn(2 * nb, C // 4, generator=g) * 0.3).cuda()
    temp = torch.tensor([0.2]).cuda()
    y1, s1 = K.chanmod_fwd(x, w1, w2, temp, nb, 0.5)
    y2, s2 = K.chanmod_fwd(x.contiguous(), w1, w2, temp, nb, 0.5)
    y3, s3 = K.chanmod_fwd(x, w1, w2, temp, nb, 0.5)
    assert torch.equal(y1, y2) and torch.equal(s1, s2)
    assert torch.equal(y1, y3) and torch.equal(s1, s3)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("G,T,C,nb", [(2, 5, 64, 2), (3, 100, 512, 8), (2, 37, 96, 6), (1, 64, 4096, 32)])
def test_chanmod_apply_and_bwd_vs_oracle(K, G, T, C, nb, dtype):
    print(f"chanmod apply/bwd G={G} T={T} C={C} nb={nb} {dtype}", flush=True)
    g = torch.Generator().manual_seed(11 + C)
    x = torch.randn(G, T, C, generator=g).to(dtype).cuda()
    scale = (1 + 0.4 * torch.rand(G, nb, generator=g) - 0.2).cuda()
    shift = torch.randn(G, nb, generator=g).cuda()
    gy = torch.randn(G, T, C, generator=g).to(dtype).cuda()
    y = K.chanmod_apply(x, scale, shift, 0.5)
    assert_close(_np(y), ocm.modulate(_np(x), _np(scale), _np(shift), 0.5), TOL[dtype], "apply")
    gx, ds, dh = K.chanmod_bwd(gy, x, scale, 0.5)
    rgx, rds, rdh = ocm.modulate_bwd(_np(gy), _np(x), _np(scale), 0.5)
    assert_close(_np(gx), rgx, TOL[dtype], "gx")
    # the sums are float32 over T*C/nb products of the (rounded) inputs
    assert_close(_np(ds), rds, 1e-5, "dscale")
    assert_close(_np(dh), rdh, 1e-5, "dshift")
    gx2, ds2, dh2 = K.chanmod_bwd(gy, x, scale, 0.5)
    assert torch.equal(gx, gx2) and torch.equal(ds, ds2) and torch.equal(dh, dh2)


def test_chanmod_empty_and_errors(K):
    from src.model._hip import WalshHipError
    x = torch.zeros(0, 5, 64, device="cuda")
    w1 = torch.zeros(16, 64, device="cuda")
    w2 = torch.zeros(4, 16, device="cuda")
    temp = torch.ones(1, device="cuda")
    y, ss = K.chanmod_fwd(x, w1, w2, temp, 2, 0.5)
    assert y.shape == (0, 5, 64)
    gx, ds, dh = K.chanmod_bwd(torch.zeros(2, 0, 64, device="cuda"), torch.zeros(2, 0, 64, device="cuda"),
                               torch.ones(2, 2, device="cuda"), 0.5)
    torch.cuda.synchronize()
    assert gx.shape == (2, 0, 64) and torch.equal(ds.cpu(), torch.zeros(2, 2)) and torch.equal(dh.cpu(), torch.zeros(2, 2))
    with pytest.raises(WalshHipError):   # C not a multiple of 4 (host-side check)
        K.chanmod_fwd(torch.zeros(1, 3, 6, device="cuda"), torch.zeros(1, 6, device="cuda"),
                      torch.zeros(2, 1, device="cuda"), temp, 1, 0.5)
    with pytest.raises(WalshHipError):   # n_blocks does not divide C
        K.chanmod_fwd(torch.zeros(1, 3, 64, device="cuda"), w1, torch.zeros(6, 16, device="cuda"), temp, 3, 0.5)


def _module_oracle(mod, prefix="cm"):
    """State dict of a HadamardChannelModulation under ``prefix`` for the model oracle."""
    return {f"{prefix}.{k}": v.detach().float().cpu() for k, v in mod.state_dict().items()}


@pytest.mark.parametrize("use_ternary", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_module_forward_and_stats(dtype, use_ternary):
    from src.model.moe import HadamardChannelModulation
    torch.manual_seed(0)
    C, B, T = 512, 3, 64
    mod = HadamardChannelModulation(n_embd=C, use_ternary=use_ternary, residual_scale=0.5).cuda()
    with torch.no_grad():
        mod.context_mlp[2].weight.mul_(30)   # visible modulation
        mod.scale_temp.fill_(0.3)
    x = torch.randn(B, T, C).to(dtype).cuda()
    with torch.no_grad():
        y = mod(x)
    torch.cuda.synchronize()
    w1 = mod.context_mlp[0].weight.detach().cpu().numpy()
    w2 = mod.context_mlp[2].weight.detach().cpu().numpy()
    ref, scale, shift = ocm.channel_mod(_np(x), w1, w2, 0.3, C // 32, 0.5, use_ternary)
    assert y.dtype == dtype
    assert_close(_np(y), ref, TOL[dtype], "module")
    st = mod.get_modulation_stats()
    assert abs(st['scale_mean'] - scale.mean()) <= 1e-5 * abs(scale.mean())
    assert abs(st['scale_std'] - scale.std(ddof=1)) <= 1e-4 * scale.std(ddof=1)
    assert abs(st['shift_mean'] - np.abs(shift).mean()) <= 1e-4 * np.abs(shift).mean()
    assert st['scale_temp'] == pytest.approx(0.3)


def test_module_autograd_vs_oracle():
    """Training path: gradients of x, both MLP weights (through the MoE STE)
    and scale_temp against float64 autograd of the model oracle's
    restatement."""
    from oracle.model import Oracle
    from src.model.moe import HadamardChannelModulation
    torch.manual_seed(1)
    C, B, T = 256, 2, 40
    mod = HadamardChannelModulation(n_embd=C, residual_scale=0.5).cuda()
    with torch.no_grad():
        mod.context_mlp[2].weight.mul_(30)
        mod.scale_temp.fill_(0.3)
    x = torch.randn(B, T, C).cuda().requires_grad_(True)
    gy = torch.randn(B, T, C)
    y = mod(x)
    (y * gy.cuda()).sum().backward()
    torch.cuda.synchronize()
    orc = Oracle(_module_oracle(mod), C, 1, 0, grad=True)
    xr = x.detach().double().cpu().requires_grad_(True)
    yr = orc.channel_mod(xr, "cm")
    (yr * gy.double()).sum().backward()
    assert_close(_np(y), _np(yr), 1e-5, "y")
    assert_close(_np(x.grad), _np(xr.grad), 1e-5, "dx")
    for name, p in mod.named_parameters():
        assert_close(_np(p.grad), _np(orc.sd["cm." + name].grad), 1e-4, "d" + name)


def test_block_fused_residual_matches_module():
    """HadamardChannelModulationBlock (moe.py:774-798): x + cm(norm(x)) in one
    fused call equals the two-step composition through the oracle."""
    from src.model import WalshConfig
    from src.model.moe import HadamardChannelModulationBlock
    torch.manual_seed(2)
    cfg = WalshConfig(n_embd=512, n_head=32, n_layer=1, vocab_size=256, block_size=64)
    blk = HadamardChannelModulationBlock(cfg).cuda()
    with torch.no_grad():
        blk.channel_mod.context_mlp[2].weight.mul_(30)
        blk.norm.weight.mul_(1.3)
    x = torch.randn(2, 33, 512).cuda()
    with torch.no_grad():
        y = blk(x)
    cm = blk.channel_mod
    ref, _, _ = ocm.block_residual(_np(x), _np(blk.norm.weight), cm.context_mlp[0].weight.detach().cpu().numpy(),
                                   cm.context_mlp[2].weight.detach().cpu().numpy(), 1.0, 8, 0.1, True)
    assert_close(_np(y), ref, 1e-5, "block")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_mhcwalsh_channel_mod_forward_vs_oracle(dtype):
    from oracle.model import Oracle
    from src.model import WalshConfig, mHCWalsh
    torch.manual_seed(0)
    C, n_layer, vocab, T = 256, 2, 512, 32
    cfg = WalshConfig(block_size=64, vocab_size=vocab, n_layer=n_layer, n_head=32, n_embd=C, algebra='hadamard',
                      head_mixing=True, use_channel_mod=True)
    model = mHCWalsh(cfg, n_streams=4).cuda().eval()
    with torch.no_grad():
        for l in model.layers:
            l.channel_mod.context_mlp[2].weight.mul_(30)
    idx = torch.randint(0, vocab, (2, T), generator=torch.Generator().manual_seed(3))
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=dtype == torch.bfloat16):
        logits, _, hidden = model(idx.cuda(), return_hidden=True)
    torch.cuda.synchronize()
    orc = Oracle(model.state_dict(), C, 32, n_layer, use_channel_mod=True)
    ref_logits, ref_hidden = orc.forward(idx, return_hidden=True)
    if dtype == torch.float32:
        assert_close(_np(hidden), _np(ref_hidden), 1e-4, "hidden")
    else:
        # bf16 storage compounds through the model: the whole-model bf16 bar
        # (no further from the float32 oracle than the oracle under bf16
        # autocast, the reference's own bf16 path, and never above
        # max(1e-2, that drift))
        with torch.autocast("cpu", dtype=torch.bfloat16):
            _, rb_hidden = orc.forward(idx, return_hidden=True)
        ref = _np(ref_hidden)
        rel = np.linalg.norm(_np(hidden) - ref) / np.linalg.norm(ref)
        drift = np.linalg.norm(_np(rb_hidden) - ref) / np.linalg.norm(ref)
        print(f"bf16 hidden rel_norm={rel:.2e} (reference-style bf16 {drift:.2e})", flush=True)
        assert rel <= max(1e-2, drift), (rel, drift)
    st = model.get_channel_mod_stats()
    assert set(st) == {'scale_mean', 'scale_std', 'shift_mean'} and st['scale_std'] > 0


def test_mhcwalsh_channel_mod_backward_vs_oracle():
    from oracle.model import Oracle
    from src.model import WalshConfig, mHCWalsh
    torch.manual_seed(0)
    C, n_layer, vocab, T = 64, 2, 256, 16
    cfg = WalshConfig(block_size=64, vocab_size=vocab, n_layer=n_layer, n_head=32, n_embd=C, algebra='hadamard',
                      head_mixing=True, use_channel_mod=True)
    model = mHCWalsh(cfg, n_streams=4).cuda().eval()
    with torch.no_grad():
        for l in model.layers:
            l.channel_mod.context_mlp[2].weight.mul_(30)
            l.channel_mod.scale_temp.fill_(0.3)   # inside the clamp: its gradient flows
    g = torch.Generator().manual_seed(1)
    idx = torch.randint(0, vocab, (2, T), generator=g)
    tgt = torch.randint(0, vocab, (2, T), generator=g)
    _, loss = model(idx.cuda(), targets=tgt.cuda())
    loss.backward()
    torch.cuda.synchronize()
    orc = Oracle(model.state_dict(), C, 32, n_layer, grad=True, use_channel_mod=True)
    ref_loss = orc.loss(idx, tgt)
    ref_loss.backward()
    assert abs(loss.item() - ref_loss.item()) <= 1e-5 * abs(ref_loss.item())
    got = {n: p.grad.double().cpu().numpy().ravel() for n, p in model.named_parameters()}
    ref = {n: orc.sd[n].grad.numpy().ravel() for n in got}
    allg = np.concatenate(list(got.values()))
    allr = np.concatenate(list(ref.values()))
    rel = np.linalg.norm(allg - allr) / np.linalg.norm(allr)
    Gmax = max(np.linalg.norm(v) for v in ref.values())
    bad = [(n, float(np.linalg.norm(got[n] - ref[n])), float(np.linalg.norm(ref[n]))) for n in got
           if np.linalg.norm(got[n] - ref[n]) > 1e-4 * np.linalg.norm(ref[n]) + 1e-6 * Gmax]
    print(f"channel-mod model backward: all-gradient rel_norm {rel:.2e}", flush=True)
    assert rel <= 1e-5, rel
    assert not bad, bad
    for n in ('layers.0.channel_mod.context_mlp.0.weight', 'layers.1.channel_mod.scale_temp',
              'layers.1.channel_mod_norm.weight'):
        assert np.linalg.norm(ref[n]) > 0, n
