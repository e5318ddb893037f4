"""GPU parity of the backward kernels against the oracle's gradients.

Hadamard linear (walsh_hadamard_linear_bwd): gx, dalpha, dbeta and the STE
weight gradient vs oracle.hadamard.hadamard_linear_bwd_f64 (itself pinned
against torch float64 autograd of the reference formula, a dense-matrix
transpose and finite differences).  Bars: ||d|| / ||ref|| and max|d| /
max|ref| <= 1e-5 in float32, 1e-2 in bfloat16 (inputs rounded to bf16
before the oracle runs).
"""
import numpy as np
import pytest
import torch

from oracle import hadamard as ohad

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2}


def assert_close(y, ref, dtype, what=""):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    d = y - ref
    n, m = np.linalg.norm(ref), np.abs(ref).max()
    r_norm = np.linalg.norm(d) / n if n > 0 else np.linalg.norm(d)
    r_max = np.abs(d).max() / m if m > 0 else np.abs(d).max()
    print(f"{what} rel_norm={r_norm:.3e} rel_max={r_max:.3e} tol={TOL[dtype]}", flush=True)
    assert r_norm <= TOL[dtype] and r_max <= TOL[dtype], (what, r_norm, r_max)


@pytest.fixture(scope="module")
def K():
    from src.model import kernels
    return kernels


def make_case(K, M, in_o, out_o, dtype, seed, big=False):
    gen = torch.Generator().manual_seed(seed)
    latent = ohad.init_weight(out_o, in_o, gen)
    if big:
        sel = torch.rand(latent.shape, generator=gen) < 0.2
        latent = torch.where(sel, latent.sign() * (1.5 + torch.rand(latent.shape, generator=gen)), latent)
    x = torch.randn(M, 32 * in_o, generator=gen).to(dtype)
    gy = torch.randn(M, 32 * out_o, generator=gen).to(dtype)
    alpha = 1 + 0.5 * torch.randn(32, in_o, generator=gen)
    beta = 0.3 * torch.randn(32, out_o, generator=gen)
    lc = latent.cuda()
    q = K.ternary_quantize(lc, codes=True, packed=True)
    kw = K.hadamard_prepare(q["packed"], in_o, out_o)
    kwt = K.hadamard_prepare_t(q["packed"], in_o, out_o)
    codes = q["codes"].cpu().numpy()
    return dict(x=x, gy=gy, alpha=alpha, beta=beta, latent=latent, lc=lc, kw=kw, kwt=kwt, codes=codes,
                packed=q["packed"])


SHAPES = [(16, 16, 300), (16, 16, 8192), (16, 64, 257), (64, 16, 100), (3, 5, 33), (20, 36, 50), (128, 128, 40),
          (1, 1, 17)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("in_o,out_o,M", SHAPES)
def test_hadamard_bwd_vs_oracle(K, in_o, out_o, M, dtype):
    print(f"case in_o={in_o} out_o={out_o} M={M} dtype={dtype}", flush=True)
    c = make_case(K, M, in_o, out_o, dtype, seed=in_o * 131 + out_o * 7 + M, big=(M % 2 == 1))
    gx, da, db, dw = K.hadamard_linear_bwd(c["x"].cuda(), c["gy"].cuda(), in_o, out_o, c["kw"], c["kwt"],
                                           c["alpha"].cuda(), c["beta"].cuda(), latent=c["lc"])
    torch.cuda.synchronize()
    ref = ohad.hadamard_linear_bwd_f64(c["x"].double().numpy(), c["codes"], c["alpha"].double().numpy(),
                                       c["beta"].double().numpy(), c["gy"].double().numpy(),
                                       latent=c["latent"].double().numpy())
    assert gx.dtype == dtype and gx.shape == c["x"].shape
    for name, got, r in (("gx", gx.float(), ref[0]), ("dalpha", da, ref[1]), ("dbeta", db, ref[2]),
                         ("dweight", dw, ref[3])):
        assert_close(got.cpu().numpy(), r, dtype, f"{name} {in_o}x{out_o} M={M}")


def test_hadamard_bwd_partial_outputs_and_determinism(K):
    c = make_case(K, 500, 16, 16, torch.bfloat16, seed=9)
    args = (c["x"].cuda(), c["gy"].cuda(), 16, 16, c["kw"], c["kwt"], c["alpha"].cuda(), c["beta"].cuda())
    full = K.hadamard_linear_bwd(*args, latent=c["lc"])
    again = K.hadamard_linear_bwd(*args, latent=c["lc"])
    for a, b in zip(full, again):
        assert torch.equal(a, b)  # fixed-order sums
    only_w = K.hadamard_linear_bwd(*args, latent=c["lc"], need=(False, False, False, True))
    assert only_w[0] is None and only_w[1] is None and only_w[2] is None
    assert torch.equal(only_w[3], full[3])
    only_a = K.hadamard_linear_bwd(*args, need=(False, True, False, False))
    assert torch.equal(only_a[1], full[1])
    only_x = K.hadamard_linear_bwd(*args, need=(True, False, False, False))
    assert torch.equal(only_x[0], full[0])
    # no latent: the raw gradient of the ternary matrix
    raw = K.hadamard_linear_bwd(*args, need=(False, False, False, True))[3]
    mask = (c["lc"] >= -1.5) & (c["lc"] <= 1.5)
    assert torch.equal(torch.where(mask, raw, torch.zeros_like(raw)), full[3])


def test_hadamard_bwd_empty_batch(K):
    c = make_case(K, 0, 16, 16, torch.float32, seed=1)
    gx, da, db, dw = K.hadamard_linear_bwd(c["x"].cuda(), c["gy"].cuda(), 16, 16, c["kw"], c["kwt"],
                                           c["alpha"].cuda(), c["beta"].cuda(), latent=c["lc"])
    torch.cuda.synchronize()
    assert gx.shape == (0, 512)
    assert torch.count_nonzero(da) == 0 and torch.count_nonzero(db) == 0 and torch.count_nonzero(dw) == 0


def test_pack_transpose_matches_oracle(K):
    from oracle import ternary as otern
    c = make_case(K, 1, 5, 7, torch.float32, seed=2)
    pt = K.hadamard_pack_transpose(c["packed"], 5, 7).cpu().numpy()
    ref = otern.pack_codes(np.ascontiguousarray(np.transpose(c["codes"], (0, 2, 1))))
    assert np.array_equal(pt, ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_hadamard_linear_module_autograd(dtype):
    """HadamardLinear.forward + loss.backward() through the HIP kernels vs the
    oracle's gradients (x's gradient in x's dtype, parameters in float32)."""
    from src.model.fht_cuda import HadamardLinear
    torch.manual_seed(5)
    layer = HadamardLinear(512, 1024).cuda()
    with torch.no_grad():
        layer.alpha.add_(0.3 * torch.randn_like(layer.alpha))
    x = torch.randn(4, 64, 512, device="cuda", dtype=dtype, requires_grad=True)
    y = layer(x)
    gy = torch.randn_like(y)
    (y * gy).sum().backward()
    torch.cuda.synchronize()
    from src.model import kernels
    codes = kernels.ternary_quantize(layer.weight.detach(), codes=True)["codes"].cpu().numpy()
    ref = ohad.hadamard_linear_bwd_f64(x.detach().double().cpu().numpy().reshape(-1, 512), codes,
                                       layer.alpha.detach().double().cpu().numpy(),
                                       layer.beta.detach().double().cpu().numpy(),
                                       gy.double().cpu().numpy().reshape(-1, 1024),
                                       latent=layer.weight.detach().double().cpu().numpy())
    assert x.grad.dtype == dtype
    assert_close(x.grad.float().cpu().numpy().reshape(-1, 512), ref[0], dtype, "module x.grad")
    assert_close(layer.alpha.grad.cpu().numpy(), ref[1], dtype, "module alpha.grad")
    assert_close(layer.beta.grad.cpu().numpy(), ref[2], dtype, "module beta.grad")
    assert_close(layer.weight.grad.cpu().numpy(), ref[3], dtype, "module weight.grad")


def test_fht_function_backward():
    from src.model.fht_cuda import fht
    x = torch.randn(8, 64, device="cuda", requires_grad=True)
    g = torch.randn(8, 64, device="cuda")
    (fht(x) * g).sum().backward()
    H = torch.tensor(ohad.sylvester(64), dtype=torch.float64)
    ref = (g.double().cpu() @ H).numpy()
    assert_close(x.grad.cpu().numpy(), ref, torch.float32, "fht grad")


# ---------------------------------------------------------------- octonion

def _oct_parts(rows, n_o):
    return np.stack(np.split(np.asarray(rows, np.float64), 8, axis=-1))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("in_o,out_o,M", [(128, 128, 300), (16, 8, 100), (5, 3, 33), (64, 128, 1), (128, 128, 4000)])
def test_octonion_bwd_vs_oracle(K, in_o, out_o, M, dtype):
    """gx on the forward GEMM (transposed block matrix), dweight / dbeta from
    the split-K product C = gy^T x (16 splits, the last partial, at M 4000;
    one at M <= 100) and the fold, against the float64 oracle."""
    from oracle import octonion as ooct
    print(f"case octonion in_o={in_o} out_o={out_o} M={M} dtype={dtype}", flush=True)
    gen = torch.Generator().manual_seed(in_o + 3 * out_o + M)
    latent = torch.rand(8, out_o, in_o, generator=gen) * 4 - 2
    beta = torch.randn(out_o, generator=gen)
    x = torch.randn(M, 8 * in_o, generator=gen).to(dtype)
    gy = torch.randn(M, 8 * out_o, generator=gen).to(dtype)
    q = K.ternary_quantize(latent.cuda(), codes=True, packed=True)
    gx, dw, db = K.octonion_linear_bwd(x.cuda(), gy.cuda(), in_o, out_o, q["packed"], beta.cuda(),
                                       latent=latent.cuda())
    torch.cuda.synchronize()
    ref = ooct.octonion_linear_bwd_f64(_oct_parts(x.double().numpy(), in_o), q["codes"].cpu().numpy(),
                                       beta.double().numpy(), _oct_parts(gy.double().numpy(), out_o),
                                       latent=latent.double().numpy())
    assert gx.dtype == dtype and gx.shape == x.shape
    assert_close(np.concatenate(list(_oct_parts(gx.float().cpu().numpy(), in_o)), axis=1),
                 np.concatenate(list(ref[0]), axis=1), dtype, f"oct gx {in_o}x{out_o} M={M}")
    assert_close(dw.cpu().numpy(), ref[1], dtype, f"oct dweight {in_o}x{out_o} M={M}")
    assert_close(db.cpu().numpy(), ref[2], dtype, f"oct dbeta {in_o}x{out_o} M={M}")


@pytest.mark.parametrize("cls", ["OctonionTernaryLinearRef", "OctonionFusedLinear"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_octonion_module_autograd(dtype, cls):
    """Gradients of both octonion modules vs float64 autograd of the layer.
    OctonionTernaryLinearRef computes in the input dtype (float32 bars for
    float32); OctonionFusedLinear multiplies bf16 operands whatever the input
    dtype (the reference GPU module, cayley_dickson_cuda.py:402), so its
    bars are bf16's."""
    from oracle import octonion as ooct
    from src.model import kernels, octonion
    torch.manual_seed(11)
    layer = getattr(octonion, cls)(256, 512).cuda()
    if cls == "OctonionFusedLinear":
        dtype_bar = torch.bfloat16
    else:
        dtype_bar = dtype
    xr = torch.randn(2, 40, 256, device="cuda", dtype=dtype)
    parts = tuple(p.detach().requires_grad_(True) for p in xr.split(32, dim=-1))
    ys = layer(parts)
    gys = [torch.randn_like(y) for y in ys]
    sum((y * g).sum() for y, g in zip(ys, gys)).backward()
    torch.cuda.synchronize()
    codes = kernels.ternary_quantize(layer.weight.detach(), codes=True)["codes"].cpu().numpy()
    ref = ooct.octonion_linear_bwd_f64(np.stack([p.detach().double().cpu().numpy().reshape(-1, 32) for p in parts]),
                                       codes, layer.beta.detach().double().cpu().numpy(),
                                       np.stack([g.double().cpu().numpy().reshape(-1, 64) for g in gys]),
                                       latent=layer.weight.detach().double().cpu().numpy())
    gx = np.stack([p.grad.float().cpu().numpy().reshape(-1, 32) for p in parts])
    assert parts[0].grad.dtype == dtype
    assert_close(gx, ref[0], dtype_bar, f"oct {cls} x.grad")
    assert_close(layer.weight.grad.cpu().numpy(), ref[1], dtype_bar, f"oct {cls} weight.grad")
    assert_close(layer.beta.grad.cpu().numpy(), ref[2], dtype_bar, f"oct {cls} beta.grad")


# ---------------------------------------------------------------- Sinkhorn

@pytest.mark.parametrize("n", [1, 2, 4, 7])
def test_sinkhorn_bwd_vs_oracle(K, n):
    from oracle import mhc as omhc
    rng = np.random.default_rng(n)
    h = rng.normal(0, 1.5, (300, n, n)).astype(np.float32)
    g = rng.normal(0, 1, (300, n, n)).astype(np.float32)
    dh = K.sinkhorn_bwd(torch.from_numpy(h).cuda(), torch.from_numpy(g).cuda()).cpu().numpy()
    ref = omhc.sinkhorn_bwd(h.astype(np.float64), g.astype(np.float64))
    if n == 1:
        # a 1x1 projection is exp(h) / (exp(h) + eps) ~ 1: the exact gradient
        # is O(eps) and rounds to 0 in float32
        assert np.abs(ref).max() < 1e-6 and np.abs(dh).max() < 1e-6
        return
    assert_close(dh, ref, torch.float32, f"sinkhorn bwd n={n}")


def test_sinkhorn_function_autograd():
    from oracle import mhc as omhc
    from src.model.mhc import SinkhornKnopp
    rng = np.random.default_rng(3)
    h = torch.from_numpy(rng.normal(0, 1, (2, 8, 4, 4)).astype(np.float32)).cuda().requires_grad_(True)
    g = torch.from_numpy(rng.normal(0, 1, (2, 8, 4, 4)).astype(np.float32)).cuda()
    (SinkhornKnopp()(h) * g).sum().backward()
    ref = omhc.sinkhorn_bwd(h.detach().double().cpu().numpy(), g.double().cpu().numpy())
    assert_close(h.grad.cpu().numpy(), ref, torch.float32, "SinkhornKnopp grad")


# ---------------------------------------------------------------- whole model

def _grad_rel(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    nb = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / nb) if nb > 0 else float(np.linalg.norm(a - b))


@pytest.mark.parametrize("C,n_layer,vocab,T", [(64, 2, 256, 16), (256, 2, 512, 32)])
def test_mhcwalsh_backward_matches_oracle(C, n_layer, vocab, T):
    """One training backward of mHCWalsh (float32) through the HIP backward
    kernels (Hadamard linears, Sinkhorn) and the differentiable training
    composition, against float64 autograd of the oracle model with the
    reference's STE; every parameter's gradient is compared."""
    from oracle.model import Oracle
    from src.model import WalshConfig, mHCWalsh
    torch.manual_seed(0)
    cfg = WalshConfig(block_size=64, vocab_size=vocab, n_layer=n_layer, n_head=32, n_embd=C, algebra='hadamard',
                      head_mixing=True)
    model = mHCWalsh(cfg, n_streams=4).cuda().eval()
    g = torch.Generator().manual_seed(1)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith(('.alpha', '.beta', 'norm.weight')) and p.dim() > 0:
                p.mul_(1 + 0.2 * torch.randn(p.shape, generator=g).to(p.device))
    idx = torch.randint(0, vocab, (2, T), generator=g)
    tgt = torch.randint(0, vocab, (2, T), generator=g)
    _, loss = model(idx.cuda(), targets=tgt.cuda())
    loss.backward()
    torch.cuda.synchronize()
    orc = Oracle(model.state_dict(), C, 32, n_layer, grad=True)
    ref_loss = orc.loss(idx, tgt)
    ref_loss.backward()
    print(f"loss gpu={loss.item():.6f} oracle={ref_loss.item():.6f}", flush=True)
    assert abs(loss.item() - ref_loss.item()) <= 1e-5 * abs(ref_loss.item())
    got, ref = {}, {}
    for name, p in model.named_parameters():
        assert p.grad is not None, f"{name}: no gradient"
        assert orc.sd[name].grad is not None, f"{name}: no oracle gradient"
        got[name] = p.grad.double().cpu().numpy().ravel()
        ref[name] = orc.sd[name].grad.numpy().ravel()
    # all gradients together at the float32 bar; each parameter within 1e-4
    # of its own norm plus 1e-6 of the largest gradient norm (some exact
    # gradients are ~0, e.g. H_res of layer 0 mixes identical streams, and
    # only a floor relative to the model's gradient scale is meaningful there)
    total = _grad_rel(np.concatenate(list(got.values())), np.concatenate(list(ref.values())))
    G = max(np.linalg.norm(v) for v in ref.values())
    bad = [(name, float(np.linalg.norm(got[name] - ref[name])), float(np.linalg.norm(ref[name])))
           for name in got if np.linalg.norm(got[name] - ref[name]) > 1e-4 * np.linalg.norm(ref[name]) + 1e-6 * G]
    worst = max((_grad_rel(got[n], ref[n]), n) for n in got if np.linalg.norm(ref[n]) > 1e-3 * G)
    print(f"C={C} L={n_layer}: {len(got)} parameters, all-gradient rel_norm {total:.2e}, worst rel_norm of the "
          f"{sum(np.linalg.norm(ref[n]) > 1e-3 * G for n in got)} with norm > 1e-3 max: {worst[0]:.2e} ({worst[1]})",
          flush=True)
    assert total <= 1e-5, total
    assert not bad, bad


# ---------------------------------------------------------------- MoE

def test_ternary_ste_bwd_modes(K):
    g = torch.tensor([-3.0, -2.0, -0.5, 0.0, 1.9, 2.5, float("nan")], device="cuda")
    w = torch.tensor([-1.6, -1.5, 0.3, 1.5, 1.51, -3.0, 0.0], device="cuda")
    m1 = K.ternary_ste_bwd(g, mode=1).cpu()
    assert torch.equal(m1[:6], torch.tensor([-2.0, -2.0, -0.5, 0.0, 1.9, 2.0])) and torch.isnan(m1[6])
    m0 = K.ternary_ste_bwd(g, w, mode=0).cpu()
    assert torch.equal(m0[:6], torch.tensor([0.0, -2.0, -0.5, 0.0, 0.0, 0.0])) and torch.isnan(m0[6])


@pytest.mark.parametrize("C,k,T", [(256, 4, 24), (512, 6, 24), (512, 6, 512), (1024, 6, 24)])
def test_moe_backward_matches_oracle(C, k, T):
    """HadamardMoE training backward (routing, balance loss, the experts'
    forward and backward on the HIP kernels over the routed pairs, MoE STE)
    against float64 autograd of the oracle's MoE (moe.py:418-447, :337-380,
    :544-560) on the same parameters; T 512 gives each expert workgroup many
    pairs, C 1024 (32 experts) leaves some workgroups without pairs."""
    from oracle.model import Oracle
    from src.model import WalshConfig
    from src.model.moe import HadamardMoE
    torch.manual_seed(4)
    cfg = WalshConfig(n_embd=C, n_head=32, n_layer=1, vocab_size=64, block_size=64)
    m = HadamardMoE(cfg, max_experts=k).cuda().train()
    with torch.no_grad():
        for lin in (m.router.gate[0], m.router.gate[2]):
            lin.weight.normal_(0, 0.2)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, T, C, generator=g).cuda().requires_grad_(True)
    gy = torch.randn(2, T, C, generator=g).cuda()
    y = m(x)
    loss = (y * gy).sum() + 0.3 * m.get_aux_loss()
    loss.backward()
    torch.cuda.synchronize()
    orc = Oracle({"m." + n: t for n, t in m.state_dict().items()}, C, 32, 1, moe_max_experts=k, grad=True)
    x64 = x.detach().double().cpu().requires_grad_(True)
    out, info = orc.moe(x64, "m")
    E = C // 32
    aux = (info["mask"].reshape(-1, E).mean(0) * info["probs"].reshape(-1, E).mean(0)).sum() * E
    ref_loss = (out * gy.double().cpu()).sum() + 0.3 * aux
    ref_loss.backward()
    assert np.array_equal(m._last_expert_mask.cpu().numpy(), info["mask"].detach().numpy()), "routing differs"
    got = {"x": x.grad}
    ref = {"x": x64.grad}
    for n, p in m.named_parameters():
        got[n], ref[n] = p.grad, orc.sd["m." + n].grad
    G = max(float(v.norm()) for v in ref.values())
    for n in got:
        a, b = got[n].double().cpu().numpy().ravel(), ref[n].numpy().ravel()
        err, nb = float(np.linalg.norm(a - b)), float(np.linalg.norm(b))
        print(f"moe C={C} k={k} {n}: rel_norm {err / max(nb, 1e-300):.2e} (|ref| {nb:.3e})", flush=True)
        assert err <= 1e-5 * nb + 1e-6 * G, (n, err, nb)


def test_moe_checkpointed_backward_equals_plain():
    """Activation checkpointing (non-reentrant, as mHCWalsh's
    gradient_checkpointing uses) recomputes the MoE forward during the
    backward; the gradients, including the routing weights' path through
    the expert outputs into the router, equal the plain backward's bitwise:
    the recomputed pair order and pair lists are the ones the backward
    reads.  The experts' own weight gradients agree to float32 summation
    order (1e-4 of the largest entry)."""
    from src.model import WalshConfig
    from src.model.moe import HadamardMoE
    torch.manual_seed(6)
    C, k, T = 512, 6, 96
    cfg = WalshConfig(n_embd=C, n_head=32, n_layer=1, vocab_size=64, block_size=128)
    m = HadamardMoE(cfg, max_experts=k).cuda().train()
    with torch.no_grad():
        for lin in (m.router.gate[0], m.router.gate[2]):
            lin.weight.normal_(0, 0.2)
    g = torch.Generator().manual_seed(7)
    x0 = torch.randn(2, T, C, generator=g).cuda()
    gy = torch.randn(2, T, C, generator=g).cuda()

    def run(ckpt):
        m.zero_grad(set_to_none=True)
        x = x0.clone().requires_grad_(True)
        y = torch.utils.checkpoint.checkpoint(m, x, use_reentrant=False) if ckpt else m(x)
        (y * gy).sum().backward()
        torch.cuda.synchronize()
        return {"x": x.grad.clone(), **{n: p.grad.clone() for n, p in m.named_parameters()}}
    plain, ck = run(False), run(True)
    assert plain["router.gate.2.weight"].abs().max() > 0
    for n in plain:
        d = float((plain[n] - ck[n]).abs().max())
        scale = float(plain[n].abs().max())
        print(f"checkpointed MoE grad {n}: max |diff| {d:.3e} (max |grad| {scale:.3e})", flush=True)
        if n.startswith("experts."):
            # the experts' weight gradients sum their pairs per workgroup; the
            # order of an expert's pair list comes from the scatter's atomics,
            # so those float32 sums may group pairs differently run to run
            assert d <= 1e-4 * scale, n
        else:
            # the routing-weight path (d expert_weights into the router) and
            # the input gradient: bitwise
            assert d == 0.0, n


def test_mhcwalsh_backward_bf16_autocast():
    """A bf16-autocast training backward runs and lands near the float64
    gradients: bf16 activations round at every layer, so the bar is the
    all-gradient relative error <= 3e-2 (the float32 run meets 1e-5)."""
    from oracle.model import Oracle
    from src.model import WalshConfig, mHCWalsh
    torch.manual_seed(0)
    C, n_layer, vocab, T = 256, 2, 512, 32
    cfg = WalshConfig(block_size=64, vocab_size=vocab, n_layer=n_layer, n_head=32, n_embd=C, algebra='hadamard',
                      head_mixing=True)
    model = mHCWalsh(cfg, n_streams=4).cuda().eval()
    g = torch.Generator().manual_seed(1)
    idx = torch.randint(0, vocab, (2, T), generator=g)
    tgt = torch.randint(0, vocab, (2, T), generator=g)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        _, loss = model(idx.cuda(), targets=tgt.cuda())
    loss.backward()
    torch.cuda.synchronize()
    orc = Oracle(model.state_dict(), C, 32, n_layer, grad=True)
    ref_loss = orc.loss(idx, tgt)
    ref_loss.backward()
    got = np.concatenate([p.grad.double().cpu().numpy().ravel() for _, p in model.named_parameters()])
    ref = np.concatenate([orc.sd[n].grad.numpy().ravel() for n, _ in model.named_parameters()])
    rel = _grad_rel(got, ref)
    print(f"bf16 autocast: loss gpu={loss.item():.5f} oracle={ref_loss.item():.5f}, all-gradient rel_norm {rel:.2e}",
          flush=True)
    assert abs(loss.item() - ref_loss.item()) <= 1e-2 * abs(ref_loss.item())
    assert rel <= 3e-2, rel


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("in_o,gsx,out_o,gsy", [(16, 16, 43, 44), (43, 44, 16, 16), (43, 48, 43, 44)])
def test_hadamard_bwd_group_padded(K, in_o, gsx, out_o, gsy, dtype):
    """walsh_hadamard_linear_ex_bwd on group-padded rows (the training SwiGLU
    hidden layout) against the oracle on the unpadded rows; gx pad slots are
    zeros, x / gy pad slots are ignored (filled with junk here)."""
    c = make_case(K, 130, in_o, out_o, dtype, seed=in_o + gsx + out_o + gsy)
    M = 130
    xp = torch.full((M, 32, gsx), 7.0, dtype=dtype)
    xp[:, :, :in_o] = c["x"].view(M, 32, in_o)
    gp = torch.full((M, 32, gsy), -5.0, dtype=dtype)
    gp[:, :, :out_o] = c["gy"].view(M, 32, out_o)
    gx, da, db, dw = K.hadamard_linear_bwd(xp.view(M, -1).cuda(), gp.view(M, -1).cuda(), in_o, out_o, c["kw"],
                                           c["kwt"], c["alpha"].cuda(), c["beta"].cuda(), latent=c["lc"], gsx=gsx,
                                           gsy=gsy)
    torch.cuda.synchronize()
    ref = ohad.hadamard_linear_bwd_f64(c["x"].double().numpy(), c["codes"], c["alpha"].double().numpy(),
                                       c["beta"].double().numpy(), c["gy"].double().numpy(),
                                       latent=c["latent"].double().numpy())
    gx3 = gx.float().cpu().view(M, 32, gsx)
    assert torch.count_nonzero(gx3[:, :, in_o:]) == 0
    assert_close(gx3[:, :, :in_o].reshape(M, -1).numpy(), ref[0], dtype, f"padded gx {in_o}/{gsx}x{out_o}/{gsy}")
    for name, got, r in (("dalpha", da, ref[1]), ("dbeta", db, ref[2]), ("dweight", dw, ref[3])):
        assert_close(got.cpu().numpy(), r, dtype, f"padded {name}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,C", [(4, 512), (3, 44), (1, 260)])
def test_stream_mixing_bwd(K, n, C, dtype):
    """walsh_mhc_aggregate_fwd/_bwd and walsh_mhc_post_bwd against float64
    autograd of layer_in = H_pre @ x and x_new = H_res @ x + H_post^T out
    (mhc.py:366-381) on the same (rounded) inputs."""
    g = torch.Generator().manual_seed(n * 1000 + C)
    M = 37
    x = torch.randn(M, n, C, generator=g).to(dtype)
    out = torch.randn(M, C, generator=g).to(dtype)
    hp = torch.rand(M, 1, n, generator=g)
    hr = torch.rand(M, n, n, generator=g)
    hq = 2 * torch.rand(M, 1, n, generator=g)
    gli = torch.randn(M, C, generator=g).to(dtype)
    gnew = torch.randn(M, n, C, generator=g).to(dtype)
    li = K.mhc_aggregate(x.cuda(), hp.cuda())
    dx1, dhp = K.mhc_aggregate_bwd(x.cuda(), hp.cuda(), gli.cuda())
    dx2, dout, dhr, dhq = K.mhc_post_bwd(x.cuda(), out.cuda(), hr.cuda(), hq.cuda(), gnew.cuda())
    torch.cuda.synchronize()
    xr, orr, hpr, hrr, hqr = (t.double().requires_grad_(True) for t in (x, out, hp, hr, hq))
    li_ref = torch.matmul(hpr, xr).squeeze(1)
    new_ref = torch.matmul(hrr, xr) + hqr.transpose(-2, -1) * orr.unsqueeze(1)
    torch.autograd.backward([li_ref, new_ref], [gli.double(), gnew.double()])
    assert_close(li.float().cpu().numpy(), li_ref.detach().numpy(), dtype, f"aggregate n={n} C={C}")
    assert_close(dhp.cpu().numpy(), hpr.grad.numpy(), dtype, "dh_pre")
    assert_close(dhr.cpu().numpy(), hrr.grad.numpy(), dtype, "dh_res")
    assert_close(dhq.cpu().numpy(), hqr.grad.numpy(), dtype, "dh_post")
    assert_close(dout.float().cpu().numpy(), orr.grad.numpy(), dtype, "d_out")
    assert_close((dx1.float() + dx2.float()).cpu().numpy(), xr.grad.numpy(), dtype, "dx")


def test_training_step_hip_graph_matches_eager():
    """A training step (forward with targets, backward, AdamW) captured as one
    HIP graph, how bench.py's train2 runs it: three replays move the
    parameters as three eager steps do (float32; torch's embedding backward
    sums with atomics, so the bar is a relative 1e-5 over all parameters),
    with eager work and synchronisation between the replays."""
    from src.model import WalshConfig, mHCWalsh
    C, n_layer, vocab, T = 64, 2, 256, 32
    cfg = WalshConfig(block_size=64, vocab_size=vocab, n_layer=n_layer, n_head=32, n_embd=C, algebra='hadamard',
                      head_mixing=True)
    g = torch.Generator().manual_seed(3)
    idx = torch.randint(0, vocab, (2, T), generator=g).cuda()
    tgt = torch.randint(0, vocab, (2, T), generator=g).cuda()
    models = []
    for _ in range(2):
        torch.manual_seed(0)
        m = mHCWalsh(cfg, n_streams=4).cuda().train()
        models.append((m, torch.optim.AdamW(m.parameters(), lr=1e-3, foreach=True, capturable=True)))

    def step(m, opt):
        opt.zero_grad(set_to_none=True)
        _, loss = m(idx, targets=tgt)
        loss.backward()
        opt.step()

    (ma, oa), (mb, ob) = models
    for _ in range(3):
        step(ma, oa)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            step(mb, ob)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    ob.zero_grad(set_to_none=True)
    with torch.cuda.graph(graph):
        _, loss = mb(idx, targets=tgt)
        loss.backward()
        ob.step()
    for i in range(3):
        step(ma, oa)
        graph.replay()
        torch.cuda.synchronize()
        pa = torch.cat([p.detach().reshape(-1) for p in ma.parameters()])
        pb = torch.cat([p.detach().reshape(-1) for p in mb.parameters()])
        rel = ((pa - pb).norm() / pa.norm()).item()
        print(f"replay {i}: parameter rel diff {rel:.2e}", flush=True)
        assert rel <= 1e-5, (i, rel)


@pytest.mark.parametrize("use_moe", [False, True])
def test_gradient_checkpointing_matches_plain_backward(use_moe):
    """mHCWalsh(gradient_checkpointing=True) in training recomputes each
    layer in the backward (mhc.py:647-649): the loss and every parameter's
    gradient equal the run without checkpointing (float32, the backward
    kernels are deterministic)."""
    from src.model import WalshConfig, mHCWalsh
    C, n_layer, vocab, T = 64, 2, 256, 16
    grads = []
    for ckpt in (False, True):
        torch.manual_seed(0)
        cfg = WalshConfig(block_size=64, vocab_size=vocab, n_layer=n_layer, n_head=32, n_embd=C,
                          algebra='hadamard', head_mixing=True, use_moe=use_moe, moe_max_experts=2)
        model = mHCWalsh(cfg, n_streams=4, gradient_checkpointing=ckpt).cuda().train()
        g = torch.Generator().manual_seed(1)
        idx = torch.randint(0, vocab, (2, T), generator=g).cuda()
        tgt = torch.randint(0, vocab, (2, T), generator=g).cuda()
        _, loss = model(idx, targets=tgt)
        loss.backward()
        torch.cuda.synchronize()
        grads.append((loss.item(), {n: p.grad.detach().clone() for n, p in model.named_parameters()}))
    (l0, g0), (l1, g1) = grads
    print(f"moe={use_moe}: loss {l0:.7f} / checkpointed {l1:.7f}")
    assert abs(l0 - l1) <= 1e-6 * abs(l0)
    assert g0.keys() == g1.keys()
    for n in g0:
        d = (g0[n] - g1[n]).norm().item()
        assert d <= 1e-6 * g0[n].norm().item() + 1e-12, f"{n}: |diff| {d:.3e}"
