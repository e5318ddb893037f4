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
