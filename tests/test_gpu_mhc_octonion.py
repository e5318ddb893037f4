"""GPU parity: Sinkhorn, fused mHC mappings/stream and the octonion layer vs the oracle."""
import numpy as np
import pytest
import torch

from oracle import mhc as omhc
from oracle import octonion as ooct
from oracle import ternary as otern

from test_gpu_hadamard import assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def K():
    from src.model import kernels
    return kernels


# ------------------------------------------------------------------ Sinkhorn

@pytest.mark.parametrize("n", [1, 2, 4, 8])
def test_sinkhorn_matches_oracle(K, n):
    rng = np.random.default_rng(n)
    h = rng.standard_normal((257, n, n)).astype(np.float32)
    out = K.sinkhorn(torch.from_numpy(h).cuda()).cpu().numpy()
    ref = omhc.sinkhorn(h.astype(np.float64))
    assert np.max(np.abs(out - ref)) < 2e-6
    ref32 = omhc.sinkhorn(h, dtype=np.float32)
    assert np.max(np.abs(out - ref32)) < 1e-6
    assert np.max(np.abs(out.sum(-1) - 1)) < 1e-6


def test_sinkhorn_module_and_invariants():
    from src.model import SinkhornKnopp
    from src.model.mhc import sinkhorn_knopp_fused
    h = torch.randn(3, 5, 4, 4, device="cuda")
    a = SinkhornKnopp(n_iter=20)(h)
    b = sinkhorn_knopp_fused(h)
    assert a.shape == h.shape and torch.equal(a, b)
    assert torch.all(a > 0)
    one = SinkhornKnopp()(torch.zeros(2, 1, 1, device="cuda"))
    assert torch.allclose(one, torch.ones_like(one))


# ------------------------------------------------------------------ mHC

def _maps(rng, n, C):
    return dict(pre=(rng.normal(0, 0.02, (n, n * C)), 0.01 + rng.uniform(0, 0.5), rng.normal(0, 1, (1, n))),
                post=(rng.normal(0, 0.02, (n, n * C)), 0.01 + rng.uniform(0, 0.5), rng.normal(0, 1, (1, n))),
                res=(rng.normal(0, 0.02, (n * n, n * C)), 0.01 + rng.uniform(0, 0.5),
                     2 * np.eye(n) + rng.normal(0, 0.3, (n, n))))


def _fused_params(maps, n, C, dtype):
    phi = np.zeros((32, n * C), np.float32)
    phi[:n] = maps['pre'][0]
    phi[n:2 * n] = maps['post'][0]
    phi[2 * n:2 * n + n * n] = maps['res'][0]
    coef = np.array([maps['pre'][1], maps['post'][1], maps['res'][1]], np.float32)
    bias = np.concatenate([maps['pre'][2].reshape(-1), maps['post'][2].reshape(-1),
                           maps['res'][2].reshape(-1)]).astype(np.float32)
    t = lambda a: torch.from_numpy(a).cuda()  # noqa: E731
    return t(phi).to(dtype), t(coef), t(bias)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,n,C", [(100, 4, 512), (33, 4, 64), (7, 2, 32), (64, 1, 16), (50, 3, 40)])
def test_mhc_pre_post_match_oracle(K, dtype, M, n, C):
    rng = np.random.default_rng(M + n + C)
    x = rng.normal(0, 1, (M, n, C)).astype(np.float32)
    maps = _maps(rng, n, C)
    xt = torch.from_numpy(x).cuda().to(dtype)
    xq = xt.float().cpu().numpy().astype(np.float64)
    eps = float(torch.finfo(dtype).eps)
    phi, coef, bias = _fused_params(maps, n, C, dtype)
    li, hp, hq, hr = K.mhc_pre(xt, phi, coef, bias, eps)
    # oracle on the same (bf16-rounded) inputs; phi rounded like the kernel's operand
    phiq = phi.float().cpu().numpy().astype(np.float64)
    m2 = dict(pre=(phiq[:n], *maps['pre'][1:]), post=(phiq[n:2 * n], *maps['post'][1:]),
              res=(phiq[2 * n:2 * n + n * n], *maps['res'][1:]))
    out = rng.normal(0, 1, (M, C)).astype(np.float32)
    outt = torch.from_numpy(out).cuda().to(dtype)
    outq = outt.float().cpu().numpy().astype(np.float64)
    x_new_ref, hp_ref, hq_ref, hr_ref, li_ref = omhc.stream_forward(xq, m2, lambda v: outq, eps)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert np.max(np.abs(hp.cpu().numpy() - hp_ref[:, 0])) < tol
    assert np.max(np.abs(hq.cpu().numpy() - hq_ref[:, 0])) < 2 * tol
    assert np.max(np.abs(hr.cpu().numpy() - hr_ref)) < tol
    assert_close(li.float().cpu().numpy(), li_ref, dtype, f"layer_in {dtype} M={M} n={n} C={C}")
    # post with the oracle's own H (isolates the apply kernel)
    x_new = K.mhc_post(xt, outt, torch.from_numpy(hr_ref.astype(np.float32)).cuda(),
                       torch.from_numpy(hq_ref[:, 0].astype(np.float32)).cuda())
    assert_close(x_new.float().cpu().numpy(), x_new_ref, dtype, f"x_new {dtype}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("tracked", [False, True])
def test_stream_module_matches_oracle(dtype, tracked):
    """The fused inference kernels (untracked) and the differentiable
    training composition (autograd tracking the call) both match the oracle."""
    with torch.set_grad_enabled(tracked):
        _stream_module_case(dtype)


def _stream_module_case(dtype):
    from src.model import mHCResidualStream
    torch.manual_seed(0)
    n, C, B, T = 4, 64, 2, 9
    s = mHCResidualStream(C, n).cuda()
    with torch.no_grad():
        for m in (s.H_pre, s.H_post, s.H_res):
            m.alpha.fill_(0.3)
            m.phi.weight.normal_(0, 0.05)
            m.bias.add_(torch.randn_like(m.bias) * 0.2)
    x = torch.randn(B, T, n, C, device="cuda").to(dtype)
    lin = torch.randn(C, C, device="cuda") / 8
    y = s(x, lambda v: (v.float() @ lin).to(v.dtype))
    maps = {k: (getattr(s, 'H_' + k).phi.weight.detach().to(dtype).double().cpu().numpy(),
                float(getattr(s, 'H_' + k).alpha), getattr(s, 'H_' + k).bias.detach().double().cpu().numpy())
            for k in ('pre', 'post', 'res')}
    xq = x.float().cpu().numpy().reshape(B * T, n, C).astype(np.float64)
    L = lin.double().cpu().numpy()
    ref, *_ = omhc.stream_forward(xq, maps, lambda v: v @ L, float(torch.finfo(dtype).eps))
    assert_close(y.detach().float().cpu().numpy().reshape(B * T, n, C), ref, dtype, f"stream {dtype}")
    # standalone mappings agree with the fused path
    xf = x.reshape(B, T, n * C)
    hr = s.H_res(xf)
    hp = s.H_pre(xf)
    _, hp_ref, _, hr_ref, _ = omhc.stream_forward(xq, maps, lambda v: v, float(torch.finfo(dtype).eps))
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert np.max(np.abs(hr.detach().cpu().numpy().reshape(-1, n, n) - hr_ref)) < tol
    assert np.max(np.abs(hp.detach().cpu().numpy().reshape(-1, n) - hp_ref[:, 0])) < tol


# ------------------------------------------------------------------ octonion

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,in_o,out_o", [(300, 128, 128), (129, 64, 64), (5, 16, 16), (77, 32, 48), (64, 171, 64),
                                          (40, 64, 171)])
def test_octonion_linear_matches_oracle(K, dtype, M, in_o, out_o):
    rng = np.random.default_rng(M + in_o + out_o)
    w = (rng.standard_normal((8, out_o, in_o)) * 0.02).astype(np.float32)
    codes = otern.ternary_codes(w, otern.absmean_gamma(w))
    beta = rng.uniform(0.05, 0.3, out_o).astype(np.float32)
    x = rng.standard_normal((M, 8 * in_o)).astype(np.float32)
    packed = torch.from_numpy(otern.pack_codes(codes)).cuda()
    B = K.octonion_prepare(packed, in_o, out_o, dtype)
    xt = torch.from_numpy(x).cuda().to(dtype)
    y = K.octonion_linear(xt, in_o, out_o, B, torch.from_numpy(beta).cuda())
    xq = xt.float().cpu().numpy().astype(np.float64)
    parts = xq.reshape(M, 8, in_o).transpose(1, 0, 2)
    ref = ooct.octonion_linear_f64(parts, codes, beta).transpose(1, 0, 2).reshape(M, 8 * out_o)
    assert_close(y.float().cpu().numpy(), ref, dtype, f"octonion {dtype} M={M} {in_o}x{out_o}")


@torch.no_grad()
def test_octonion_module_tuple_interface(K):
    """OctonionFusedLinear keeps the reference GPU module's contract
    (cayley_dickson_cuda.py:650-668): x rounded to bf16, the float32 sum
    rounded to bf16, times the float32 beta, a float32 result with or
    without autocast.  OctonionTernaryLinearRef (physics.py:53-82) computes
    in float32 for float32 inputs.  The bf16-output kernel that chains the
    layers in a stack stores bf16(x W^T beta), within one bf16 ulp of
    bf16(the module's output)."""
    from src.model.cayley_dickson_cuda import OctonionFusedLinear, cayley_dickson_fused
    from src.model.physics import OctonionTernaryLinearRef
    torch.manual_seed(1)
    layer = OctonionFusedLinear(512, 256).cuda()
    with torch.no_grad():
        layer.beta.mul_(1 + 0.2 * torch.randn_like(layer.beta))
    x = torch.randn(2, 10, 512, device="cuda")
    parts = x.split(64, dim=-1)
    ys = layer(parts)
    assert len(ys) == 8 and ys[0].shape == (2, 10, 32) and ys[0].dtype == torch.float32
    w = layer.weight.detach().cpu().numpy()
    codes = otern.ternary_codes(w, otern.absmean_gamma(w))
    beta = layer.beta.detach().cpu().numpy()
    xp = x.double().cpu().numpy().reshape(20, 8, 64).transpose(1, 0, 2)
    ref = ooct.octonion_linear_gpu_semantics(xp, codes, beta)
    got = torch.stack(ys).double().cpu().numpy().reshape(8, 20, 32)
    assert_close(got, ref, torch.bfloat16, "module fp32 in (bf16 operands)")
    # away from a bf16 rounding boundary of the float32 sum the result is the
    # oracle's to float32 rounding of the beta product
    acc = ooct.octonion_linear_f64(ooct.bf16_round(xp).astype(np.float64), codes, np.ones(32))
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(acc), 1e-30))) - 7)
    safe = np.abs(acc / ulp - np.floor(acc / ulp) - 0.5) > 0.05  # not within 5% of an ulp of a midpoint
    d = np.abs(got - ref)[safe] / np.maximum(np.abs(ref[safe]), 1e-30)
    print(f"octonion module: {int(safe.sum())} of {safe.size} away from a bf16 boundary, max rel {d.max():.2e}")
    assert d.max() <= 2 ** -23
    # non-adjacent parts (a copy is made) give the same result
    ys2 = layer(tuple(p.clone() for p in parts))
    assert all(torch.equal(a, b) for a, b in zip(ys, ys2))
    # bf16 autocast: the same float32 result (the input is rounded to bf16 either way)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        yb = layer(parts)
    assert yb[0].dtype == torch.float32
    assert all(torch.equal(a, b) for a, b in zip(ys, yb))
    # the stack's bf16 kernel output (beta folded, one rounding) is within
    # one bf16 ulp of bf16(module output)
    yk = K.octonion_linear(x.bfloat16().reshape(20, 512), 64, 32, layer.block_matrix(torch.bfloat16), layer.beta)
    ym = torch.cat(ys, -1).reshape(20, 256)
    d = (yk.float() - ym.bfloat16().float()).abs()
    assert torch.all(d <= torch.exp2(torch.floor(torch.log2(ym.abs().clamp_min(1e-30))) - 7) * 1.01)
    # Ref class: float32 math for float32 input
    ref_layer = OctonionTernaryLinearRef(512, 256).cuda()
    yr = ref_layer(parts)
    assert yr[0].dtype == torch.float32
    w = ref_layer.weight.detach().cpu().numpy()
    codes_r = otern.ternary_codes(w, otern.absmean_gamma(w))
    assert_close(torch.stack(yr).double().cpu().numpy().reshape(8, 20, 32),
                 ooct.octonion_linear_f64(xp, codes_r, ref_layer.beta.detach().cpu().numpy()), torch.float32,
                 "Ref module fp32")
    # the functional form returns the kernel's bf16 (no beta)
    wq = torch.from_numpy(codes.astype(np.float32)).cuda()
    yf = cayley_dickson_fused(parts, wq)
    assert yf[0].dtype == torch.bfloat16
    assert_close(torch.stack(yf).double().cpu().numpy().reshape(8, 20, 32), ooct.bf16_round(acc.astype(np.float32)),
                 torch.bfloat16, "functional form (bf16, no beta)")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,n,C", [(100, 4, 512), (33, 4, 64), (7, 2, 32), (64, 1, 16), (50, 4, 1024), (40, 3, 48)])
@pytest.mark.parametrize("with_norm", [False, True])
def test_mhc_pre_norm_matches_oracle(K, dtype, M, n, C, with_norm):
    if not K.mhc_pre_supported(n, C, dtype):
        pytest.skip("shape served by walsh_mhc_pre_fwd (row too large for the LDS tile)")
    rng = np.random.default_rng(M * 7 + n + C)
    x = rng.normal(0, 1, (M, n, C)).astype(np.float32)
    maps = _maps(rng, n, C)
    xt = torch.from_numpy(x).cuda().to(dtype)
    xq = xt.float().cpu().numpy().astype(np.float64)
    eps = float(torch.finfo(dtype).eps)
    phi, coef, bias = _fused_params(maps, n, C, dtype)
    w = rng.uniform(0.5, 1.5, C).astype(np.float32)
    li, hp, hq, hr = K.mhc_pre_norm(xt, K.phi_fragments(phi), coef, bias, eps,
                                    norm_w=torch.from_numpy(w).cuda() if with_norm else None, norm_eps=1e-6)
    phiq = phi.float().cpu().numpy().astype(np.float64)
    m2 = dict(pre=(phiq[:n], *maps['pre'][1:]), post=(phiq[n:2 * n], *maps['post'][1:]),
              res=(phiq[2 * n:2 * n + n * n], *maps['res'][1:]))
    _, hp_ref, hq_ref, hr_ref, li_ref = omhc.stream_forward(xq, m2, lambda v: v, eps)
    if with_norm:
        li_ref = li_ref / np.sqrt((li_ref ** 2).mean(-1, keepdims=True) + 1e-6) * w
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert np.max(np.abs(hp.cpu().numpy() - hp_ref[:, 0])) < tol
    assert np.max(np.abs(hq.cpu().numpy() - hq_ref[:, 0])) < 2 * tol
    assert np.max(np.abs(hr.cpu().numpy() - hr_ref)) < tol
    assert_close(li.float().cpu().numpy(), li_ref, dtype, f"pre_norm {dtype} M={M} n={n} C={C} norm={with_norm}")
    # identical H to the one-pass-per-K-slice kernel
    _, hp1, hq1, hr1 = K.mhc_pre(xt, phi, coef, bias, eps)
    assert torch.allclose(hr, hr1, atol=1e-6) and torch.allclose(hp, hp1, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("M,n,C", [(100, 4, 512), (33, 4, 64), (7, 2, 32), (40, 3, 96), (1, 4, 512), (50, 4, 1024)])
def test_mhc_post_pre_norm_equals_separate_kernels(K, dtype, M, n, C):
    """The fused stream update + next mappings (walsh_mhc_post_pre_norm_fwd)
    give bitwise the results of walsh_mhc_post_fwd followed by
    walsh_mhc_pre_norm_fwd (which the oracle tests pin)."""
    if not K.mhc_post_pre_supported(n, C, dtype):
        pytest.skip("shape outside the fused kernel (LDS tile or 16-byte chunks)")
    print(f"post+pre fused M={M} n={n} C={C} {dtype}", flush=True)
    rng = np.random.default_rng(M * 5 + n + C)
    x_old = torch.from_numpy(rng.normal(0, 1, (M, n, C)).astype(np.float32)).cuda().to(dtype)
    out = torch.from_numpy(rng.normal(0, 1, (M, C)).astype(np.float32)).cuda().to(dtype)
    h_res_prev = torch.from_numpy(rng.uniform(0, 0.5, (M, n, n)).astype(np.float32)).cuda()
    h_post_prev = torch.from_numpy(rng.uniform(0, 2, (M, n)).astype(np.float32)).cuda()
    maps = _maps(rng, n, C)
    phi, coef, bias = _fused_params(maps, n, C, dtype)
    frag = K.phi_fragments(phi)
    eps = float(torch.finfo(dtype).eps)
    w = torch.from_numpy(rng.uniform(0.5, 1.5, C).astype(np.float32)).cuda()
    x_new, li, hp, hq, hr = K.mhc_post_pre_norm(x_old, out, h_res_prev, h_post_prev, frag, coef, bias, eps,
                                                norm_w=w, norm_eps=1e-6)
    x_ref = K.mhc_post(x_old, out, h_res_prev, h_post_prev)
    li_r, hp_r, hq_r, hr_r = K.mhc_pre_norm(x_ref, frag, coef, bias, eps, norm_w=w, norm_eps=1e-6)
    torch.cuda.synchronize()
    assert torch.equal(x_new, x_ref)
    assert torch.equal(li, li_r) and torch.equal(hp, hp_r) and torch.equal(hq, hq_r) and torch.equal(hr, hr_r)
