"""GPU parity: ternary quantisation and the Hadamard-32 linear kernel vs the oracle.

Bars: ternary codes and packed bytes bit-exact; activations
||y - ref|| / ||ref|| <= 1e-5 and max|y - ref| <= 1e-5 * max|ref| for float32,
1e-2 for both in bfloat16 (inputs rounded to bf16 before the oracle runs).
"""
import numpy as np
import pytest
import torch

from oracle import hadamard as ohad
from oracle import ternary as otern

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2}


def rel_errors(y, ref):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    d = y - ref
    n = np.linalg.norm(ref)
    m = np.abs(ref).max()
    return (np.linalg.norm(d) / n if n > 0 else np.linalg.norm(d),
            np.abs(d).max() / m if m > 0 else np.abs(d).max())


def assert_close(y, ref, dtype, what=""):
    r_norm, r_max = rel_errors(y, ref)
    tol = TOL[dtype]
    print(f"{what} rel_norm={r_norm:.3e} rel_max={r_max:.3e} tol={tol}")
    assert r_norm <= tol and r_max <= tol, (what, r_norm, r_max)


@pytest.fixture(scope="module")
def K():
    from src.model import kernels
    return kernels


# --------------------------------------------------------------- ternary

@pytest.mark.parametrize("shape", [(32, 16, 16), (32, 43, 16), (32, 16, 43), (8, 128, 128), (16, 128, 32), (7,)])
def test_gamma_and_codes_bit_exact(K, shape):
    """gamma is the correctly rounded float32 mean of |W| plus 1e-8 (the
    value physics.py:24 approximates), bit for bit, so the codes, packed
    bytes and gamma-scaled values are bit-exact end to end."""
    rng = np.random.default_rng(sum(shape))
    w = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    wt = torch.from_numpy(w).cuda()
    g_rounded = otern.absmean_gamma_rounded(w)
    g_torch = otern.absmean_gamma(w)
    out = K.ternary_quantize(wt, codes=True, packed=True, scaled=True)
    g = np.float32(out["gamma"].item())
    print(f"shape={shape} gamma gpu={g!r} rounded={g_rounded!r} torch-cpu={g_torch!r}")
    assert g.view(np.int32) == g_rounded.view(np.int32)
    c_ref = otern.ternary_codes(w, g_rounded)
    c = out["codes"].cpu().numpy()
    assert np.array_equal(c, c_ref)
    assert np.array_equal(out["packed"].cpu().numpy(), otern.pack_codes(c_ref))
    assert np.array_equal(out["scaled"].cpu().numpy(), c.astype(np.float32) * g)
    assert np.array_equal(K.ternary_unpack(out["packed"], w.shape[-1]).cpu().numpy(), c)
    # codes given any caller gamma (here torch-CPU's): bit-exact as well
    gt = torch.tensor([g_torch], dtype=torch.float32, device="cuda")
    out2 = K.ternary_quantize(wt, gamma=gt, codes=True, packed=True)
    assert np.array_equal(out2["codes"].cpu().numpy(), otern.ternary_codes(w, g_torch))


def test_gamma_and_codes_at_config5_scale(K):
    """Config-5 weight tensors (n_embd 4096: Hadamard linears [32, 128, 128],
    MoE gate/up [128, 128, 32] and down [128, 32, 128]; 48 tensors, 25 M
    weights): the GPU gamma equals the correctly rounded one bit for bit
    and every code is bit-exact.  The codes also equal those of torch-CPU's
    float32 mean (the reference's own gamma, physics.py:24) at 1 thread and
    at the default count: that mean is within an ulp of the correctly
    rounded one and depends on the threads, and no weight of these tensors
    sits close enough to a rounding boundary for the ulp to change a code."""
    import torch as T
    shapes = [(32, 128, 128)] * 24 + [(128, 128, 32)] * 16 + [(128, 32, 128)] * 8
    flips = {1: 0, T.get_num_threads(): 0}
    ulps = {k: 0 for k in flips}
    total = 0
    for i, shape in enumerate(shapes):
        w = (np.random.default_rng(1000 + i).standard_normal(shape) * 0.02).astype(np.float32)
        out = K.ternary_quantize(T.from_numpy(w).cuda(), codes=True)
        g = np.float32(out["gamma"].item())
        g_rounded = otern.absmean_gamma_rounded(w)
        assert g.view(np.int32) == g_rounded.view(np.int32), (i, shape, g, g_rounded)
        c = out["codes"].cpu().numpy()
        assert np.array_equal(c, otern.ternary_codes(w, g_rounded)), (i, shape)
        total += w.size
        nt0 = T.get_num_threads()
        for nt in flips:
            T.set_num_threads(nt)
            g_t = otern.absmean_gamma(w)
            d = abs(int(g_t.view(np.int32)) - int(g.view(np.int32)))
            ulps[nt] = max(ulps[nt], d)
            if d:
                flips[nt] += int(np.count_nonzero(otern.ternary_codes(w, g_t) != c))
        T.set_num_threads(nt0)
    print(f"{len(shapes)} tensors, {total} weights: GPU gamma == correctly rounded gamma; "
          f"codes differing under torch-CPU's float32 mean: {flips} (max gamma distance in ulps {ulps})")
    assert all(v == 0 for v in flips.values()), flips


def test_codes_rounding_boundaries(K):
    # mean |w| = 2 -> gamma = 2 (+1e-8 vanishes): w/gamma hits 0.5 (tie -> 0)
    # and 1.5 (-> 2 -> clamp 1) exactly
    w = np.tile(np.array([1.0, -1.0, 3.0, -3.0], np.float32), 16)
    out = K.ternary_quantize(torch.from_numpy(w).cuda(), codes=True)
    assert out["gamma"].item() == 2.0
    assert out["codes"].cpu().numpy()[:4].tolist() == [0, 0, 1, -1]
    z = K.ternary_quantize(torch.zeros(64, device="cuda"), codes=True)
    assert np.float32(z["gamma"].item()) == np.float32(1e-8)
    assert np.all(z["codes"].cpu().numpy() == 0)


# --------------------------------------------------------------- hadamard linear

def _prepare(K, codes):
    out_o, in_o = codes.shape[1], codes.shape[2]
    packed = torch.from_numpy(otern.pack_codes(codes)).cuda()
    return K.hadamard_prepare(packed, in_o, out_o)


def _run(K, x, codes, alpha, beta, dtype):
    out_o, in_o = codes.shape[1], codes.shape[2]
    kw = _prepare(K, codes)
    xt = torch.from_numpy(np.ascontiguousarray(x)).cuda().to(dtype)
    y = K.hadamard_linear(xt, in_o, out_o, kw, torch.from_numpy(alpha).cuda(), torch.from_numpy(beta).cuda())
    torch.cuda.synchronize()
    return y.float().cpu().numpy(), xt.float().cpu().numpy()


def test_config1_hadamard_linear_fp32(K):
    """Single Hadamard ternary linear, n_embd 512 (16 blocks of 32D), latent
    weights N(0, 0.02) absmean-ternarised, x fp32 N(0,1) [4, 256, 512], seed 0."""
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(4, 256, 512, generator=gen).numpy()
    w = ohad.init_weight(16, 16, gen).numpy()
    codes = otern.ternary_codes(w, otern.absmean_gamma(w))
    hist = np.bincount(codes.reshape(-1) + 1, minlength=3) / codes.size
    print("code histogram -1/0/+1:", hist)
    alpha = np.ones((32, 16), np.float32)
    beta = np.full((32, 16), ohad.beta_init(16), np.float32)
    y, _ = _run(K, x.reshape(-1, 512), codes, alpha, beta, torch.float32)
    ref = ohad.hadamard_linear_f64(x.reshape(-1, 512), codes, alpha, beta)
    assert_close(y, ref, torch.float32, "config1")
    # the reference float32 CPU evaluation order agrees to the same bar
    ref32 = ohad.hadamard_linear_torch32(x.reshape(-1, 512), codes, alpha, beta).numpy()
    assert_close(y, ref32, torch.float32, "config1-vs-torch32")


SHAPES = [(16, 16), (16, 43), (43, 16), (8, 8), (1, 1), (4, 12), (20, 36), (32, 16), (16, 48), (128, 128)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("in_o,out_o", SHAPES)
def test_hadamard_linear_shapes(K, dtype, in_o, out_o):
    rng = np.random.default_rng(in_o * 1000 + out_o)
    M = 77
    codes = rng.integers(-1, 2, size=(32, out_o, in_o)).astype(np.int8)
    alpha = rng.uniform(0.5, 1.5, size=(32, in_o)).astype(np.float32)
    beta = rng.uniform(0.05, 0.3, size=(32, out_o)).astype(np.float32)
    x = rng.standard_normal((M, 32 * in_o)).astype(np.float32)
    y, xq = _run(K, x, codes, alpha, beta, dtype)
    ref = ohad.hadamard_linear_f64(xq, codes, alpha, beta)
    assert_close(y, ref, dtype, f"{dtype} in_o={in_o} out_o={out_o}")


@pytest.mark.parametrize("in_o,out_o,M", [(128, 128, 1), (128, 128, 17), (128, 128, 4200), (64, 64, 300),
                                          (100, 128, 77), (128, 68, 77), (36, 64, 77), (128, 112, 33)])
def test_hadamard_wide_bf16(K, in_o, out_o, M):
    # bf16 layers with 16 < in_o <= 128 and 64 <= out_o <= 128 run the base-3
    # 16x16x32 kernel: partial 32-column chunks (in_o 100, 36), a partial last
    # output tile (68), fewer than 8 output tiles (112, 64), and more 16-row
    # tiles than workgroups (4200 rows)
    rng = np.random.default_rng(in_o * 7 + out_o + M)
    codes = rng.integers(-1, 2, size=(32, out_o, in_o)).astype(np.int8)
    alpha = rng.uniform(0.5, 1.5, size=(32, in_o)).astype(np.float32)
    beta = rng.uniform(0.05, 0.3, size=(32, out_o)).astype(np.float32)
    x = rng.standard_normal((M, 32 * in_o)).astype(np.float32)
    y, xq = _run(K, x, codes, alpha, beta, torch.bfloat16)
    ref = ohad.hadamard_linear_f64(xq, codes, alpha, beta)
    assert_close(y, ref, torch.bfloat16, f"wide in_o={in_o} out_o={out_o} M={M}")


@pytest.mark.parametrize("M", [1, 15, 16, 17, 1000])
def test_hadamard_linear_row_tails(K, M):
    rng = np.random.default_rng(M)
    codes = rng.integers(-1, 2, size=(32, 16, 16)).astype(np.int8)
    alpha = np.ones((32, 16), np.float32)
    beta = np.full((32, 16), 0.25, np.float32)
    x = rng.standard_normal((M, 512)).astype(np.float32)
    for dtype in (torch.float32, torch.bfloat16):
        y, xq = _run(K, x, codes, alpha, beta, dtype)
        assert y.shape == (M, 512)
        assert_close(y, ohad.hadamard_linear_f64(xq, codes, alpha, beta), dtype, f"M={M}")


def test_hadamard_linear_empty_and_strided(K):
    rng = np.random.default_rng(5)
    codes = rng.integers(-1, 2, size=(32, 16, 16)).astype(np.int8)
    kw = _prepare(K, codes)
    a = torch.ones(32, 16, device="cuda")
    b = torch.full((32, 16), 0.25, device="cuda")
    y0 = K.hadamard_linear(torch.empty(0, 512, device="cuda"), 16, 16, kw, a, b)
    assert y0.shape == (0, 512)
    # a column slice of a wider buffer (row stride 1536) is read in place
    big = torch.from_numpy(rng.standard_normal((50, 1536)).astype(np.float32)).cuda()
    xs = big[:, 512:1024]
    y = K.hadamard_linear(xs, 16, 16, kw, a, b)
    ref = ohad.hadamard_linear_f64(xs.cpu().numpy(), codes, np.ones((32, 16)), np.full((32, 16), 0.25))
    assert_close(y.cpu().numpy(), ref, torch.float32, "strided")


def test_hadamard_linear_closed_form_identity(K):
    # all codes +1 with in_o = out_o = 1 makes the layer y = beta*alpha*x
    codes = np.ones((32, 1, 1), np.int8)
    x = np.random.default_rng(6).standard_normal((33, 32)).astype(np.float32)
    y, _ = _run(K, x, codes, np.full((32, 1), 2.0, np.float32), np.full((32, 1), 0.5, np.float32), torch.float32)
    assert np.max(np.abs(y - x)) < 1e-6


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("in_o,hid_o", [(16, 43), (16, 16), (8, 21), (4, 12)])
def test_hadamard_swiglu_and_padded_down(K, dtype, in_o, hid_o):
    """silu(gate(x)) * up(x) into the group-padded layout, then down_proj
    reading it in place, against the oracle's three separate layers."""
    rng = np.random.default_rng(in_o * 100 + hid_o)
    M = 70
    cg = rng.integers(-1, 2, size=(32, hid_o, in_o)).astype(np.int8)
    cu = rng.integers(-1, 2, size=(32, hid_o, in_o)).astype(np.int8)
    cd = rng.integers(-1, 2, size=(32, in_o, hid_o)).astype(np.int8)
    ag, au = (rng.uniform(0.5, 1.5, (32, in_o)).astype(np.float32) for _ in range(2))
    bg, bu = (rng.uniform(0.1, 0.4, (32, hid_o)).astype(np.float32) for _ in range(2))
    ad = rng.uniform(0.5, 1.5, (32, hid_o)).astype(np.float32)
    bd = rng.uniform(0.1, 0.4, (32, in_o)).astype(np.float32)
    x = rng.standard_normal((M, 32 * in_o)).astype(np.float32)
    t = lambda a: torch.from_numpy(a).cuda()  # noqa: E731
    xt = t(x).to(dtype)
    h = K.hadamard_swiglu(xt, in_o, hid_o, (_prepare(K, cg), t(ag), t(bg)), (_prepare(K, cu), t(au), t(bu)))
    gsh = ((hid_o + 3) // 4) * 4
    assert h.shape == (M, 32 * gsh)
    hv = h.float().cpu().numpy().reshape(M, 32, gsh)
    assert np.all(hv[:, :, hid_o:] == 0)                     # pad slots are exact zeros
    xq = xt.float().cpu().numpy().astype(np.float64)
    g = ohad.hadamard_linear_f64(xq, cg, ag, bg)
    u = ohad.hadamard_linear_f64(xq, cu, au, bu)
    h_ref = g / (1 + np.exp(-g)) * u
    assert_close(hv[:, :, :hid_o].reshape(M, -1), h_ref, dtype, f"swiglu h {dtype} {in_o}->{hid_o}")
    y = K.hadamard_linear(h, hid_o, in_o, _prepare(K, cd), t(ad), t(bd), gsx=gsh)
    hq = hv[:, :, :hid_o].reshape(M, -1).astype(np.float64)
    assert_close(y.float().cpu().numpy(), ohad.hadamard_linear_f64(hq, cd, ad, bd), dtype, f"down {dtype}")


@pytest.mark.parametrize("M,in_o,hid_o", [(8192, 16, 43), (20000, 16, 43), (100, 16, 48), (1, 16, 43),
                                          (700, 16, 32), (333, 12, 20)])
def test_hadamard_mlp_equals_swiglu_then_down(K, M, in_o, hid_o):
    """walsh_hadamard_mlp_fwd (the whole SwiGLU MLP in one launch, the hidden
    activation on chip) against walsh_hadamard_swiglu_fwd followed by the
    down projection reading the padded hidden layout: bitwise.  20,000 rows
    give a workgroup several 16-token tiles (the chunk areas reused across
    tiles); hid_o 20 / 32 take two hidden tiles, 43 / 48 three; 1 and 333
    rows leave partial tiles.  The output also against the float64 oracle of
    the three layers."""
    out_o = in_o
    print(f"mlp case M={M} in_o={in_o} hid_o={hid_o}", flush=True)
    rng = np.random.default_rng(M + hid_o)
    cg = rng.integers(-1, 2, size=(32, hid_o, in_o)).astype(np.int8)
    cu = rng.integers(-1, 2, size=(32, hid_o, in_o)).astype(np.int8)
    cd = rng.integers(-1, 2, size=(32, out_o, hid_o)).astype(np.int8)
    ag, au = (rng.uniform(0.5, 1.5, (32, in_o)).astype(np.float32) for _ in range(2))
    bg, bu = (rng.uniform(0.1, 0.4, (32, hid_o)).astype(np.float32) for _ in range(2))
    ad = rng.uniform(0.5, 1.5, (32, hid_o)).astype(np.float32)
    bd = rng.uniform(0.1, 0.4, (32, out_o)).astype(np.float32)
    t = lambda a: torch.from_numpy(a).cuda()  # noqa: E731
    gen = torch.Generator(device="cuda").manual_seed(M)
    x = torch.randn(M, 32 * in_o, device="cuda", generator=gen).bfloat16()
    gate, up, down = (_prepare(K, cg), t(ag), t(bg)), (_prepare(K, cu), t(au), t(bu)), (_prepare(K, cd), t(ad), t(bd))
    assert K.hadamard_mlp_supported(x, in_o, hid_o, out_o)
    y = K.hadamard_mlp(x, in_o, hid_o, out_o, gate, up, down)
    h = K.hadamard_swiglu(x, in_o, hid_o, gate, up)
    gsh = ((hid_o + 3) // 4) * 4
    y2 = K.hadamard_linear(h, hid_o, out_o, *down, gsx=gsh)
    torch.cuda.synchronize()
    nd = int((y.view(torch.int16) != y2.view(torch.int16)).sum())
    print(f"mlp M={M} hid_o={hid_o}: {nd} of {y.numel()} outputs differ bitwise from the two launches", flush=True)
    assert nd == 0
    rows = np.unique(np.r_[0, M - 1, rng.integers(0, M, 64)])
    xq = x[torch.from_numpy(rows).cuda()].float().cpu().numpy().astype(np.float64)
    g = ohad.hadamard_linear_f64(xq, cg, ag, bg)
    u = ohad.hadamard_linear_f64(xq, cu, au, bu)
    ref = ohad.hadamard_linear_f64(g / (1 + np.exp(-g)) * u, cd, ad, bd)
    assert_close(y[torch.from_numpy(rows).cuda()].float().cpu().numpy(), ref, torch.bfloat16, f"mlp M={M}")


def test_launch_timer_records_kernel_time(K):
    """walsh_timing_*: every entry-point call inside LaunchTimer gets its
    kernel's own duration (hipExtLaunchKernelGGL events)."""
    from src.model import _hip
    from src.model.hadamard import HadamardLinear
    torch.manual_seed(0)
    lin = HadamardLinear(512, 512).cuda()
    x = torch.randn(4096, 512, device="cuda")
    lin(x)
    with _hip.LaunchTimer() as lt:
        for _ in range(3):
            lin(x)
    s = lt.summary()
    assert len(s) == 1
    (name, d), = s.items()
    assert name.startswith("hadamard_fwd_kernel") and d["launches"] == 3
    assert 0.0 < d["ms"] < 100.0
    # timing is off again: untimed launches still work
    lin(x)
    torch.cuda.synchronize()


# --------------------------------------------------------------- head mixer

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,T,D", [(2, 64, 16), (1, 17, 16), (3, 5, 8), (2, 9, 12), (1, 33, 32), (2, 7, 5)])
def test_head_mixer_vs_oracle(K, dtype, B, T, D):
    rng = np.random.default_rng(B * 100 + T * 10 + D)
    x = rng.standard_normal((B, 32, T, D)).astype(np.float32)
    W = (rng.standard_normal((32, D, D)) * 0.2).astype(np.float32)
    beta = rng.uniform(0.1, 0.5, size=D).astype(np.float32)
    xt = torch.from_numpy(x).cuda().to(dtype)
    Wt = torch.from_numpy(W).cuda()
    kw = K.head_mixer_prepare(Wt, dtype)
    y = K.head_mixer(xt, kw, torch.from_numpy(beta).cuda())
    torch.cuda.synchronize()
    assert y.shape == (B, T, 32 * D)
    Wq = Wt.to(dtype).float().cpu().numpy()   # the weights the matrix cores see
    ref = ohad.head_mixer_f64(xt.float().cpu().numpy(), Wq, beta).transpose(0, 2, 1, 3).reshape(B, T, 32 * D)
    assert_close(y.float().cpu().numpy(), ref, dtype, f"mixer {dtype} B={B} T={T} D={D}")


def test_head_mixer_group_view_and_output_slice(K):
    # heads 32..63 of a 64-head attention output, written into the second
    # half of token-major [B, T, 64*D] rows
    rng = np.random.default_rng(11)
    B, T, D = 2, 40, 16
    x = rng.standard_normal((B, 64, T, D)).astype(np.float32)
    W = (rng.standard_normal((32, D, D)) * 0.2).astype(np.float32)
    beta = rng.uniform(0.1, 0.5, size=D).astype(np.float32)
    xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    kw = K.head_mixer_prepare(torch.from_numpy(W).cuda(), torch.bfloat16)
    out = torch.zeros(B, T, 64 * D, device="cuda", dtype=torch.bfloat16)
    K.head_mixer(xt.view(B, 2, 32, T, D)[:, 1], kw, torch.from_numpy(beta).cuda(), out=out[:, :, 32 * D:])
    torch.cuda.synchronize()
    Wq = torch.from_numpy(W).to(torch.bfloat16).float().numpy()
    ref = ohad.head_mixer_f64(xt[:, 32:].float().cpu().numpy(), Wq, beta).transpose(0, 2, 1, 3).reshape(B, T, 32 * D)
    o = out.float().cpu().numpy()
    assert np.all(o[:, :, :32 * D] == 0)
    assert_close(o[:, :, 32 * D:], ref, torch.bfloat16, "mixer group view")


@torch.no_grad()
def test_head_mixer_module_matches_torch_path():
    from src.model.hadamard import HadamardHeadMixerFused
    torch.manual_seed(3)
    m = HadamardHeadMixerFused(16)
    x = torch.randn(2, 32, 24, 16)
    ref = m(x)                       # CPU: the reference's three products in torch
    mg = m.cuda()
    y = mg(x.cuda())                 # GPU: walsh_head_mixer_fwd (float32)
    torch.cuda.synchronize()
    assert y.shape == ref.shape
    assert_close(y.cpu().numpy(), ref.detach().numpy(), torch.float32, "mixer module f32")
    with torch.autocast("cuda", dtype=torch.bfloat16):
        yb = mg(x.cuda().to(torch.bfloat16))
    assert yb.dtype == torch.bfloat16
    assert_close(yb.float().cpu().numpy(), ref.detach().numpy(), torch.bfloat16, "mixer module bf16")


# --------------------------------------------------------------- fused rotary embedding

def _freqs_cis(T, D, start=0):
    f = 1.0 / (10000.0 ** (torch.arange(0, D, 2)[: D // 2].float() / D))
    ang = torch.outer(torch.arange(start, start + T).float(), f)
    return torch.polar(torch.ones_like(ang), ang)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("in_o,out_o,D,B,T", [(16, 16, 16, 2, 40), (16, 16, 8, 3, 7), (128, 128, 128, 2, 37),
                                                (16, 32, 16, 1, 20), (64, 64, 64, 2, 17)])
def test_hadamard_linear_rope(K, dtype, in_o, out_o, D, B, T):
    rng = np.random.default_rng(in_o + out_o + D + T)
    codes = rng.integers(-1, 2, size=(32, out_o, in_o)).astype(np.int8)
    alpha = rng.uniform(0.5, 1.5, size=(32, in_o)).astype(np.float32)
    beta = rng.uniform(0.05, 0.3, size=(32, out_o)).astype(np.float32)
    x = rng.standard_normal((B, T, 32 * in_o)).astype(np.float32)
    kw = _prepare(K, codes)
    xt = torch.from_numpy(x).cuda().to(dtype)
    fc = _freqs_cis(T, D, start=5)
    y = K.hadamard_linear_rope(xt, in_o, out_o, kw, torch.from_numpy(alpha).cuda(), torch.from_numpy(beta).cuda(),
                               fc.cuda(), D)
    torch.cuda.synchronize()
    lin = ohad.hadamard_linear_f64(xt.float().cpu().numpy().reshape(B * T, -1), codes, alpha, beta)
    ref = ohad.rope_f64(lin.reshape(B, T, -1), fc.numpy(), D)
    assert_close(y.float().cpu().numpy(), ref, dtype, f"rope {dtype} in_o={in_o} out_o={out_o} D={D}")


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 128), (torch.bfloat16, 16), (torch.float32, 16)])
@pytest.mark.parametrize("T", [1, 48])
def test_head_mixer_batch_one_with_short_batch_stride(K, dtype, D, T):
    """The attention output of one sequence as the model hands it over:
    x = y.view(1, 1, 32, T, D)[:, 0] of a token-major [1, 32, T, D] tensor,
    whose size-1 batch dimension carries the token stride (32 D), shorter
    than the T rows it holds.  Every row must be read (the input buffer's
    extent comes from all three strides, not from B x batch stride)."""
    rng = np.random.default_rng(T + D)
    base = torch.from_numpy(rng.standard_normal((1, T, 32, D)).astype(np.float32)).cuda().to(dtype)
    x = base.as_strided((1, 32, T, D), (32 * D, D, 32 * D, 1))
    assert x.stride(0) < (T - 1) * x.stride(2) + 32 * D or T == 1
    W = (rng.standard_normal((32, D, D)) * 0.05).astype(np.float32)
    beta = rng.uniform(0.1, 0.5, size=D).astype(np.float32)
    Wt = torch.from_numpy(W).cuda()
    kw = K.head_mixer_prepare(Wt, dtype)
    y = K.head_mixer(x, kw, torch.from_numpy(beta).cuda())
    torch.cuda.synchronize()
    Wq = Wt.to(dtype).float().cpu().numpy()
    ref = ohad.head_mixer_f64(x.float().cpu().numpy(), Wq, beta).transpose(0, 2, 1, 3).reshape(1, T, 32 * D)
    assert_close(y.float().cpu().numpy(), ref, dtype, f"mixer B=1 T={T} D={D} {dtype} short batch stride")


@pytest.mark.parametrize("B,T,D", [(2, 40, 128), (1, 17, 64), (3, 5, 96), (1, 300, 128)])
def test_head_mixer_wide_bf16(K, B, T, D):
    # head_dim above 32 in bf16: the wide kernel with streamed dense weights
    rng = np.random.default_rng(B + T + D)
    x = rng.standard_normal((B, 32, T, D)).astype(np.float32)
    W = (rng.standard_normal((32, D, D)) * 0.05).astype(np.float32)
    beta = rng.uniform(0.1, 0.5, size=D).astype(np.float32)
    xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    Wt = torch.from_numpy(W).cuda()
    kw = K.head_mixer_prepare(Wt, torch.bfloat16)
    y = K.head_mixer(xt, kw, torch.from_numpy(beta).cuda())
    torch.cuda.synchronize()
    Wq = Wt.to(torch.bfloat16).float().cpu().numpy()
    ref = ohad.head_mixer_f64(xt.float().cpu().numpy(), Wq, beta).transpose(0, 2, 1, 3).reshape(B, T, 32 * D)
    assert_close(y.float().cpu().numpy(), ref, torch.bfloat16, f"wide mixer B={B} T={T} D={D}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("in_o,out_o,T", [(16, 16, 1024), (16, 16, 37), (64, 64, 20), (128, 128, 1100),
                                           (100, 128, 700)])
def test_hadamard_linear_multi_equals_single_launches(K, dtype, in_o, out_o, T):
    """walsh_hadamard_linear_multi_fwd (q, k with RoPE, v in one launch) is
    bitwise the three single-layer calls, also for the bf16 n_embd-4096
    shapes above 256 rows (one wide launch per layer)."""
    torch.manual_seed(in_o + T)
    B, D = 2, 16
    x = torch.randn(B, T, 32 * in_o, device="cuda").to(dtype)
    f = _freqs_cis(T, D).cuda()
    layers, singles = [], []
    for i, rope in enumerate((True, True, False)):
        w = torch.randn(32, out_o, in_o) * 0.02
        q = K.ternary_quantize(w.cuda(), packed=True)
        kw = K.hadamard_prepare(q["packed"], in_o, out_o)
        a = (1 + 0.3 * torch.randn(32, in_o)).cuda()
        b = (0.2 * torch.randn(32, out_o)).cuda()
        layers.append((kw, a, b, rope))
        singles.append(K.hadamard_linear_rope(x, in_o, out_o, kw, a, b, f, D) if rope
                       else K.hadamard_linear(x, in_o, out_o, kw, a, b))
    outs = K.hadamard_linear_multi(x, in_o, out_o, layers, f, D)
    torch.cuda.synchronize()
    for o, s in zip(outs, singles):
        assert torch.equal(o, s)


@pytest.mark.parametrize("rope", [False, True])
def test_bf16_kernels_bitwise_across_tile_counts(K, rope):
    """bf16 16x16 layers take wavefront pairs up to 1024 16-row tiles on
    contiguous rows (2048 on strided ones) and the pipelined one-wavefront
    kernel above; that kernel moves whole 512-value rows through per-wave LDS
    areas when the rows are contiguous, and 32-byte row segments per lane quad
    otherwise, for one layer or several in one launch.  All compute the same
    butterflies in the same order, so their outputs are equal bitwise."""
    torch.manual_seed(11 + rope)
    B, T, D = 5, 8001, 16   # 40005 rows: 2501 tiles, the last one ragged
    codes = np.random.default_rng(11 + rope).integers(-1, 2, size=(32, 16, 16)).astype(np.int8)
    kw = _prepare(K, codes)
    a = (1 + 0.3 * torch.randn(32, 16)).cuda()
    b = (0.2 * torch.randn(32, 16)).cuda()
    x = torch.randn(B, T, 512, device="cuda").to(torch.bfloat16)
    wide = torch.zeros(B, T, 1024, device="cuda", dtype=torch.bfloat16)
    wide[:, :, 256:768] = x
    xs = wide[:, :, 256:768]   # same values at row stride 1024
    f = _freqs_cis(T, D).cuda()

    def run(v):
        return K.hadamard_linear_rope(v, 16, 16, kw, a, b, f, D) if rope else K.hadamard_linear(v, 16, 16, kw, a, b)
    y = run(x)           # whole rows through LDS
    y_seg = run(xs)      # row segments
    y_pair = run(x[:2])  # 16002 rows: wavefront pairs
    plain = K.hadamard_linear(x, 16, 16, kw, a, b)
    multi = K.hadamard_linear_multi(x, 16, 16, [(kw, a, b, rope), (kw, a, b, False)], f, D)
    torch.cuda.synchronize()
    assert torch.equal(y, y_seg)
    assert torch.equal(y[:2], y_pair)
    assert torch.equal(multi[0], y) and torch.equal(multi[1], plain)
    if not rope:
        tail = x[-1, -7:].float().cpu().numpy()
        ref = ohad.hadamard_linear_f64(tail, codes, a.cpu().numpy(), b.cpu().numpy())
        assert_close(y[-1, -7:].float().cpu().numpy(), ref, torch.bfloat16, "last rows")


@pytest.mark.parametrize("in_o", [24, 43, 64])
def test_bf16_chunk_kernels_bitwise_across_tile_counts(K, in_o):
    """bf16 layers with 2-4 input chunks and one output tile run on one
    wavefront pair per chunk and tile up to 2048 tiles, and on the
    one-wavefront chunk loop above; both accumulate the chunks in order
    through one matrix-core chain, so their outputs are equal bitwise."""
    rng = np.random.default_rng(in_o)
    torch.manual_seed(in_o)
    M = 2048 * 16 + 35   # 2051 tiles
    codes = rng.integers(-1, 2, size=(32, 16, in_o)).astype(np.int8)
    kw = _prepare(K, codes)
    a = (1 + 0.3 * torch.randn(32, in_o)).cuda()
    b = (0.2 * torch.randn(32, 16)).cuda()
    x = torch.randn(M, 32 * in_o, device="cuda").to(torch.bfloat16)
    y = K.hadamard_linear(x, in_o, 16, kw, a, b)
    y_pair = K.hadamard_linear(x[:5003], in_o, 16, kw, a, b)   # 313 tiles, the last one ragged
    torch.cuda.synchronize()
    assert torch.equal(y[:5003], y_pair)
    ref = ohad.hadamard_linear_f64(x[4996:5003].float().cpu().numpy(), codes, a.cpu().numpy(), b.cpu().numpy())
    assert_close(y_pair[-7:].float().cpu().numpy(), ref, torch.bfloat16, f"in_o={in_o} last rows")


@pytest.mark.parametrize("B,T,layout", [(8, 1024, "heads"), (3, 37, "heads"), (2, 50, "tokens"),
                                        (24, 1024, "heads"), (24, 1024, "tokens")])
def test_head_mixer_proj_bitwise_two_launches(K, B, T, layout):
    """walsh_head_mixer_proj_fwd (the head mixer and the 16x16 output
    projection in one launch) equals walsh_head_mixer_fwd followed by
    walsh_hadamard_linear_fwd bitwise, on head-major x and on the attention
    output's token-major layout viewed head-major.  At 24 x 1024 rows (1,536
    tiles) the grid holds fewer wavefront pairs than tiles, so pairs loop
    over several tiles and reuse their LDS exchange areas; the model's
    callers stop at 16,384 rows, the C entry point takes any count."""
    torch.manual_seed(B * T)
    D = 16
    if layout == "heads":
        x = torch.randn(B, 32, T, D, device="cuda").to(torch.bfloat16)
    else:
        x = torch.randn(B, T, 32, D, device="cuda").to(torch.bfloat16).transpose(1, 2)
    W = torch.randn(32, D, D, device="cuda") * 0.2
    mkw = K.head_mixer_prepare(W, torch.bfloat16)
    mbeta = (1 + 0.1 * torch.randn(D)).cuda()
    codes = np.random.default_rng(B + T).integers(-1, 2, size=(32, 16, 16)).astype(np.int8)
    pkw = _prepare(K, codes)
    pa = (1 + 0.3 * torch.randn(32, 16)).cuda()
    pb = (0.2 * torch.randn(32, 16)).cuda()
    assert K.head_mixer_proj_supported(x, B * T) == (B * T <= 16 * K.PAIR_MAX_TILES_ROWS)
    y = K.head_mixer_proj(x, mkw, mbeta, pkw, pa, pb)
    mid = K.head_mixer(x, mkw, mbeta)
    ref = K.hadamard_linear(mid.view(B * T, 512), 16, 16, pkw, pa, pb).view(B, T, 512)
    torch.cuda.synchronize()
    assert torch.equal(y, ref)


# --------------------------------------------------------------- decode-sized batches

@pytest.mark.parametrize("in_o,out_o", [(128, 128), (100, 128), (128, 68), (36, 64)])
def test_split_kernel_bitwise_equals_wide_kernel(K, in_o, out_o):
    """Row counts up to 256 of the bf16 wide shapes run the split kernel
    (one workgroup per token tile and output tile), larger ones the wide3
    kernel: both round and sum in the same order, so the first k rows of a
    512-row call equal a k-row call bitwise, for the plain linear, the RoPE
    variant and the three-layer q/k/v launch."""
    torch.manual_seed(in_o + out_o)
    T, D = 512, 4 if out_o % 128 else 128
    x = torch.randn(1, T, 32 * in_o, device="cuda").to(torch.bfloat16)
    f = _freqs_cis(T, D).cuda()
    layers = []
    for rope in (True, True, False):
        w = torch.randn(32, out_o, in_o) * 0.02
        q = K.ternary_quantize(w.cuda(), packed=True)
        kw = K.hadamard_prepare(q["packed"], in_o, out_o)
        layers.append((kw, (1 + 0.3 * torch.randn(32, in_o)).cuda(), (0.2 * torch.randn(32, out_o)).cuda(), rope))
    kw, a, b, _ = layers[0]
    big = K.hadamard_linear(x, in_o, out_o, kw, a, b)
    big_rope = K.hadamard_linear_rope(x, in_o, out_o, kw, a, b, f, D)
    big_multi = K.hadamard_linear_multi(x, in_o, out_o, layers, f, D)
    for k in (1, 5, 16, 33, 256):
        xs = x[:, :k]
        assert torch.equal(K.hadamard_linear(xs, in_o, out_o, kw, a, b), big[:, :k]), k
        assert torch.equal(K.hadamard_linear_rope(xs, in_o, out_o, kw, a, b, f[:k], D), big_rope[:, :k]), k
        for o, ref in zip(K.hadamard_linear_multi(xs, in_o, out_o, layers, f[:k], D), big_multi):
            assert torch.equal(o, ref[:, :k]), k


@pytest.mark.parametrize("B,D", [(1, 128), (3, 96)])
def test_split_head_mixer_bitwise_equals_wide_kernel(K, B, D):
    """The head mixer at head_dim above 32 in bf16: B * T rows up to 256 run
    the split kernel; the first k positions of a 512-position call equal a
    k-position call (a strided view of the same tensor) bitwise."""
    rng = np.random.default_rng(B * D)
    T = 512 // B + 1
    x = torch.from_numpy(rng.standard_normal((B, 32, T, D)).astype(np.float32)).cuda().to(torch.bfloat16)
    W = torch.from_numpy((rng.standard_normal((32, D, D)) * 0.05).astype(np.float32)).cuda()
    beta = torch.from_numpy(rng.uniform(0.1, 0.5, size=D).astype(np.float32)).cuda()
    kw = K.head_mixer_prepare(W, torch.bfloat16)
    big = K.head_mixer(x, kw, beta)
    for k in (1, 7, 16, 256 // B):
        assert torch.equal(K.head_mixer(x[:, :, :k], kw, beta), big[:, :k]), k
