"""The oracle against the reference's own outputs (tests/golden fixtures).

The fixtures were written by ``tests/golden/make_fixtures.py`` from the
reference's ``src.model`` modules on the CPU (float32, eval mode, perturbed
parameters).  These tests pin

* the assembled model oracle (``oracle/model.py``): mHCWalsh.forward
  (src/model/mhc.py:617-681), mHCLlamaBlock.forward (mhc.py:507-534),
  CausalSelfAttention.forward (src/model/chassis.py:424-483), SwiGLUMLP,
  HadamardMoE and channel modulation, end to end;
* each function-level oracle against the reference module it restates;
* each method of the assembled oracle against the function-level oracle of
  the same step (so both restatements agree and one of them is pinned).

Bars: float32 reference against a float32 or float64 restatement, 1e-5
relative (norm) and the same on the maximum; codes and expert masks exact.
"""
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oatt
from oracle import hadamard as ohad
from oracle import mhc as omhc
from oracle import moe as omoe
from oracle import octonion as ooct
from oracle import ternary as otern
from oracle.model import Oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 1e-5


def load(name):
    path = os.path.join(GOLDEN, name)
    if not os.path.exists(path):
        pytest.skip(f"fixture {name} not present")
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def section(fx, prefix):
    n = len(prefix) + 1
    return {k[n:]: torch.from_numpy(v.copy()) for k, v in fx.items() if k.startswith(prefix + "/")}


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = max(np.linalg.norm(b), 1e-30)
    return np.linalg.norm(a - b) / den, np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)


def assert_close(a, b, tol=TOL, what=""):
    r_norm, r_max = rel(a, b)
    assert r_norm <= tol and r_max <= 10 * tol, f"{what}: rel {r_norm:.3e}, max-rel {r_max:.3e} (bar {tol})"


def model_oracle(fx, **kw):
    c = {k[4:]: (str(v) if v.dtype.kind == "U" else int(v)) for k, v in fx.items() if k.startswith("cfg/")}
    sd = section(fx, "sd")
    return Oracle(sd, n_embd=c["n_embd"], n_head=c["n_head"], n_layer=c["n_layer"], n_streams=4,
                  head_mixing=bool(c["head_mixing"]), block_size=c["block_size"], use_moe=bool(c["use_moe"]),
                  moe_max_experts=c["max_experts"], use_channel_mod=bool(c["use_channel_mod"]),
                  algebra=c.get("algebra", "hadamard"), **kw), c


# --------------------------------------------------------------- whole model
@pytest.mark.parametrize("name", ["model_c64.npz", "model_c96_moe.npz", "model_oct_c64.npz"])
def test_model_oracle_matches_reference(name):
    """oracle/model.py reproduces mHCWalsh.forward of the reference: the
    last-position logits, the final hidden states of every position and the
    training loss (mhc.py:617-681)."""
    fx = load(name)
    orc, cfg = model_oracle(fx)
    idx = torch.from_numpy(fx["in/idx"])
    targets = torch.from_numpy(fx["in/targets"])
    seen = []
    if cfg["use_moe"]:
        moe = orc.moe

        def traced(x, p):
            out, info = moe(x, p)
            seen.append(info["mask"])
            return out, info
        orc.moe = traced
    with torch.no_grad():
        logits, ho = orc.forward(idx, return_hidden=True)
        loss = orc.loss(idx, targets)
    assert_close(logits.numpy(), fx["out/logits_last"], what="last-position logits")
    assert_close(ho.numpy(), fx["out/h_out"], what="final hidden states")
    full = (ho @ orc.sd["output.weight"].t()).numpy()
    assert_close(full, fx["out/logits_all"], what="all-position logits")
    assert abs(float(loss) - float(fx["out/loss"])) <= TOL * abs(float(fx["out/loss"]))
    if cfg["use_moe"]:
        # the loss pass ran the layers again: the first n_layer masks belong to forward()
        for l in range(cfg["n_layer"]):
            assert np.array_equal(seen[l].numpy(), fx[f"out/moe_mask_{l}"]), f"layer {l} expert mask"


def test_octonion_model_fixture_discriminates():
    """The octonion model fixture (algebra "octonion", the CPU module
    OctonionTernaryLinearRef and the pure-torch OctonionHeadMixer) catches
    an octonion layer with W[i^j] transposed per block, the head mixer
    applied with its weights transposed (chassis.py:395 multiplies by W, not
    W^T), and the conjugate sign table (x_j and w swapped in the product)."""
    from oracle import model as omodel
    fx = load("model_oct_c64.npz")
    idx = torch.from_numpy(fx["in/idx"])
    ref = fx["out/logits_last"]

    def run(orc):
        with torch.no_grad():
            return orc.forward(idx).numpy()
    orc, _ = model_oracle(fx)
    assert rel(run(orc), ref)[0] <= TOL
    # per-block transposed weights: only square blocks (in_o == out_o) take it
    orc, _ = model_oracle(fx)
    base = orc.octonion_linear

    def lin_t(x, p):
        w = orc.codes(p + '.weight')
        if w.shape[1] != w.shape[2]:
            return base(x, p)
        orc._codes[p + '.weight'] = w.transpose(1, 2).contiguous()
        try:
            return base(x, p)
        finally:
            orc._codes[p + '.weight'] = w
    orc.octonion_linear = lin_t
    assert rel(run(orc), ref)[0] > 100 * TOL
    # head mixer with W^T
    orc, _ = model_oracle(fx)
    for k in list(orc.sd):
        if k.endswith("head_mixer.W"):
            orc.sd[k] = orc.sd[k].transpose(1, 2).contiguous()
    assert rel(run(orc), ref)[0] > 100 * TOL
    # conjugate signs: S[i][j] of x . w replaced by that of w . x (S[j][i]
    # with the non-scalar cross terms negated)
    saved = omodel.OCT_SIGN
    try:
        omodel.OCT_SIGN = tuple(tuple(saved[i][j] if (i == 0 or j == 0 or i == j) else -saved[i][j]
                                      for j in range(8)) for i in range(8))
        orc, _ = model_oracle(fx)
        assert rel(run(orc), ref)[0] > 100 * TOL
    finally:
        omodel.OCT_SIGN = saved


def test_octonion_gpu_semantics_mode_is_bf16_close():
    """The oracle's octonion_gpu mode (the reference GPU module's bf16
    roundings) stays within bf16 reach of the CPU reference's float32 model
    and is not identical to it."""
    fx = load("model_oct_c64.npz")
    idx = torch.from_numpy(fx["in/idx"])
    orc, _ = model_oracle(fx, octonion_gpu=True)
    with torch.no_grad():
        out = orc.forward(idx).numpy()
    r = rel(out, fx["out/logits_last"])[0]
    assert 1e-5 < r < 3e-2, r


def test_model_fixture_discriminates():
    """The fixture catches plausible composition mistakes: dropping the head
    mixer, mixing the streams with H_res transposed, or taking the first
    instead of the last position all move the logits far beyond the bar."""
    fx = load("model_c64.npz")
    idx = torch.from_numpy(fx["in/idx"])
    ref = fx["out/logits_last"]

    orc, _ = model_oracle(fx)
    orc.head_mixing = False
    with torch.no_grad():
        assert rel(orc.forward(idx).numpy(), ref)[0] > 1e-2

    orc, _ = model_oracle(fx)
    stream = orc.stream

    def transposed_res(x, p, layer_fn):  # H_res^T instead of H_res
        B, T, n, C = x.shape
        xf = x.reshape(B, T, n * C)
        hp = orc.mapping(xf, p + '.H_pre', 'pre')
        hq = orc.mapping(xf, p + '.H_post', 'post')
        hr = orc.mapping(xf, p + '.H_res', 'res').transpose(-2, -1)
        out = layer_fn(torch.matmul(hp, x).squeeze(2))
        return torch.matmul(hr, x) + torch.matmul(hq.transpose(-2, -1), out.unsqueeze(2))
    orc.stream = transposed_res
    with torch.no_grad():
        assert rel(orc.forward(idx).numpy(), ref)[0] > 1e-3
    orc.stream = stream

    orc, _ = model_oracle(fx)
    with torch.no_grad():
        _, ho = orc.forward(idx, return_hidden=True)
        first = ho[:, [0], :] @ orc.sd["output.weight"].t()
    assert rel(first.numpy(), ref)[0] > 1e-2


# --------------------------------------------------------------- layers
def test_hadamard_linear_oracles_match_reference():
    """HadamardLinear (fht_cuda.py:489-519): hadamard_linear_f64 with the
    oracle's codes, and the model oracle's float32 method, reproduce the
    reference's output; the codes come from the oracle's absmean quantiser."""
    fx = load("hadamard_linear.npz")
    sd = section(fx, "sd")
    x = fx["in/x"].reshape(-1, 512)
    w = sd["weight"].numpy()
    codes = otern.ternary_codes(w, otern.absmean_gamma(w))
    assert set(np.unique(codes)) <= {-1, 0, 1}
    y = ohad.hadamard_linear_f64(x, codes, sd["alpha"].numpy(), sd["beta"].numpy())
    assert_close(y, fx["out/y"].reshape(-1, 512), what="hadamard_linear_f64")
    orc = Oracle({"l.weight": sd["weight"], "l.alpha": sd["alpha"], "l.beta": sd["beta"]},
                 n_embd=512, n_head=16, n_layer=0)
    with torch.no_grad():
        y32 = orc.hadamard_linear(torch.from_numpy(x), "l")
    assert_close(y32.numpy(), fx["out/y"].reshape(-1, 512), what="Oracle.hadamard_linear")


def test_octonion_oracle_matches_reference():
    """OctonionTernaryLinearRef (physics.py:53-82) on 8 parts of 8 features."""
    fx = load("octonion_ref.npz")
    sd = section(fx, "sd")
    x = fx["in/x"].reshape(-1, 64)
    w = sd["weight"].numpy()
    codes = otern.ternary_codes(w, otern.absmean_gamma(w))
    parts = np.stack(np.split(x, 8, axis=-1))
    y = ooct.octonion_linear_f64(parts, codes, sd["beta"].numpy())
    y = np.concatenate(list(y), axis=-1)
    assert_close(y, fx["out/y"].reshape(-1, 64), what="octonion_linear_f64")


def test_sinkhorn_oracle_matches_reference():
    """SinkhornKnopp (mhc.py:214-229) in float32 and float64; the fixture
    includes h = 0 (uniform 1/n) and h = 2I."""
    fx = load("sinkhorn.npz")
    h, y = fx["in/h"], fx["out/y"]
    assert_close(omhc.sinkhorn(h, dtype=np.float32), y, what="float32")
    assert_close(omhc.sinkhorn(h), y, what="float64")
    np.testing.assert_allclose(y[0], np.full((4, 4), 0.25), rtol=1e-6)


@pytest.mark.parametrize("kind", ["res", "pre", "post"])
def test_mapping_oracles_match_reference(kind):
    """ResidualStreamMapping (mhc.py:283-318) at n_embd 64, 4 streams:
    oracle.mhc.mapping (float64) and Oracle.mapping (float32)."""
    fx = load("mapping_c64.npz")
    s = section(fx, f"sd_{kind}")
    x = fx["in/x"]
    xf = x.reshape(-1, 4 * 64)
    h = omhc.mapping(xf, s["phi.weight"].numpy(), float(s["alpha"]), s["bias"].numpy(), kind, 4,
                     omhc.rms_eps(np.float32))
    ref = fx[f"out/{kind}"].reshape(h.shape)
    assert_close(h, ref, what=f"oracle.mhc.mapping {kind}")
    orc = Oracle({f"m.{k}": v for k, v in s.items()}, n_embd=64, n_head=4, n_layer=0)
    with torch.no_grad():
        h32 = orc.mapping(torch.from_numpy(xf.copy()), "m", kind)
    assert_close(h32.numpy().reshape(h.shape), ref, what=f"Oracle.mapping {kind}")


def test_stream_oracles_match_reference():
    """mHCResidualStream.forward (mhc.py:345-381) with a fixed layer
    tanh(x W^T): oracle.mhc.stream_forward (float64) and Oracle.stream."""
    fx = load("mapping_c64.npz")
    s = section(fx, "sd_stream")
    x = fx["in/x"]
    wl = fx["in/w_layer"].astype(np.float64)
    maps = {k: (s[f"H_{k}.phi.weight"].numpy(), float(s[f"H_{k}.alpha"]), s[f"H_{k}.bias"].numpy())
            for k in ("pre", "post", "res")}
    xn, *_ = omhc.stream_forward(x.reshape(-1, 4, 64), maps, lambda v: np.tanh(v @ wl.T), omhc.rms_eps(np.float32))
    ref = fx["out/stream"]
    assert_close(xn.reshape(ref.shape), ref, what="oracle.mhc.stream_forward")
    orc = Oracle({f"s.{k}": v for k, v in s.items()}, n_embd=64, n_head=4, n_layer=0)
    wl32 = torch.from_numpy(fx["in/w_layer"])
    with torch.no_grad():
        y = orc.stream(torch.from_numpy(x), "s", lambda v: torch.tanh(v @ wl32.t()))
    assert_close(y.numpy(), ref, what="Oracle.stream")


def test_moe_oracles_match_reference():
    """HadamardMoE.forward (moe.py:512-542) with 8 experts and k = 6:
    oracle.moe.moe_forward (float64) and Oracle.moe (float32) give the
    reference's output, probabilities, routing weights, expert mask and
    balance loss."""
    fx = load("moe_c256.npz")
    sd = section(fx, "sd")
    x = fx["in/x"]
    r = omoe.moe_forward(x.reshape(-1, 256), sd["router.gate.0.weight"].numpy(), sd["router.gate.2.weight"].numpy(),
                         sd["experts.gate_weights"].numpy(), sd["experts.up_weights"].numpy(),
                         sd["experts.down_weights"].numpy(), 6)
    assert_close(r["out"], fx["out/y"].reshape(-1, 256), what="moe_forward out")
    assert_close(r["probs"], fx["out/probs"].reshape(-1, 8), what="probs")
    assert_close(r["weights"], fx["out/weights"].reshape(-1, 8), what="weights")
    assert np.array_equal(r["mask"], fx["out/mask"].reshape(-1, 8))
    assert np.array_equal(fx["out/last_mask"], fx["out/mask"])
    assert abs(r["aux"] - float(fx["out/aux"])) <= TOL * abs(float(fx["out/aux"]))
    orc = Oracle({f"f.{k}": v for k, v in sd.items()}, n_embd=256, n_head=8, n_layer=0, use_moe=True,
                 moe_max_experts=6)
    with torch.no_grad():
        y, info = orc.moe(torch.from_numpy(x), "f")
    assert_close(y.numpy(), fx["out/y"], what="Oracle.moe")
    assert np.array_equal(info["mask"].numpy(), fx["out/mask"])


# --------------------------------------------------------------- cross-checks
def test_model_attention_equals_function_oracles():
    """Oracle.attention (float32, torch ops) equals the composition of the
    pinned float64 function oracles: hadamard_linear_f64 for q, k, v and
    wo, rope_f64, causal_attention_f64 and head_mixer_f64
    (chassis.py:424-483)."""
    fx = load("model_c64.npz")
    orc, cfg = model_oracle(fx)
    C, nh = cfg["n_embd"], cfg["n_head"]
    hd = C // nh
    gen = torch.Generator().manual_seed(3)
    B, T = 2, 12
    x = torch.randn(B, T, C, generator=gen)
    p = "layers.1.attention"
    with torch.no_grad():
        y = orc.attention(x, p, orc.sd["freqs_cis"][:T])

    def lin(v, name):
        w = orc.sd[f"{p}.{name}.inner.weight"].numpy()
        c = otern.ternary_codes(w, otern.absmean_gamma(w))
        return ohad.hadamard_linear_f64(v.reshape(-1, C), c, orc.sd[f"{p}.{name}.inner.alpha"].numpy(),
                                        orc.sd[f"{p}.{name}.inner.beta"].numpy()).reshape(B, T, C)
    xs = x.numpy().astype(np.float64)
    freqs = fx["sd/freqs_cis"]
    q = ohad.rope_f64(lin(xs, "wq"), freqs, hd)
    k = ohad.rope_f64(lin(xs, "wk"), freqs, hd)
    v = lin(xs, "wv")
    heads = lambda a: a.reshape(B, T, nh, hd).transpose(0, 2, 1, 3)  # noqa: E731
    o = oatt.causal_attention_f64(heads(q), heads(k), heads(v))
    o = ohad.head_mixer_f64(o, orc.sd[f"{p}.head_mixer.W"].numpy(), orc.sd[f"{p}.head_mixer.beta"].numpy())
    ref = lin(o.transpose(0, 2, 1, 3).reshape(B, T, C), "wo")
    assert_close(y.numpy(), ref, what="attention")


def test_model_swiglu_and_mapping_equal_function_oracles():
    """Oracle.swiglu equals hadamard_linear_f64 gate/up/down with silu; the
    model oracle's stream step equals oracle.mhc.stream_forward with the
    same layer function (chassis.py:498-507, mhc.py:345-381)."""
    fx = load("model_c64.npz")
    orc, cfg = model_oracle(fx)
    C = cfg["n_embd"]
    gen = torch.Generator().manual_seed(4)
    x = torch.randn(2, 6, C, generator=gen)
    p = "layers.0.feed_forward"
    with torch.no_grad():
        y = orc.swiglu(x, p)

    def lin(v, name):
        w = orc.sd[f"{p}.{name}.inner.weight"].numpy()
        c = otern.ternary_codes(w, otern.absmean_gamma(w))
        return ohad.hadamard_linear_f64(v, c, orc.sd[f"{p}.{name}.inner.alpha"].numpy(),
                                        orc.sd[f"{p}.{name}.inner.beta"].numpy())
    xs = x.numpy().reshape(-1, C).astype(np.float64)
    g, u = lin(xs, "gate_proj"), lin(xs, "up_proj")
    ref = lin(omoe.silu(g) * u, "down_proj")
    assert_close(y.numpy().reshape(ref.shape), ref, what="swiglu")

    xst = torch.randn(2, 6, 4, C, generator=gen)
    s = "layers.0.ffn_stream"
    with torch.no_grad():
        got = orc.stream(xst, s, lambda v: torch.tanh(v))
    maps = {k: (orc.sd[f"{s}.H_{k}.phi.weight"].numpy(), float(orc.sd[f"{s}.H_{k}.alpha"]),
                orc.sd[f"{s}.H_{k}.bias"].numpy()) for k in ("pre", "post", "res")}
    xn, *_ = omhc.stream_forward(xst.numpy().reshape(-1, 4, C), maps, np.tanh, omhc.rms_eps(np.float32))
    assert_close(got.numpy().reshape(xn.shape), xn, what="stream")


def test_model_moe_equals_function_oracle():
    """Oracle.moe (float32) equals oracle.moe.moe_forward (float64) on the
    MoE model fixture's first FFN, including the expert mask (moe.py:512-542)."""
    fx = load("model_c96_moe.npz")
    orc, cfg = model_oracle(fx)
    C = cfg["n_embd"]
    gen = torch.Generator().manual_seed(5)
    x = torch.randn(3, 7, C, generator=gen)
    p = "layers.0.feed_forward"
    with torch.no_grad():
        y, info = orc.moe(x, p)
    sd = orc.sd
    r = omoe.moe_forward(x.numpy().reshape(-1, C), sd[p + ".router.gate.0.weight"].numpy(),
                         sd[p + ".router.gate.2.weight"].numpy(), sd[p + ".experts.gate_weights"].numpy(),
                         sd[p + ".experts.up_weights"].numpy(), sd[p + ".experts.down_weights"].numpy(),
                         cfg["max_experts"])
    assert_close(y.numpy().reshape(-1, C), r["out"], what="moe")
    assert np.array_equal(info["mask"].numpy().reshape(-1, C // 32), r["mask"])


def test_rope_and_rmsnorm_harness():
    """Oracle.rope equals rope_f64 and Oracle.rmsnorm equals x/sqrt(mean x^2 + 1e-6)*w
    (chassis.py:96-106, 332-345) on the model fixture's frequency table."""
    fx = load("model_c64.npz")
    orc, cfg = model_oracle(fx)
    gen = torch.Generator().manual_seed(6)
    B, T, nh, hd = 2, 10, 4, 16
    q = torch.randn(B, T, nh, hd, generator=gen)
    k = torch.randn(B, T, nh, hd, generator=gen)
    freqs = torch.polar(torch.ones(T, hd // 2), torch.randn(T, hd // 2, generator=gen))
    qr, kr = orc.rope(q, k, freqs)
    assert_close(qr.numpy().reshape(B, T, -1), ohad.rope_f64(q.numpy().reshape(B, T, -1), freqs.numpy(), hd))
    assert_close(kr.numpy().reshape(B, T, -1), ohad.rope_f64(k.numpy().reshape(B, T, -1), freqs.numpy(), hd))
    x = torch.randn(5, 64, generator=gen)
    w = torch.randn(64, generator=gen)
    xd = x.double()
    ref = xd / torch.sqrt((xd * xd).mean(-1, keepdim=True) + 1e-6) * w.double()
    assert_close(orc.rmsnorm(x, w).numpy(), ref.numpy())
    assert math.isclose(float(F.rms_norm(torch.ones(1, 4), (4,)).sum()), 4.0, rel_tol=1e-6)
