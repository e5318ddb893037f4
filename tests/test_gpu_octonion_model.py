"""The octonion-algebra model on the GPU against the reference's own output.

``tests/golden/model_oct_c64.npz`` holds a 2-layer mHCWalsh with
algebra="octonion" (n_embd 64, 8 heads of 8, octonion head mixing, SwiGLU
FFN) run by the reference on the CPU, where its layers are
OctonionTernaryLinearRef (physics.py:53-82) and the head mixer is the
pure-torch OctonionHeadMixer (chassis.py:347-399).  The same state dict is
loaded into this build's mHCWalsh (chassis.get_linear_layer's octonion
branch, chassis.py:54-65; attention split by 8, :424-434):

* with chassis.OctonionTernaryLinear bound to OctonionTernaryLinearRef (as
  the fixture was made) the float32 logits, hidden states and loss agree
  within 1e-5;
* with the default GPU module, OctonionFusedLinear (the reference's
  cayley_dickson_cuda.py:622-668: bf16 operands, the sum rounded to bf16,
  times beta, float32 out), the result agrees with the model oracle run
  with those roundings (octonion_gpu) and lies within bf16 reach of the
  reference's float32 output;
* under bf16 autocast, within the bf16 bars of the reference's own bf16
  drift (the oracle under CPU autocast).
"""
import os

import numpy as np
import pytest
import torch

from oracle.model import Oracle

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)), \
        float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def _fixture():
    with np.load(os.path.join(GOLDEN, "model_oct_c64.npz"), allow_pickle=False) as z:
        fx = {k: z[k] for k in z.files}
    c = {k[4:]: (str(v) if v.dtype.kind == "U" else int(v)) for k, v in fx.items() if k.startswith("cfg/")}
    assert c["algebra"] == "octonion"
    sd = {k[3:]: torch.from_numpy(v.copy()) for k, v in fx.items() if k.startswith("sd/")}
    return fx, c, sd


def _model(c, sd):
    from src.model import WalshConfig, mHCWalsh
    cfg = WalshConfig(block_size=c["block_size"], vocab_size=c["vocab"], n_layer=c["n_layer"], n_head=c["n_head"],
                      n_embd=c["n_embd"], algebra="octonion", head_mixing=bool(c["head_mixing"]))
    model = mHCWalsh(cfg, n_streams=4)
    model.load_state_dict(sd, strict=True)
    return model.cuda().eval()


def _oracle(c, sd, **kw):
    return Oracle(dict(sd), c["n_embd"], c["n_head"], c["n_layer"], head_mixing=bool(c["head_mixing"]),
                  algebra="octonion", **kw)


def test_octonion_model_ref_module_fp32(monkeypatch):
    from src.model import chassis
    from src.model.octonion import OctonionTernaryLinearRef
    fx, c, sd = _fixture()
    monkeypatch.setattr(chassis, "OctonionTernaryLinear", OctonionTernaryLinearRef)
    model = _model(c, sd)
    assert type(model.layers[0].attention.wq) is OctonionTernaryLinearRef
    idx = torch.from_numpy(fx["in/idx"]).cuda()
    targets = torch.from_numpy(fx["in/targets"]).cuda()
    with torch.no_grad():
        logits, _, h = model(idx, return_hidden=True)
        _, loss = model(idx, targets=targets)
    rl, rh = rel(logits.cpu(), fx["out/logits_last"]), rel(h.cpu(), fx["out/h_out"])
    print(f"octonion model (OctonionTernaryLinearRef) fp32: logits {rl}, hidden {rh}, loss {float(loss):.7f} vs "
          f"{float(fx['out/loss']):.7f}", flush=True)
    assert max(rl) <= 1e-5 and max(rh) <= 1e-5
    assert abs(float(loss) - float(fx["out/loss"])) <= 1e-5 * abs(float(fx["out/loss"]))


def test_octonion_model_fused_module():
    from src.model.octonion import OctonionFusedLinear
    fx, c, sd = _fixture()
    model = _model(c, sd)
    assert type(model.layers[0].attention.wq) is OctonionFusedLinear
    idx = torch.from_numpy(fx["in/idx"]).cuda()
    with torch.no_grad():
        logits, _, h = model(idx, return_hidden=True)
    with torch.no_grad():
        _, h_gpu_sem = _oracle(c, sd, octonion_gpu=True).forward(idx.cpu(), return_hidden=True)
    h32 = fx["out/h_out"]
    d_sem = rel(h.cpu(), h_gpu_sem)[0]
    d_ref = rel(h_gpu_sem, h32)[0]
    d_gpu = rel(h.cpu(), h32)[0]
    print(f"octonion model (OctonionFusedLinear) fp32 activations: vs the oracle with the GPU module's roundings "
          f"{d_sem:.3e}; that oracle vs the reference's float32 {d_ref:.3e}; GPU vs the reference's float32 "
          f"{d_gpu:.3e}", flush=True)
    # the same roundings, float32 sums in another order: rare one-ulp flips
    assert d_sem <= 2e-3
    assert d_gpu <= max(1e-2, 1.25 * d_ref)

    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        _, _, hb = model(idx, return_hidden=True)
    with torch.no_grad(), torch.autocast("cpu", dtype=torch.bfloat16):
        _, hr = _oracle(c, sd).forward(idx.cpu(), return_hidden=True)
    d_ref_b = rel(hr.float(), h32)[0]
    d_gpu_b = rel(hb.float().cpu(), h32)[0]
    d_pair = rel(hb.float().cpu(), hr.float())[0]
    print(f"octonion model bf16 autocast: GPU vs reference fp32 {d_gpu_b:.3e}; reference-style bf16 vs fp32 "
          f"{d_ref_b:.3e}; GPU vs reference-style bf16 {d_pair:.3e}", flush=True)
    assert d_gpu_b <= max(1e-2, 1.25 * d_ref_b) and d_pair <= max(1e-2, 2.0 * d_ref_b)
