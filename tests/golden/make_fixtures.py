"""Write the golden fixtures of tests/golden from the reference's own modules.

Run in the build container only, on the CPU:

    python tests/golden/make_fixtures.py [/path/to/Walsh-Research]

It imports the reference's ``src.model`` package (pulseofthemachine/
Walsh-Research) from the given checkout (default ``/root/reference``), builds
small modules under fixed seeds, perturbs their parameters away from the
symmetric initial values (so that a composition mistake such as a swapped
stream, a dropped bias or a transposed mapping changes the output), runs their
CPU forward in float32 and stores inputs, parameters and outputs as ``.npz``
archives (plain arrays, no pickles).  The fixtures are data: nothing of the
reference's source travels with them, and the GPU tests never need the
reference checkout.

Fixtures (each well under 1 MB):

* ``model_c64.npz``        mHCWalsh, hadamard algebra, head mixing, 2 layers,
                           n_embd 64, n_head 32, SwiGLU FFN (src/model/mhc.py:549-681)
* ``model_c96_moe.npz``    mHCWalsh, 2 layers, n_embd 96, n_head 3, MoE
                           (3 experts, k 2) and channel modulation
* ``moe_c256.npz``         HadamardMoE, x [2, 8, 256] (8 experts), max_experts 6 (moe.py:450-560)
* ``mapping_c64.npz``      ResidualStreamMapping res/pre/post and one
                           mHCResidualStream with a fixed layer (mhc.py:232-381)
* ``sinkhorn.npz``         SinkhornKnopp on [64, 4, 4] (mhc.py:198-229)
* ``hadamard_linear.npz``  HadamardLinear 512 -> 512 on x [2, 8, 512] (fht_cuda.py:436-519)
* ``octonion_ref.npz``     OctonionTernaryLinearRef 64 -> 64 on x [2, 8, 64] (physics.py:53-82)
* ``tiny_hadamard.walsh``  compress.py's compress_model (the reference's .walsh v4
  ``tiny_octonion.walsh``  writer, compress.py:121-358) run on tiny Walsh
  ``walsh_files.npz``      checkpoints (chassis.py:533-668; n_embd 64, one
                           layer, Hadamard with head mixing / octonion), and the
                           checkpoints' tensors the files were written from
* ``model_oct_c64.npz``    mHCWalsh, octonion algebra, head mixing, 2 layers,
                           n_embd 64, n_head 8, SwiGLU FFN, with the CPU
                           module the reference selects when its GPU kernels
                           are absent (chassis.OctonionTernaryLinear =
                           physics.OctonionTernaryLinearRef, physics.py:84-91)
                           and the pure-torch OctonionHeadMixer
                           (chassis.py:347-399, chosen without CUDA at :14-19)
"""
import math
import os
import sys
import tempfile

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _import_reference(root):
    if root not in sys.path:
        sys.path.insert(0, root)
    import src.model as m  # noqa: F401  (the reference package)
    from src.model import chassis, fht_cuda, mhc, moe, physics
    return chassis, fht_cuda, mhc, moe, physics


def _np(t):
    t = t.detach().cpu()
    if t.is_complex():
        return t.numpy().astype(np.complex64)
    if t.dtype == torch.bool:
        return t.numpy()
    if t.is_floating_point():
        return t.float().numpy()
    return t.numpy()


def _state(module):
    return {f"sd/{k}": _np(v) for k, v in module.state_dict().items()}


@torch.no_grad()
def _perturb(module, gen):
    """Move every parameter away from its symmetric initial value.

    Ternary latents stay as initialised (their codes are what the layer
    uses); scales, biases, norms and the stream projections get relative
    noise; the mapping gains (alpha, 0.01 at init) are raised so that the
    dynamic part of each mapping is not negligible."""
    for name, p in module.named_parameters():
        leaf = name.rsplit(".", 1)[-1]
        if leaf in ("weight",) and any(s in name for s in (".wq.", ".wk.", ".wv.", ".wo.", "_proj.inner",
                                                           ".gate_proj.", ".up_proj.", ".down_proj.")):
            continue  # ternary latents
        if name.endswith("_weights"):
            continue  # MoE ternary latents
        if leaf == "alpha" and p.numel() == 1:  # mapping gain
            p.copy_(torch.empty(()).uniform_(0.3, 0.7, generator=gen))
            continue
        scale = float(p.detach().float().pow(2).mean().sqrt()) if p.numel() else 1.0
        if scale == 0.0:  # zero-initialised: mapping biases [1, n] get O(1) values, others small ones
            p.add_(torch.randn(p.shape, generator=gen) * (0.5 if p.dim() == 2 else 0.02))
            continue
        p.add_(torch.randn(p.shape, generator=gen) * 0.2 * scale)


def model_fixture(chassis, mhc, path, *, n_embd, n_head, n_layer, use_moe=False, max_experts=4,
                  use_channel_mod=False, head_mixing=True, vocab=128, block_size=32, B=2, T=16, seed=0,
                  algebra="hadamard"):
    torch.manual_seed(seed)
    cfg = chassis.WalshConfig(block_size=block_size, vocab_size=vocab, n_layer=n_layer, n_head=n_head,
                              n_embd=n_embd, algebra=algebra, head_mixing=head_mixing, use_moe=use_moe,
                              moe_max_experts=max_experts, use_channel_mod=use_channel_mod)
    model = mhc.mHCWalsh(cfg, n_streams=4)
    gen = torch.Generator().manual_seed(seed + 1)
    _perturb(model, gen)
    model.eval()
    idx = torch.randint(0, vocab, (B, T), generator=gen)
    targets = torch.randint(0, vocab, (B, T), generator=gen)
    with torch.no_grad():
        logits_last, _, h_out = model(idx, return_hidden=True)
        logits_all, loss = model(idx, targets=targets)
    out = _state(model)
    out.update({
        "cfg/n_embd": np.int64(n_embd), "cfg/n_head": np.int64(n_head), "cfg/n_layer": np.int64(n_layer),
        "cfg/use_moe": np.int64(use_moe), "cfg/max_experts": np.int64(max_experts),
        "cfg/use_channel_mod": np.int64(use_channel_mod), "cfg/head_mixing": np.int64(head_mixing),
        "cfg/vocab": np.int64(vocab), "cfg/block_size": np.int64(block_size),
        "cfg/algebra": np.array(algebra),
        "in/idx": idx.numpy(), "in/targets": targets.numpy(),
        "out/logits_last": _np(logits_last), "out/h_out": _np(h_out),
        "out/logits_all": _np(logits_all), "out/loss": _np(loss),
    })
    if use_moe:
        for l, layer in enumerate(model.layers):
            out[f"out/moe_mask_{l}"] = _np(layer.feed_forward._last_expert_mask)
            out[f"out/moe_aux_{l}"] = _np(layer.feed_forward._aux_loss)
    np.savez_compressed(path, **out)


def octonion_model_fixture(chassis, mhc, physics, path):
    """The octonion-algebra model on the reference's CPU path.  Without a GPU
    the reference would still bind chassis.OctonionTernaryLinear to the
    Triton module when triton imports (physics.py:84-88), and that module
    cannot run on a CPU; the CPU module is what physics.py:89-91 falls back
    to, so it is bound here for the duration of the construction."""
    assert not torch.cuda.is_available()
    bound = chassis.OctonionTernaryLinear
    chassis.OctonionTernaryLinear = physics.OctonionTernaryLinearRef
    try:
        model_fixture(chassis, mhc, path, n_embd=64, n_head=8, n_layer=2, algebra="octonion", seed=9)
    finally:
        chassis.OctonionTernaryLinear = bound


def walsh_file_fixtures(chassis, root, seed=0):
    """Tiny Walsh checkpoints of plain tensors, compressed to .walsh v4 by the
    reference's own writer.  The .npz keeps every tensor of each checkpoint
    (prefix ``hadamard/`` or ``octonion/``) so a reader's output can be
    checked against what was written: ternary latents (the writer quantises
    them itself), float16 and int8 entries (the writer rounds them)."""
    if root not in sys.path:
        sys.path.insert(0, root)
    import compress  # the reference's compress.py
    out = {}
    for algebra, mixing in (("hadamard", True), ("octonion", False)):
        torch.manual_seed(seed)
        args = dict(block_size=16, vocab_size=64, n_layer=1, n_head=32 if algebra == "hadamard" else 8, n_embd=64,
                    algebra=algebra, head_mixing=mixing)
        model = chassis.Walsh(chassis.WalshConfig(**args))
        _perturb(model, torch.Generator().manual_seed(seed + 1))
        with tempfile.TemporaryDirectory() as d:
            ckpt = os.path.join(d, "ckpt.pt")
            torch.save({"model_args": args, "model": model.state_dict()}, ckpt)
            compress.compress_model(ckpt, os.path.join(HERE, f"tiny_{algebra}.walsh"))
        out.update({f"{algebra}/{k}": _np(v) for k, v in model.state_dict().items()})
    np.savez_compressed(os.path.join(HERE, "walsh_files.npz"), **out)


def moe_fixture(chassis, moe, path, seed=0):
    torch.manual_seed(seed)
    cfg = chassis.WalshConfig(n_embd=256, n_head=8, algebra="hadamard", use_moe=True)
    layer = moe.HadamardMoE(cfg, threshold=0.1, min_experts=1, max_experts=6)
    gen = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for m in layer.router.gate:
            if isinstance(m, torch.nn.Linear):
                m.weight.normal_(0.0, 0.02, generator=gen)
    layer.eval()
    x = torch.randn(2, 8, 256, generator=gen)
    with torch.no_grad():
        y = layer(x)
        w, mask, probs = layer.router(x)
    out = _state(layer)
    out.update({"in/x": _np(x), "out/y": _np(y), "out/mask": _np(mask), "out/probs": _np(probs),
                "out/weights": _np(w), "out/aux": _np(layer._aux_loss), "out/last_mask": _np(layer._last_expert_mask)})
    np.savez_compressed(path, **out)


def mapping_fixture(mhc, path, seed=0, n_embd=64, n=4):
    torch.manual_seed(seed)
    gen = torch.Generator().manual_seed(seed + 1)
    out = {}
    x = torch.randn(2, 8, n, n_embd, generator=gen)
    xf = x.reshape(2, 8, n * n_embd)
    for kind in ("res", "pre", "post"):
        m = mhc.ResidualStreamMapping(n_embd, n, kind)
        _perturb(m, gen)
        with torch.no_grad():
            h = m(xf)
        out.update({f"sd_{kind}/{k}": _np(v) for k, v in m.state_dict().items()})
        out[f"out/{kind}"] = _np(h)
    stream = mhc.mHCResidualStream(n_embd, n)
    _perturb(stream, gen)
    w_layer = torch.randn(n_embd, n_embd, generator=gen) / math.sqrt(n_embd)
    with torch.no_grad():
        y = stream(x, lambda v: torch.tanh(v @ w_layer.t()))
    out.update({f"sd_stream/{k}": _np(v) for k, v in stream.state_dict().items()})
    out.update({"in/x": _np(x), "in/w_layer": _np(w_layer), "out/stream": _np(y)})
    np.savez_compressed(path, **out)


def sinkhorn_fixture(mhc, path, seed=0):
    gen = torch.Generator().manual_seed(seed)
    h = torch.randn(64, 4, 4, generator=gen) * 1.5
    h[0] = 0.0
    h[1] = 2.0 * torch.eye(4)
    sk = mhc.SinkhornKnopp(n_iter=20, eps=1e-8)
    with torch.no_grad():
        y = sk(h)
    np.savez_compressed(path, **{"in/h": _np(h), "out/y": _np(y)})


def hadamard_fixture(fht_cuda, path, seed=0):
    torch.manual_seed(seed)
    gen = torch.Generator().manual_seed(seed + 1)
    layer = fht_cuda.HadamardLinear(512, 512)
    with torch.no_grad():
        layer.alpha.add_(torch.randn(layer.alpha.shape, generator=gen) * 0.2)
        layer.beta.mul_(1 + torch.randn(layer.beta.shape, generator=gen) * 0.2)
    x = torch.randn(2, 8, 512, generator=gen)
    with torch.no_grad():
        y = layer(x)
    out = _state(layer)
    out.update({"in/x": _np(x), "out/y": _np(y)})
    np.savez_compressed(path, **out)


def octonion_fixture(physics, path, seed=0):
    torch.manual_seed(seed)
    gen = torch.Generator().manual_seed(seed + 1)
    layer = physics.OctonionTernaryLinearRef(64, 64)
    with torch.no_grad():
        layer.beta.mul_(1 + torch.randn(layer.beta.shape, generator=gen) * 0.2)
    x = torch.randn(2, 8, 64, generator=gen)
    parts = x.split(8, dim=-1)
    with torch.no_grad():
        y = torch.cat(layer(parts), dim=-1)
    out = _state(layer)
    out.update({"in/x": _np(x), "out/y": _np(y)})
    np.savez_compressed(path, **out)


def main():
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    torch.set_num_threads(1)
    chassis, fht_cuda, mhc, moe, physics = _import_reference(root)
    model_fixture(chassis, mhc, os.path.join(HERE, "model_c64.npz"), n_embd=64, n_head=32, n_layer=2)
    model_fixture(chassis, mhc, os.path.join(HERE, "model_c96_moe.npz"), n_embd=96, n_head=3, n_layer=2,
                  use_moe=True, max_experts=2, use_channel_mod=True, head_mixing=False, seed=5)
    moe_fixture(chassis, moe, os.path.join(HERE, "moe_c256.npz"))
    mapping_fixture(mhc, os.path.join(HERE, "mapping_c64.npz"))
    sinkhorn_fixture(mhc, os.path.join(HERE, "sinkhorn.npz"))
    hadamard_fixture(fht_cuda, os.path.join(HERE, "hadamard_linear.npz"))
    octonion_fixture(physics, os.path.join(HERE, "octonion_ref.npz"))
    octonion_model_fixture(chassis, mhc, physics, os.path.join(HERE, "model_oct_c64.npz"))
    walsh_file_fixtures(chassis, root)
    for f in sorted(os.listdir(HERE)):
        if f.endswith((".npz", ".walsh")):
            print(f"{f}: {os.path.getsize(os.path.join(HERE, f))} bytes")


if __name__ == "__main__":
    main()
