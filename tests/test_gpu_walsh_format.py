"""The .walsh v4 format on the GPU: bitmask + sign decode against the
oracle (bit-exact), the file round trip, and HadamardPackedLinear."""
import numpy as np
import pytest
import torch

from oracle import ternary as otern
from oracle import walsh_format as owf

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape", [(32, 16, 16), (32, 43, 16), (32, 16, 43), (1, 5), (7, 3), (1000, 1037)])
def test_ternary_from_bitmask_vs_oracle(shape):
    from src.model import kernels
    rng = np.random.default_rng(sum(shape))
    codes = rng.choice(np.array([-1, 0, 1], np.int8), size=shape, p=[0.3, 0.4, 0.3])
    bm, sg, nnz = owf.encode_codes(codes)
    out = kernels.ternary_from_bitmask(torch.from_numpy(bm).cuda(), torch.from_numpy(sg).cuda(), nnz, shape,
                                       packed=True, codes=True)
    torch.cuda.synchronize()
    assert np.array_equal(out["codes"].cpu().numpy(), codes)
    assert np.array_equal(out["packed"].cpu().numpy(), otern.pack_codes(codes))
    # a num_nonzero cut leaves the later non-zeros at 0, as the reference loader does
    cut = nnz // 2
    out2 = kernels.ternary_from_bitmask(torch.from_numpy(bm).cuda(), torch.from_numpy(sg).cuda(), cut, shape,
                                        packed=False, codes=True)
    assert np.array_equal(out2["codes"].cpu().numpy(), owf.decode_codes(bm, sg, shape, cut))


def _walsh(seed=0):
    from src.model import Walsh, WalshConfig
    torch.manual_seed(seed)
    cfg = WalshConfig(block_size=64, vocab_size=300, n_layer=2, n_head=32, n_embd=128, algebra='hadamard',
                      head_mixing=True)
    return cfg, Walsh(cfg).cuda().eval()


def test_walsh_file_round_trip(tmp_path):
    """save_walsh -> load_walsh: ternary codes bit-exact, float16 / int8
    entries as stored; a model loaded from the file computes exactly what the
    original computes with the same stored (rounded) parameters."""
    from src.model import kernels
    from src.walsh_format import load_walsh, save_walsh
    cfg, model = _walsh()
    path = str(tmp_path / "m.walsh")
    sd = model.state_dict()
    save_walsh(path, sd, {"n_layer": 2, "n_embd": 128})
    loaded, conf = load_walsh(path)
    assert conf == {"n_layer": 2, "n_embd": 128}
    n_tern = 0
    for name, t in sd.items():
        if name.endswith('.weight') and any(k in name for k in ('wq', 'wk', 'wv', 'wo', '_proj')):
            ref = kernels.ternary_quantize(t.float(), codes=True, packed=False)["codes"].float()
            assert torch.equal(loaded[name], ref), name
            n_tern += 1
    assert n_tern == 2 * 7
    # the model on the stored values: codes as latents (their absmean codes are themselves), other
    # parameters as stored
    ref_model = _walsh()[1]
    with torch.no_grad():
        for name, p in list(ref_model.named_parameters()) + list(ref_model.named_buffers()):
            if name in loaded:
                p.copy_(loaded[name].to(p.dtype))
    other = _walsh(seed=1)[1]
    missing, unexpected = other.load_state_dict(loaded, strict=False)
    # output.weight is tied to the embedding (stored once, as compress.py does); H are constant buffers
    assert other.output.weight is other.tok_embeddings.weight
    assert not unexpected and all(m.endswith('.H') or m == 'output.weight' for m in missing), (missing, unexpected)
    idx = torch.randint(0, 300, (2, 16), generator=torch.Generator().manual_seed(0)).cuda()
    with torch.no_grad():
        a, _ = ref_model(idx)
        b, _ = other(idx)
    assert torch.equal(a, b)
    # packed ternary straight into HadamardPackedLinear buffers
    packed, _ = load_walsh(path, packed_ternary=True)
    name = 'layers.0.attention.wq.inner.weight'
    pk = kernels.ternary_quantize(sd[name].float(), packed=True)["packed"]
    assert torch.equal(packed[name], pk)


def test_hadamard_packed_linear_and_optimize_for_inference():
    from src.model.fht_cuda import HadamardLinear, HadamardPackedLinear, optimize_for_inference
    torch.manual_seed(2)
    lin = HadamardLinear(512, 1376).cuda()
    with torch.no_grad():
        lin.alpha.uniform_(0.5, 1.5)
        lin.beta.uniform_(0.1, 0.3)
    pk = HadamardPackedLinear.from_trained(lin)
    assert pk.beta.shape == (32, 43) and pk.alpha.shape == (32, 16)
    x = torch.randn(3, 7, 512, device="cuda")
    with torch.no_grad():
        assert torch.equal(pk(x), lin(x))
        cfg, model = _walsh(seed=3)
        idx = torch.randint(0, 300, (2, 16), generator=torch.Generator().manual_seed(1)).cuda()
        ref, _ = model(idx)
        optimize_for_inference(model)
        assert not any(isinstance(m, HadamardLinear) for m in model.modules())
        got, _ = model(idx)
    assert torch.equal(got, ref)


@pytest.mark.parametrize("algebra", ["hadamard", "octonion"])
def test_load_reference_written_walsh_file(algebra):
    """load_walsh on a file the reference's compress_model wrote
    (tests/golden/tiny_<algebra>.walsh, compress.py:121-358): the ternary
    weights decode on the GPU to the absmean codes of the latents the file
    was written from (float codes and 2-bit packed buffers), float16 entries
    are the latents rounded to float16, the embedding is its int8 codes times
    the stored scale, RoPE as stored."""
    import os
    from src.walsh_format import load_walsh
    golden = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    path = os.path.join(golden, f"tiny_{algebra}.walsh")
    with np.load(os.path.join(golden, "walsh_files.npz"), allow_pickle=False) as z:
        ref = {k.split("/", 1)[1]: z[k] for k in z.files if k.startswith(algebra + "/")}
    sd, config = load_walsh(path, device="cuda")
    sdp, _ = load_walsh(path, device="cuda", packed_ternary=True)
    torch.cuda.synchronize()
    assert config["algebra"] == algebra
    n_ternary = 0
    for name, t in sd.items():
        w = ref[name]
        if name.endswith(".weight") and any(k in name for k in ("wq", "wk", "wv", "wo", "_proj")):
            codes = otern.ternary_codes(w, otern.absmean_gamma(w))
            assert np.array_equal(t.cpu().numpy(), codes.astype(np.float32)), name
            assert np.array_equal(sdp[name].cpu().numpy(), otern.pack_codes(codes)), name
            n_ternary += 1
        elif name == "tok_embeddings.weight":
            scale = np.float32(np.abs(w).max() / 127.0)
            q = np.clip(np.round(w / scale), -127, 127).astype(np.float32)
            assert np.array_equal(t.cpu().numpy(), q * scale)
        elif name == "freqs_cis":
            assert torch.equal(t.cpu(), torch.from_numpy(w))
        else:
            assert np.array_equal(t.cpu().numpy(), w.astype(np.float16).astype(np.float32)), name
    assert n_ternary == 7 and "output.weight" not in sd
