"""GPU checks of the module surface: Hadamard layer classes, tuple interface,
standalone FHT and packing helpers against the oracle."""
import numpy as np
import pytest
import torch

from oracle import hadamard as ohad
from oracle import ternary as otern

from test_gpu_hadamard import assert_close

pytestmark = pytest.mark.gpu


def _codes(w):
    w = w.detach().cpu().numpy()
    return otern.ternary_codes(w, otern.absmean_gamma(w))


@pytest.mark.parametrize("cls_name", ["HadamardLinear", "HadamardTernaryLinear"])
def test_hadamard_layer_classes(cls_name):
    import src.model.fht_cuda as fc
    torch.manual_seed(0)
    layer = getattr(fc, cls_name)(512, 1376).cuda()
    with torch.no_grad():
        layer.alpha.uniform_(0.5, 1.5)
        layer.beta.uniform_(0.1, 0.3)
    x = torch.randn(3, 7, 512, device="cuda")
    y = layer(x)
    assert y.shape == (3, 7, 1376) and y.dtype == torch.float32
    ref = ohad.hadamard_linear_f64(x.reshape(-1, 512).cpu().numpy(), _codes(layer.weight),
                                   layer.alpha.detach().cpu().numpy(), layer.beta.detach().cpu().numpy())
    assert_close(y.detach().reshape(-1, 1376).cpu().numpy(), ref, torch.float32, cls_name)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        yb = layer(x)
    assert yb.dtype == torch.float32          # cast back to the input dtype, as the reference does
    assert_close(yb.detach().reshape(-1, 1376).cpu().numpy(), ref, torch.bfloat16, cls_name + " autocast")


def test_tuple_interface_in_place_and_copy():
    from src.model.fht_cuda import HadamardTernaryLinearTuple
    torch.manual_seed(1)
    layer = HadamardTernaryLinearTuple(512, 512).cuda()
    x = torch.randn(2, 5, 512, device="cuda")
    parts = x.split(16, dim=-1)
    ys = layer(parts)
    assert len(ys) == 32 and ys[0].shape == (2, 5, 16)
    ys2 = layer(tuple(p.clone() for p in parts))       # non-adjacent parts -> cat path
    assert all(torch.equal(a, b) for a, b in zip(ys, ys2))
    full = layer.forward_full(x)
    assert torch.equal(torch.cat(ys, -1), full)
    assert layer.weight is layer.inner.weight and layer.beta is layer.inner.beta
    with pytest.raises(AssertionError):
        layer(parts[:31])


def test_fht_and_packing_helpers():
    from src.model.fht_cuda import fht, hadamard_matrix, pack_ternary_weights, unpack_ternary_weights
    assert torch.allclose(hadamard_matrix(32), torch.from_numpy(ohad.sylvester(32)).float())
    for N in (2, 32, 64, 1024, 8192):
        x = torch.randn(37, N, device="cuda")
        ref = ohad.fht(x.double().cpu().numpy())
        assert np.max(np.abs(fht(x).double().cpu().numpy() - ref)) < 1e-5 * max(1.0, np.abs(ref).max())
    # Rust KAT: fht twice on x[i] = i returns x
    xi = torch.arange(32, dtype=torch.float32, device="cuda")
    assert torch.max(torch.abs(fht(fht(xi)) - xi)) < 1e-5
    rng = np.random.default_rng(2)
    c = rng.integers(-1, 2, size=(32, 16, 16)).astype(np.int8)
    p = pack_ternary_weights(torch.from_numpy(c).float().cuda())
    assert np.array_equal(p.cpu().numpy(), otern.pack_codes(c))
    assert np.array_equal(unpack_ternary_weights(p, 16).cpu().numpy(), c.astype(np.float32))


def test_quantize_ternary_value_and_ste():
    from src.model.physics import quantize_ternary
    w = (torch.randn(32, 43, 16) * 0.02).cuda().requires_grad_(True)
    q = quantize_ternary(w)
    c = _codes(w)
    assert np.array_equal(q.detach().cpu().numpy(), c.astype(np.float32))
    q.sum().backward()                       # STE: gradient passes to the latent weight
    assert w.grad is not None and torch.all(w.grad.abs() <= 2)


def test_cpu_tensors_are_rejected():
    from src.model.fht_cuda import HadamardLinear
    layer = HadamardLinear(64, 64)
    with pytest.raises(RuntimeError, match="GPU"):
        layer(torch.randn(1, 2, 64))
