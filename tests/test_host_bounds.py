"""Host-side bounds checks of the training-path kernels that address memory
through raw pointers (the stream-mixing backward: mhc_agg_bwd_kernel and
mhc_post_bwd_kernel walk dense [M][n][C], [M][C], [M][n][n] and [M][n]
rows).  An operand holding fewer elements than the kernel would address is
rejected on the host, before any launch.  (The Hadamard backward reads and
writes its rows through bounds-checked buffer resources and checks its
workspace size in walsh_hadamard_linear_ex_bwd.)"""
import pytest
import torch

from src.model import kernels as K


def _post_operands(M=8, n=4, C=64):
    return dict(x=torch.zeros(M, n, C), out=torch.zeros(M, C), h_res=torch.zeros(M, n, n),
                h_post=torch.zeros(M, n), d_new=torch.zeros(M, n, C))


@pytest.mark.parametrize("short", ["out", "h_res", "h_post", "d_new"])
def test_post_bwd_rejects_short_operands(short):
    ops = _post_operands()
    ops[short] = ops[short].reshape(-1)[:-1]
    with pytest.raises(ValueError, match="mhc_post_bwd: operand"):
        K.mhc_post_bwd(ops["x"], ops["out"], ops["h_res"], ops["h_post"], ops["d_new"])


@pytest.mark.parametrize("short", ["h_pre", "d_li"])
def test_aggregate_bwd_rejects_short_operands(short):
    M, n, C = 8, 4, 64
    ops = dict(x=torch.zeros(M, n, C), h_pre=torch.zeros(M, n), d_li=torch.zeros(M, C))
    ops[short] = ops[short].reshape(-1)[:-1]
    with pytest.raises(ValueError, match="mhc_aggregate_bwd: operand"):
        K.mhc_aggregate_bwd(ops["x"], ops["h_pre"], ops["d_li"])


def test_moe_decode_rejects_fewer_partial_rows_than_tokens():
    """walsh_moe_decode_fwd writes partial row t of the per-expert counts and
    probability sums for token t; a caller passing n_part < M would lose
    tokens, so the entry point rejects it (WALSH_EINVAL) before any launch.
    The pointers are never dereferenced: the check comes first."""
    from src.model import _hip
    L = _hip.lib()
    p = 4096  # aligned, non-null, never read
    M, C, H, E, k, He = 3, 4096, 1024, 128, 6, 128
    rc = L.walsh_moe_decode_fwd(p, C, M, C, H, p, p, E, k, He, p, p, p, p, p, 1 << 20, p, p, p, p, p, p, p, p,
                                M - 1, p, C, 1, None)
    assert rc == -1
    assert "n_part" in L.walsh_last_error().decode()


def test_half_range_check_of_wide_kernel_scales():
    """The n_embd-4096 bf16 Hadamard kernels hold alpha and beta as float16;
    values float16 cannot hold (overflow, non-finite, non-zeros that would
    flush to zero) are rejected on the host (once per parameter version)
    instead of being rounded away silently."""
    assert K.half_scales_used(torch.bfloat16, 128, 128)
    assert not K.half_scales_used(torch.float32, 128, 128)
    assert not K.half_scales_used(torch.bfloat16, 16, 16) and not K.half_scales_used(torch.bfloat16, 43, 16)
    ok = torch.tensor([0.0, 1.0, -3e-3, 6e4, 2.4e-5, 1e-7])
    K.check_half_range("alpha", ok)
    for bad in (torch.tensor([1.0, 7e4]), torch.tensor([1.0, -1e-8]), torch.tensor([float("inf")]),
                torch.tensor([float("nan"), 1.0])):
        with pytest.raises(ValueError, match="float16"):
            K.check_half_range("beta", bad)
    # an in-place update (new version) is checked again
    p = torch.nn.Parameter(torch.ones(4))
    K.check_half_range("beta", p)
    with torch.no_grad():
        p.mul_(1e5)
    with pytest.raises(ValueError):
        K.check_half_range("beta", p)
