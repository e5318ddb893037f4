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
