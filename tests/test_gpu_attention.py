"""GPU parity of the split-K decode attention (walsh_decode_attention)
against oracle.attention.decode_attention_f64 on the same (rounded) inputs.
Bars: ||d|| / ||ref|| and max|d| / max|ref| <= 1e-5 in float32, 1e-2 in
bfloat16."""
import numpy as np
import pytest
import torch

from oracle import attention as oatt

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2}


def assert_close(y, ref, dtype, what=""):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    d = y - ref
    r_norm = np.linalg.norm(d) / np.linalg.norm(ref)
    r_max = np.abs(d).max() / np.abs(ref).max()
    print(f"{what} rel_norm={r_norm:.3e} rel_max={r_max:.3e}", flush=True)
    assert r_norm <= TOL[dtype] and r_max <= TOL[dtype], (what, r_norm, r_max)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,H,L,D,max_len", [(2, 3, 1, 128, 8), (3, 32, 4095, 128, 4096), (1, 32, 4096, 128, 4096),
                                             (2, 4, 777, 64, 1024), (4, 8, 130, 32, 256), (2, 32, 300, 16, 300),
                                             (1, 2, 5000, 128, 5000)])
def test_decode_attention_vs_oracle(B, H, L, D, max_len, dtype):
    from src.model import kernels
    print(f"case B={B} H={H} L={L} D={D} {dtype}", flush=True)
    g = torch.Generator().manual_seed(B * 7 + L)
    q = torch.randn(B, H, 1, D, generator=g).to(dtype)
    kc = torch.randn(B, H, max_len, D, generator=g).to(dtype)   # cache storage, first L rows valid
    vc = torch.randn(B, H, max_len, D, generator=g).to(dtype)
    qd, kd, vd = q.cuda(), kc.cuda(), vc.cuda()
    k, v = kd[:, :, :L], vd[:, :, :L]
    assert kernels.decode_attention_supported(qd, k, v)
    o = kernels.decode_attention(qd, k, v)
    torch.cuda.synchronize()
    ref = oatt.decode_attention_f64(q[:, :, 0].double().numpy(), kc[:, :, :L].double().numpy(),
                                    vc[:, :, :L].double().numpy())
    assert o.shape == (B, H, 1, D) and o.dtype == dtype
    assert_close(o[:, :, 0].float().cpu().numpy(), ref, dtype, f"decode attn B={B} H={H} L={L} D={D}")


def test_decode_attention_matches_sdpa_in_model_view():
    """The KV-cache view the attention module passes (transposed storage of
    [batch, n_head, max_seq, head_dim]) gives the same result as torch's SDPA."""
    from src.model import kernels
    torch.manual_seed(0)
    B, H, D, Lmax, L = 2, 32, 128, 512, 300
    store_k = torch.randn(B, H, Lmax, D, device="cuda", dtype=torch.bfloat16)
    store_v = torch.randn(B, H, Lmax, D, device="cuda", dtype=torch.bfloat16)
    k = store_k.transpose(1, 2)[:, :L].transpose(1, 2)     # what KVCache.update + transpose(1, 2) give
    v = store_v.transpose(1, 2)[:, :L].transpose(1, 2)
    q = torch.randn(B, 1, H, D, device="cuda", dtype=torch.bfloat16).transpose(1, 2)
    o = kernels.decode_attention(q, k, v)
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float())
    assert_close(o.float().cpu().numpy(), ref.cpu().numpy(), torch.bfloat16, "model view vs SDPA")


@pytest.mark.parametrize("B,H,T,D,layout", [(2, 32, 1024, 16, "bthd"), (1, 4, 37, 16, "bthd"), (2, 3, 64, 32, "bhtd"),
                                            (1, 8, 200, 64, "bthd"), (1, 4, 130, 128, "bhtd"), (2, 2, 1, 16, "bthd"),
                                            (1, 8, 1024, 128, "bthd"), (1, 2, 3000, 16, "bthd")])
def test_prefill_attention_vs_oracle(B, H, T, D, layout):
    """Causal prefill attention (walsh_prefill_attention) against the float64
    oracle on the bf16-rounded inputs; q/k/v read in place from the
    projections' [B, T, H, D] rows or from [B, H, T, D] tensors.  head_dim 16
    up to about 2,300 positions runs the whole-head kernel, the rest (T =
    3000 included) the chunked one."""
    from src.model import kernels
    print(f"prefill case B={B} H={H} T={T} D={D} {layout}", flush=True)
    g = torch.Generator().manual_seed(B * 11 + T + D)
    shape = (B, T, H, D) if layout == "bthd" else (B, H, T, D)
    q, k, v = (torch.randn(*shape, generator=g).to(torch.bfloat16).cuda() for _ in range(3))
    if layout == "bthd":
        q, k, v = (t.transpose(1, 2) for t in (q, k, v))
    assert kernels.prefill_attention_supported(q, k, v)
    o = kernels.prefill_attention(q, k, v)
    o2 = kernels.prefill_attention(q, k, v)
    torch.cuda.synchronize()
    assert o.shape == (B, H, T, D) and o.is_contiguous()
    assert torch.equal(o, o2)
    ref = oatt.causal_attention_f64(*(t.double().cpu().numpy() for t in (q, k, v)))
    assert_close(o.double().cpu().numpy(), ref, torch.bfloat16, f"prefill B={B} H={H} T={T} D={D}")
