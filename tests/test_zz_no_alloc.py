"""walsh_decode_attention_static, the allocation-free decode attention,
against walsh_decode_attention (workspace entry point) through the C ABI.

The two share their kernels and split, so the results are bitwise equal.
Two calls in a row on one GPU share the static scratch array; the second is
smaller than the first, so stale partials of the first call would show up
if the second read any slot it did not write.  A shape whose partials exceed
the array is rejected on the host before any launch.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import attention as oatt

pytestmark = pytest.mark.gpu


def _case(B, H, L, D, dtype, Lmax, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn(B, H, 1, D, device="cuda", generator=g).to(dtype)
    cache_k = torch.randn(B, H, Lmax, D, device="cuda", generator=g).to(dtype)
    cache_v = torch.randn(B, H, Lmax, D, device="cuda", generator=g).to(dtype)
    return q, cache_k[:, :, :L], cache_v[:, :, :L]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_static_decode_attention_equals_workspace_variant(dtype):
    from src.model import kernels
    print(f"no-alloc decode attention, dtype {dtype}", flush=True)
    shapes = [(64, 32, 4096, 128), (3, 32, 700, 64)]    # the second call is smaller
    outs = {}
    for i, (B, H, L, D) in enumerate(shapes):
        q, k, v = _case(B, H, L, D, dtype, Lmax=L + 8, seed=i)
        ref = kernels.decode_attention(q, k, v)
        out = torch.full_like(ref, float("nan"))
        got = kernels.decode_attention_static(q, k, v, out=out)
        torch.cuda.synchronize()
        assert got is out
        assert torch.equal(out, ref), f"call {i} B={B} H={H} L={L} D={D}"
        o64 = oatt.decode_attention_f64(q[:, :, 0].float().cpu().numpy(), k.float().cpu().numpy(),
                                        v.float().cpu().numpy())
        r = np.linalg.norm(out[:, :, 0].float().cpu().numpy() - o64) / np.linalg.norm(o64)
        print(f"call {i} B={B} H={H} L={L} D={D}: bitwise equal to the workspace variant; rel to float64 {r:.2e}")
        assert r <= (1e-2 if dtype == torch.bfloat16 else 1e-5)
        outs[i] = out


def test_static_decode_attention_rejects_shapes_beyond_its_scratch():
    from src.model import _hip
    lib = _hip.lib()
    q, k, v = _case(1, 1, 8, 128, torch.bfloat16, Lmax=8, seed=3)
    o = torch.empty_like(q)
    B, H, L, D = 4096, 32, 4096, 128          # 136 MB of partials > 8 MiB
    need = lib.walsh_decode_attention_workspace_bytes(B, H, L, D)
    assert need > 8 << 20
    rc = lib.walsh_decode_attention_static(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(),
                                           k.stride(0), k.stride(1), k.stride(2), B, H, L, D, ctypes.c_float(0.1),
                                           o.data_ptr(), o.stride(0), o.stride(1), _hip.dtype_code(q.dtype),
                                           _hip.stream(q.device))
    msg = lib.walsh_last_error().decode()
    print(f"rc {rc}: {msg}")
    assert rc != 0 and "static maximum" in msg
