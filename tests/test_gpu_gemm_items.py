"""GPU parity of the persistent bf16 GEMM (csrc/gemm256.h) at the sizes where
each workgroup loops over several 256 x 256 work items: the octonion forward
at config-4 row counts (cayley_dickson_cuda.py:313-421), the n_embd-4096 MoE
router's first layer at prefill row counts (moe.py:407-411) and the octonion
weight gradient's split-K product (cayley_dickson_cuda.py:225-307).

A workgroup runs items first, first + G, ... of its XCD's share (G = its
XCD's workgroup count), so a wrong item index, a super-stage left over from
the previous item or an epilogue that overlaps the next item's loads shows
up as a whole wrong 256 x 256 tile.  Every test prints how many items the
busiest workgroup ran and requires more than one; rows at every 256-row tile
edge (and a few inside) are checked against the float64 oracle, and the whole
output against a float32 product of the same bf16 operands.
"""
import numpy as np
import pytest
import torch

from oracle import moe as omoe
from oracle import octonion as ooct
from oracle import ternary as otern

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def K():
    from src.model import kernels
    return kernels


def _items_per_workgroup(M, N, splits=1):
    """Items of the busiest workgroup under gemm256_plan (csrc/gemm256.h)."""
    cu = torch.cuda.get_device_properties(0).multi_processor_count
    items = -(-M // 256) * -(-N // 256) * splits
    per_xcd = -(-items // 8)
    wg_per_xcd = min(per_xcd, max(cu // 8, 1))
    return items, -(-per_xcd // wg_per_xcd)


def _edge_rows(M, extra=(1, 127, 128, 254)):
    """Rows at every 256-row tile edge plus a few inside each tile."""
    rows = set()
    for t in range(0, M, 256):
        for o in (0, 255) + tuple(extra):
            if t + o < M:
                rows.add(t + o)
    rows.add(M - 1)
    return np.array(sorted(rows))


def _bf16_ulp(a):
    e = np.floor(np.log2(np.maximum(np.abs(a), 2.0 ** -126)))
    return 2.0 ** (e - 7)


@pytest.mark.parametrize("M", [16700, 65536])
def test_octonion_forward_many_items(K, M):
    """OctonionFusedLinear(1024, 1024) on M rows in bf16 (config 4 at 65,536:
    1,024 items, 4 per workgroup; 16,700: a ragged last tile row)."""
    in_o = out_o = 128
    items, per_wg = _items_per_workgroup(M, 8 * out_o)
    print(f"octonion forward M={M}: {items} items, up to {per_wg} per workgroup", flush=True)
    assert per_wg > 1
    rng = np.random.default_rng(M)
    w = (rng.standard_normal((8, out_o, in_o)) * 0.02).astype(np.float32)
    codes = otern.ternary_codes(w, otern.absmean_gamma(w))
    beta = rng.uniform(0.05, 0.3, out_o).astype(np.float32)
    packed = torch.from_numpy(otern.pack_codes(codes)).cuda()
    B = K.octonion_prepare(packed, in_o, out_o, torch.bfloat16)
    gen = torch.Generator(device="cuda").manual_seed(M)
    x = torch.randn(M, 8 * in_o, device="cuda", generator=gen).bfloat16()
    bt = torch.from_numpy(beta).cuda()
    y = K.octonion_linear(x, in_o, out_o, B, bt)           # bf16 stack output
    yf = K.octonion_fused_linear(x, in_o, out_o, B, bt)     # the module's float32 output
    torch.cuda.synchronize()
    # the two epilogues agree on every item: bf16(acc beta) and
    # bf16(float(bf16(acc)) beta) differ by at most one bf16 ulp
    yb = yf.bfloat16().float()
    ulp_y = torch.exp2(torch.floor(torch.log2(yb.abs().clamp_min(2.0 ** -126))) - 7)
    assert torch.all((y.float() - yb).abs() <= ulp_y * 1.01)
    # whole output: float32 product of the same bf16 operands (hipBLASLt),
    # rounded to bf16 and scaled as the epilogue does
    A = torch.from_numpy(ooct.dense_matrix(codes, np.ones(out_o)).astype(np.float32)).cuda()
    acc = x.float() @ A.t()
    ref = acc.bfloat16().float() * bt.repeat(8)
    d = (yf - ref).abs()
    # the two float32 sums differ by rounding only; where they straddle a bf16
    # midpoint the bf16 values differ by one ulp
    ulp = torch.exp2(torch.floor(torch.log2(acc.abs().clamp_min(2.0 ** -126))) - 7)
    tol = ulp * bt.repeat(8) * 1.01 + 1e-6
    bad = int((d > tol).sum())
    nd = int((d > 0).sum())
    print(f"octonion forward M={M}: {nd} of {d.numel()} differ from the float32 product by at most one bf16 ulp, "
          f"{bad} by more", flush=True)
    assert bad == 0
    assert nd <= d.numel() // 100
    # float64 oracle on the tile-edge rows
    rows = _edge_rows(M)
    xs = x[torch.from_numpy(rows).cuda()].float().cpu().numpy().astype(np.float64)
    parts = xs.reshape(len(rows), 8, in_o).transpose(1, 0, 2)
    ref64 = ooct.octonion_linear_gpu_semantics(parts, codes, beta).transpose(1, 0, 2).reshape(len(rows), -1)
    got = yf[torch.from_numpy(rows).cuda()].double().cpu().numpy()
    a64 = ooct.octonion_linear_f64(parts, codes, np.ones(out_o)).transpose(1, 0, 2).reshape(len(rows), -1)
    tol64 = _bf16_ulp(a64) * np.tile(beta, 8).astype(np.float64) * 1.01 + 1e-6
    assert np.all(np.abs(got - ref64) <= tol64), float(np.max(np.abs(got - ref64) - tol64))


def _router_ref(x, w1, w2):
    """float64 router with autocast's bf16 roundings: (pre-activation,
    hidden = bf16(silu(bf16(x W1^T))), logits)."""
    def bf(a):
        return ooct.bf16_round(np.asarray(a, np.float32)).astype(np.float64)
    pre = bf(bf(x) @ bf(w1).T)
    s = bf(omoe.silu(pre))
    return pre, s, bf(s @ bf(w2).T)


@pytest.mark.parametrize("M", [16640, 65536])
def test_router_wide_many_items(K, M):
    """walsh_moe_router_wide_fwd at n_embd 4096 (config 5's router, W1 [1024,
    4096], 128 experts, k 6) on prefill row counts: the first product runs
    on the 256 x 256 GEMM with several items per workgroup.  Hidden units on
    the tile-edge rows within 1e-2 of the float64 oracle; routing bit-exact
    on the kernel's own probabilities for every token; assignments equal to
    the oracle's on the checked rows except where its k-th and (k+1)-th bf16
    logits lie within 4 bf16 ulps."""
    C, H, E, k = 4096, 1024, 128, 6
    items, per_wg = _items_per_workgroup(M, H)
    print(f"router M={M}: {items} items, up to {per_wg} per workgroup", flush=True)
    assert per_wg > 1
    rng = np.random.default_rng(M + 1)
    w1 = (rng.standard_normal((H, C)) * 0.02).astype(np.float32)
    w2 = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    gen = torch.Generator(device="cuda").manual_seed(M + 1)
    xt = torch.randn(M, C, device="cuda", generator=gen).bfloat16()
    w1t, w2t = (torch.from_numpy(a).cuda().bfloat16().contiguous() for a in (w1, w2))
    r, h = K.moe_router_wide(xt, w1t, w2t, E, k, dense=True, return_hidden=True)
    torch.cuda.synchronize()
    probs = r.probs.cpu().numpy()
    idx = r.topk_idx.cpu().numpy()
    assert np.array_equal(idx, omoe.topk_indices(probs, k).astype(np.int32))
    assert np.array_equal(r.count.cpu().numpy(), np.bincount(idx.reshape(-1), minlength=E).astype(np.int32))
    rows = _edge_rows(M)
    x_rows = xt[torch.from_numpy(rows).cuda()].float().cpu().numpy()
    _, h_ref, lg_ref = _router_ref(x_rows, w1, w2)
    hg = h[torch.from_numpy(rows).cuda()].float().cpu().numpy()
    err = np.abs(hg - h_ref).max() / np.abs(h_ref).max()
    print(f"router M={M}: hidden rel_max {err:.3e} on {len(rows)} rows", flush=True)
    assert err <= 1e-2
    # every checked row on its own (a wrong or stale 256 x 256 item would put
    # whole rows of some 256-column range off by O(1)): bf16 roundings of
    # the same values, one-ulp flips where the float32 and float64 sums
    # straddle a rounding midpoint
    per_row = np.linalg.norm(hg - h_ref, axis=1) / np.linalg.norm(h_ref, axis=1)
    per_blk = np.abs(hg - h_ref).reshape(len(rows), H // 256, 256).max(-1) / np.abs(h_ref).max()
    print(f"router M={M}: worst row rel_norm {per_row.max():.3e}, worst 256-column block rel_max "
          f"{per_blk.max():.3e}", flush=True)
    assert per_row.max() <= 5e-3 and per_blk.max() <= 1e-2
    _, _, idx_ref = omoe.route_from_probs(omoe.softmax(lg_ref), k)
    same = np.all(np.sort(idx[rows], -1) == np.sort(idx_ref, -1), axis=-1)
    srt = -np.sort(-lg_ref, axis=-1)
    gap = srt[:, k - 1] - srt[:, k]
    band = gap <= 4 * _bf16_ulp(srt[:, k - 1])
    print(f"router M={M}: rows={len(rows)} differ={int((~same).sum())} in_band={int(band.sum())} "
          f"exact_ties={int((gap == 0).sum())}", flush=True)
    assert np.all(same | band)


def test_octonion_weight_grad_many_items(K):
    """walsh_octonion_bwd_params at in_o = out_o = 128 and 20,000 tokens: C =
    gy^T x as 16 tiles x 32 K splits = 512 items (2 per workgroup), the last
    split partial, the partials added in split order, then the fold; dweight
    and dbeta against float64 (the octonion oracle's backward)."""
    in_o = out_o = 128
    M = 20000
    items, per_wg = _items_per_workgroup(8 * out_o, 8 * in_o, splits=32)
    print(f"octonion dW M={M}: {items} items, up to {per_wg} per workgroup", flush=True)
    assert per_wg > 1
    gen = torch.Generator().manual_seed(20000)
    latent = torch.rand(8, out_o, in_o, generator=gen) * 4 - 2
    beta = torch.randn(out_o, generator=gen)
    x = torch.randn(M, 8 * in_o, generator=gen).bfloat16()
    gy = torch.randn(M, 8 * out_o, generator=gen).bfloat16()
    q = K.ternary_quantize(latent.cuda(), codes=True, packed=True)
    _, dw, db = K.octonion_linear_bwd(x.cuda(), gy.cuda(), in_o, out_o, q["packed"], beta.cuda(),
                                      latent=latent.cuda(), need=(False, True, True))
    torch.cuda.synchronize()
    xp = np.stack(np.split(x.double().numpy(), 8, axis=-1))
    gp = np.stack(np.split(gy.double().numpy(), 8, axis=-1))
    _, dw_ref, db_ref = ooct.octonion_linear_bwd_f64(xp, q["codes"].cpu().numpy(), beta.double().numpy(), gp,
                                                     latent=latent.double().numpy())
    # float32 accumulation over 20,000 exact bf16 products: relative 1e-5
    for got, ref, what in ((dw.cpu().numpy(), dw_ref, "dweight"), (db.cpu().numpy(), db_ref, "dbeta")):
        e_norm = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        e_max = np.abs(got - ref).max() / np.abs(ref).max()
        print(f"octonion {what} M={M}: rel_norm {e_norm:.3e} rel_max {e_max:.3e}", flush=True)
        assert e_norm <= 1e-5 and e_max <= 1e-5, (what, e_norm, e_max)
