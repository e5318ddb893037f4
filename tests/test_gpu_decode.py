"""Batched KV-cache decode (config-5 decode harness) and config-5 layer shapes.

* A prefill with a KV cache followed by single-token decode steps at batch M
  gives the same last-position logits as an uncached forward over the whole
  prefix (the reference's parity definition for cached generation,
  chassis.py:612-650): float32 within 1e-5 relative.  In bf16 the cached
  steps run the split-K decode attention (float32 softmax weights) while the
  uncached forward runs torch's SDPA (bf16 weights), so both bf16 paths are
  held against the float32 uncached forward: the cached one within
  max(1e-2, 1.25 x the uncached bf16 path's own distance).
* One config-5 layer (n_embd 4096, 32 heads of 128, MoE with 128 experts,
  k = 6, 4 streams) in float32 against the oracle within 1e-5.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30), np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)


def make(C, n_layer, n_head, use_moe, block, seed=0, vocab=1000, kmax=6):
    from src.model import WalshConfig, mHCWalsh
    torch.manual_seed(seed)
    cfg = WalshConfig(block_size=block, vocab_size=vocab, n_layer=n_layer, n_head=n_head, n_embd=C,
                      algebra="hadamard", head_mixing=True, use_moe=use_moe, moe_max_experts=kmax,
                      use_channel_mod=False)
    return cfg, mHCWalsh(cfg, n_streams=4).cuda().eval()


@pytest.mark.parametrize("C,n_layer,use_moe,dtype", [(512, 2, False, torch.float32), (512, 2, True, torch.float32),
                                                     (512, 2, False, torch.bfloat16), (512, 2, True, torch.bfloat16),
                                                     (4096, 1, True, torch.float32)])
def test_cached_decode_matches_uncached(C, n_layer, use_moe, dtype):
    from src.model import KVCache
    cfg, model = make(C, n_layer, 32, use_moe, block=64, seed=C + n_layer)
    B, T0, steps = 3, 8, 4
    gen = torch.Generator().manual_seed(7)
    idx = torch.randint(0, cfg.vocab_size, (B, T0 + steps), generator=gen).cuda()
    kv = KVCache(n_layer, cfg.block_size, 32, C // 32, torch.device("cuda"),
                 dtype=torch.float32 if dtype == torch.float32 else torch.bfloat16, batch=B)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    ac = torch.autocast("cuda", dtype=torch.bfloat16, enabled=dtype == torch.bfloat16)
    with torch.no_grad(), ac:
        lg, _ = model(idx[:, :T0], kv_cache=kv, start_pos=0)
        kv.increment(T0)
        ref, _ = model(idx[:, :T0])
        r = rel(lg.float().cpu(), ref.float().cpu())
        print(f"prefill C={C} {dtype}: rel={r}")
        assert max(r) <= tol
        for s in range(steps):
            pos = T0 + s
            lg, _ = model(idx[:, pos:pos + 1], kv_cache=kv, start_pos=pos)
            kv.increment(1)
            ref, _ = model(idx[:, :pos + 1])
            if dtype == torch.float32:
                r = rel(lg[:, -1].float().cpu(), ref[:, -1].float().cpu())
                print(f"decode step {s} (M={B}, KV {pos + 1}): rel={r}")
                assert max(r) <= tol
                continue
            with torch.autocast("cuda", enabled=False):
                ref32, _ = model(idx[:, :pos + 1])
            r_unc = rel(ref[:, -1].float().cpu(), ref32[:, -1].cpu())
            r = rel(lg[:, -1].float().cpu(), ref32[:, -1].cpu())
            print(f"decode step {s} (M={B}, KV {pos + 1}): cached vs fp32 {r}, uncached bf16 vs fp32 {r_unc}")
            assert max(r) <= max(tol, 1.25 * max(r_unc))


def test_config5_layer_fp32_vs_oracle():
    from oracle.model import Oracle
    cfg, model = make(4096, 1, 32, True, block=64, seed=5)
    gen = torch.Generator().manual_seed(3)
    idx = torch.randint(0, cfg.vocab_size, (1, 16), generator=gen)
    with torch.no_grad():
        logits, _, h = model(idx.cuda(), return_hidden=True)
    sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    orc = Oracle(sd, 4096, 32, 1, n_streams=4, use_moe=True, moe_max_experts=6)
    with torch.no_grad():
        ref_logits, ref_h = orc.forward(idx, return_hidden=True)
    r = rel(h.cpu(), ref_h)
    print(f"config-5 layer hidden rel={r}")
    assert max(r) <= 1e-5
    r = rel(logits.cpu(), ref_logits)
    print(f"config-5 layer logits rel={r}")
    assert max(r) <= 1e-5


@pytest.mark.parametrize("C,use_moe", [(512, True), (4096, True)])
def test_decode_step_hip_graph_replays_match_eager(C, use_moe):
    """One decode step captured as a HIP graph (how the decode benchmark runs
    it): every replay, with eager work and synchronisation in between, equals
    the eager step."""
    from src.model import KVCache
    n_layer = 2 if C == 512 else 1
    cfg, model = make(C, n_layer, 32, use_moe, block=64, seed=11)
    B, pos = 4, 16
    kv = KVCache(n_layer, cfg.block_size, 32, C // 32, torch.device("cuda"), dtype=torch.bfloat16, batch=B)
    gen = torch.Generator().manual_seed(5)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        model(torch.randint(0, cfg.vocab_size, (B, pos), generator=gen).cuda(), kv_cache=kv, start_pos=0)
    idx = torch.randint(0, cfg.vocab_size, (B, 1), generator=gen).cuda()

    def step():
        kv.cached_len = pos
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            return model(idx, kv_cache=kv, start_pos=pos)[0]
    eager = step().float().clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = step()
    for r in range(3):
        junk = torch.randn(1024, 1024, device="cuda") @ torch.randn(1024, 1024, device="cuda")  # eager work between
        g.replay()
        torch.cuda.synchronize()
        diff = (out.float() - eager).abs().max().item()
        print(f"replay {r}: max |graph - eager| = {diff:.3e} (junk {junk.norm().item():.1f})")
        assert torch.equal(out.float(), eager)
