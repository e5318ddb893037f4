"""Benchmark: tokens/s of the mHCWalsh forward on one MI355X.

Workload (the configuration the headline metric is quoted on): full
mHCWalsh forward, random init, bf16 autocast, n_layer 16, n_head 32,
n_embd 512, Hadamard algebra with head mixing, 4 mHC streams, MoE and channel
modulation off, tokens uniform over a 50257 vocabulary, batch 8 x seq 1024.
A step is one forward over that batch (inputs resident in HBM).

Prints ONE JSON line.  Besides the timed region it
  * repeats the K steps with HIP events around every hot-path launch (on the
    launching stream) to find the dominant kernel and its achieved
    algorithmic GB/s -> "roofline";
  * times the oracle's float32 CPU forward (the reference CPU path restated)
    on a bounded sample of the same workload -> "cpu_baseline".
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "walsh-research_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0
METRIC = "tokens/sec through Walsh layer stack at 1 GPU; % of HBM roofline (GB/s)"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--seq", type=int, default=1024)
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline (profiling runs)")
    ap.add_argument("--no-roofline", action="store_true", help="skip the instrumented pass (profiling runs)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 256 MiB device copy 5 times (reference for HBM byte counters)")
    return ap.parse_args()


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "mhcwalsh_forward_hbm_traffic.txt")


def measured_traffic(kernel: str):
    """HBM bytes per launch of ``kernel`` measured with rocprofv3 counters
    (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration), from
    the committed summary; None when that kernel was not measured."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("kernel=") and "traffic_bytes=" in line:
                    fields = dict(kv.split("=", 1) for kv in line.split())
                    if fields["kernel"] == kernel:
                        return int(float(fields["traffic_bytes"]))
    except OSError:
        pass
    return None


def calibrate_copy(torch):
    """A plain device copy of known size: its FETCH_SIZE / WRITE_SIZE readings
    give the scale factor from counter units to bytes."""
    n = 256 << 20
    src = torch.ones(n // 4, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "device copy", "bytes_read_per_launch": n, "bytes_written_per_launch": n,
                      "launches": 5}), flush=True)


def build_model(torch, batch, seq):
    from src.model import WalshConfig, mHCWalsh
    torch.manual_seed(0)
    cfg = WalshConfig(block_size=max(1024, seq), vocab_size=50257, n_layer=16, n_head=32, n_embd=512,
                      algebra="hadamard", head_mixing=True, use_moe=False, use_channel_mod=False)
    model = mHCWalsh(cfg, n_streams=4).cuda().eval()
    gen = torch.Generator().manual_seed(0)
    idx = torch.randint(0, cfg.vocab_size, (batch, seq), generator=gen).cuda()
    return cfg, model, idx


def cpu_baseline(torch, model, cfg, seq, budget_s):
    """Oracle float32 forward on the host cores: 1 x seq tokens per call,
    repeated until the budget is spent (at least once)."""
    from oracle.model import Oracle
    threads = torch.get_num_threads()
    sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    orc = Oracle(sd, cfg.n_embd, cfg.n_head, cfg.n_layer, n_streams=4)
    gen = torch.Generator().manual_seed(1)
    idx = torch.randint(0, cfg.vocab_size, (1, seq), generator=gen)
    with torch.no_grad():
        orc.forward(idx[:, :64])                      # warm caches (ternary codes, allocator)
        reps, t0 = 0, time.perf_counter()
        while True:
            orc.forward(idx)
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget_s or el / reps * (reps + 1) > 2.5 * budget_s:
                break
    return dict(value=round(reps * seq / el, 2), unit="tokens/s", cores=threads, kind="port",
                sample=f"{reps} x (1 x {seq} tokens) of the same 16-layer forward in float32 "
                       f"(oracle/model.py), {el:.1f} s on {threads} threads")


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              f"(the hot path shards over tokens with no exchange, see DESIGN.md)", file=sys.stderr)
        sys.exit(2)
    import torch
    from src.model import _hip

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.calibrate_copy:
        calibrate_copy(torch)
        return
    _hip.lib()
    cfg, model, idx = build_model(torch, args.batch, args.seq)
    tokens = args.batch * args.seq

    def step():
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            return model(idx)[0]

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms = dt * 1000.0 / args.steps
    value = tokens * args.steps / dt

    roofline = None
    kernels = None
    if not args.no_roofline:
        with _hip.LaunchTimer() as lt:
            for _ in range(args.steps):
                step()
        kernels = lt.summary()
        dom = max(kernels, key=lambda k: kernels[k]["ms"])
        d = kernels[dom]
        avg_ms = d["ms"] / d["launches"]
        bytes_per_launch = d["bytes"] / d["launches"]
        achieved = bytes_per_launch / (avg_ms * 1e-3) / 1e9
        roofline = dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                        frac=round(achieved / HBM_PEAK_GBS, 4), traffic=measured_traffic(dom), kernel=dom,
                        avg_launch_us=round(avg_ms * 1000, 2), launches_per_step=d["launches"] // args.steps,
                        algorithmic_bytes_per_launch=int(bytes_per_launch))

    cpu = None if args.no_cpu else cpu_baseline(torch, model, cfg, args.seq, args.cpu_seconds)

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: random-init weights, tokens uniform over 50257",
        "config": {"workload": "mHCWalsh forward, n_layer 16, n_head 32, n_embd 512, hadamard + head mixing, "
                               "4 mHC streams, MoE off", "global_batch": args.batch, "seq_len": args.seq,
                   "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    if kernels is not None:
        line["kernels"] = {k: dict(launches_per_step=v["launches"] // args.steps,
                                   us_per_launch=round(v["ms"] * 1000 / v["launches"], 2),
                                   gbs=round(v["bytes"] / (v["ms"] * 1e-3) / 1e9, 1),
                                   ms_per_step=round(v["ms"] / args.steps, 3)) for k, v in kernels.items()}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
