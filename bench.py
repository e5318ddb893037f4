"""Benchmark: tokens/s of the mHCWalsh forward on one MI355X.

Workload (the configuration the headline metric is quoted on): full
mHCWalsh forward, random init, bf16 autocast, n_layer 16, n_head 32,
n_embd 512, Hadamard algebra with head mixing, 4 mHC streams, MoE and channel
modulation off, tokens uniform over a 50257 vocabulary, batch 8 x seq 1024.
A step is one forward over that batch (inputs resident in HBM), replayed
as one captured HIP graph (``--eager`` times the launches one by one).

Other workloads (``--workload``), each printing one JSON line of its own:
  moe       HadamardMoE alone, bf16 autocast, n_embd 512 (16 experts, k = 6),
            x [16, 1024, 512]; inputs and outputs rotate over buffers larger
            than the 256 MB Infinity Cache so reads come from HBM;
  octonion  8 OctonionFusedLinear(1024, 1024) layers, bf16, x [32, 2048, 1024];
  hadamard  one HadamardLinear(512, 512), fp32, x [4, 256, 512] and a
            token sweep up to 262144 rows (rotated);
  prefill5  scaled model: n_embd 4096 (32 heads of 128), 24 layers, MoE with
            128 experts (k = 6), 4 streams, bf16, prefill of 64 x 1024 tokens;
  decode5   the same model decoding one token per sequence against a
            synthetic KV cache of length 4096, at batch 1, 16 and 64;
  hadamard_bwd  backward of one HadamardLinear(512, 512), bf16, x and the
            output gradient [8192, 512] (the headline model's layer shape),
            and a token sweep up to 262144 rows (rotated);
  train2    one training step of the headline model (bf16 autocast forward
            with targets, backward, AdamW), batch x seq tokens;
  walsh_load  a .walsh v4 file of config-5 ternary weights decoded on the
            GPU straight into 2-bit packed buffers;
  router    HadamardRouter alone at the n_embd-4096 width (hidden 1024,
            128 experts, k = 6), bf16, x [64, 1024, 4096];
  chanmod   the block's channel modulation x + cm(RMSNorm(x)) on the
            headline model's streams ([8, 1024, 4, 512] bf16, viewed as 32
            groups of 1024 rows), and a sweep with rotated buffers.

Prints ONE JSON line.  Besides the timed region it
  * repeats the K steps with HIP events around every hot-path launch (on the
    launching stream) to find the dominant kernel and its achieved
    algorithmic GB/s -> "roofline";
  * times the oracle's float32 CPU forward (the reference CPU path restated)
    on a bounded sample of the same workload -> "cpu_baseline".
"""
import argparse
import re
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "walsh-research_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
METRIC = "tokens/sec through Walsh layer stack at 1 GPU; % of HBM roofline (GB/s)"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=300)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--seq", type=int, default=1024)
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="budget of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline (profiling runs)")
    ap.add_argument("--no-roofline", action="store_true", help="skip the instrumented pass (profiling runs)")
    ap.add_argument("--eager", action="store_true", help="time eager launches instead of a captured HIP graph")
    ap.add_argument("--workload", default="mhcwalsh",
                    choices=["mhcwalsh", "moe", "octonion", "hadamard", "prefill5", "decode5", "hadamard_bwd",
                             "train2", "walsh_load", "chanmod", "router"])
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 256 MiB device copy 5 times (reference for HBM byte counters)")
    return ap.parse_args()


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "mhcwalsh_forward_hbm_traffic.txt")


def measured_traffic(kernel: str, workload: str = "mhcwalsh"):
    """HBM bytes per launch of ``kernel`` measured with rocprofv3 counters
    (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration), from
    the committed summary of the default workload; None when that kernel
    was not measured at this workload's shapes."""
    if workload != "mhcwalsh":
        return None
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                m = re.match(r"kernel=(\S+) .*\btraffic_bytes=([0-9.]+)", line)
                if m and m.group(1) == kernel:
                    return int(float(m.group(2)))
    except OSError:
        pass
    return None


def calibrate_copy(torch):
    """A plain device copy of known size: its FETCH_SIZE / WRITE_SIZE readings
    give the scale factor from counter units to bytes.  Also times torch's
    copy of 1 GiB each way (read + write), the practical HBM rate of a
    kernel that reads and writes each byte once."""
    n = 256 << 20
    src = torch.ones(n // 4, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "device copy", "bytes_read_per_launch": n, "bytes_written_per_launch": n,
                      "launches": 5}), flush=True)
    big = 1 << 30
    a = torch.ones(big // 4, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 100.0
    print(json.dumps({"copy": "torch copy_ of 1 GiB (read + write)", "us_per_copy": round(us, 1),
                      "read_plus_write_gbs": round(2 * big / (us * 1e-6) / 1e9, 1),
                      "frac_of_8tbs": round(2 * big / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}), flush=True)


def build_model(torch, batch, seq):
    from src.model import WalshConfig, mHCWalsh
    torch.manual_seed(0)
    cfg = WalshConfig(block_size=max(1024, seq), vocab_size=50257, n_layer=16, n_head=32, n_embd=512,
                      algebra="hadamard", head_mixing=True, use_moe=False, use_channel_mod=False)
    model = mHCWalsh(cfg, n_streams=4).cuda().eval()
    gen = torch.Generator().manual_seed(0)
    idx = torch.randint(0, cfg.vocab_size, (batch, seq), generator=gen).cuda()
    return cfg, model, idx


def cpu_setup(torch):
    """Run the CPU baseline on the physical cores this process may use: the
    affinity set's distinct (package, core) pairs from sysfs, capped by
    OMP_NUM_THREADS when set; torch.set_num_threads to that count.  Returns
    the host record reported beside every CPU figure."""
    import subprocess
    aff = sorted(os.sched_getaffinity(0))
    cores = set()
    for c in aff:
        base = f"/sys/devices/system/cpu/cpu{c}/topology/"
        try:
            with open(base + "physical_package_id") as f:
                pkg = f.read().strip()
            with open(base + "core_id") as f:
                core = f.read().strip()
            cores.add((pkg, core))
        except OSError:
            cores.add(("?", str(c)))
    host = {"affinity_cpus": len(aff), "physical_cores_in_affinity": len(cores)}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        f = {k.strip(): v.strip() for k, v in (ln.split(":", 1) for ln in out.splitlines() if ":" in ln)}
        host["lscpu_model"] = f.get("Model name")
        host["lscpu_n_phys"] = int(f.get("Socket(s)", "0")) * int(f.get("Core(s) per socket", "0"))
        host["lscpu_threads_per_core"] = int(f.get("Thread(s) per core", "1"))
    except (OSError, ValueError, subprocess.SubprocessError):
        pass
    n = len(cores)
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        host["omp_num_threads"] = int(omp)
        n = min(n, int(omp))
    torch.set_num_threads(max(1, n))
    host["torch_threads"] = torch.get_num_threads()
    return host


def cpu_baseline(torch, model, cfg, seq, budget_s):
    """Oracle float32 forward on the host cores: 1 x seq tokens per call,
    repeated until the budget is spent (at least once)."""
    from oracle.model import Oracle
    host = cpu_setup(torch)
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
                       f"(oracle/model.py), {el:.1f} s on {threads} threads", host=host)


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
    if args.workload != "mhcwalsh":
        line = {"moe": bench_moe, "octonion": bench_octonion, "hadamard": bench_hadamard, "prefill5": bench_prefill5,
                "decode5": bench_decode5, "hadamard_bwd": bench_hadamard_bwd,
                "train2": bench_train2, "walsh_load": bench_walsh_load,
                "chanmod": bench_chanmod, "router": bench_router}[args.workload](torch, args)
        print(json.dumps(line), flush=True)
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
    run = step
    graph = None
    if not args.eager:
        # the forward as one HIP graph (captured once, after the warmup has
        # built the weight caches): the same kernels, without the host's
        # per-launch cost between them
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        run = graph.replay
        run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms = dt * 1000.0 / args.steps
    value = tokens * args.steps / dt
    sustained = _sustained(torch, run)

    roofline = None
    kernels = None
    if not args.no_roofline:
        # per-kernel durations from an instrumented eager pass of up to 8
        # forwards, queued behind a GPU spin so that the launches run back
        # to back as in the graph (the host issues a forward's ~200 launches
        # and their timing events more slowly than the GPU runs them, several
        # times more slowly under a kernel tracer)
        n_roof = min(args.steps, 8)
        _queue_ahead(torch, n_roof, us_per_step=25000.0)
        with _hip.LaunchTimer() as lt:
            for _ in range(n_roof):
                step()
        kernels = lt.summary()
        # the HBM roofline is quoted for the dominant HBM-bound kernel: the
        # causal attention at head_dim 16 (between the q/k/v and output
        # projections) is bound by its exponentials and VALU work, not by
        # memory, so it is left out of the choice (its time stays in the
        # breakdown and in whole_forward)
        hbm_bound = [k for k in kernels if not k.startswith("prefill_attn")] or list(kernels)
        dom = max(hbm_bound, key=lambda k: kernels[k]["ms"])
        d = kernels[dom]
        avg_ms = d["ms"] / d["launches"]
        bytes_per_launch = d["bytes"] / d["launches"]
        achieved = bytes_per_launch / (avg_ms * 1e-3) / 1e9
        excluded = sorted(set(kernels) - set(hbm_bound))
        by_time = max(kernels, key=lambda k: kernels[k]["ms"])
        roofline = dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                        frac=round(achieved / HBM_PEAK_GBS, 4), traffic=measured_traffic(dom), kernel=dom,
                        avg_launch_us=round(avg_ms * 1000, 2), launches_per_step=d["launches"] // n_roof,
                        algorithmic_bytes_per_launch=int(bytes_per_launch),
                        selection="largest time per step among the HBM-bound hot-path kernels",
                        excluded_kernels={k: dict(reason="bound by its exponentials and VALU work, not memory",
                                                  ms_per_step=round(kernels[k]["ms"] / n_roof, 3))
                                          for k in excluded},
                        dominant_by_time=dict(kernel=by_time,
                                              ms_per_step=round(kernels[by_time]["ms"] / n_roof, 3)))
        # the whole forward: every hot-path kernel's algorithmic bytes per
        # step over the measured time per step (torch's embedding, stream
        # projection / merge and LM head are not counted)
        fwd_bytes = sum(v["bytes"] for v in kernels.values()) / n_roof
        whole = fwd_bytes / (ms * 1e-3) / 1e9
        roofline["whole_forward"] = dict(algorithmic_bytes_per_step=int(fwd_bytes), achieved=round(whole, 1),
                                         frac=round(whole / HBM_PEAK_GBS, 4),
                                         kernel_ms_per_step=round(sum(v["ms"] for v in kernels.values())
                                                                  / n_roof, 3))

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
        "execution": "eager launches" if graph is None else "one HIP graph per forward (captured after warmup)",
        "sustained": sustained,
    }
    if kernels is not None:
        line["kernels"] = {k: dict(launches_per_step=v["launches"] // n_roof,
                                   us_per_launch=round(v["ms"] * 1000 / v["launches"], 2),
                                   gbs=round(v["bytes"] / (v["ms"] * 1e-3) / 1e9, 1),
                                   ms_per_step=round(v["ms"] / n_roof, 3)) for k, v in kernels.items()}
    print(json.dumps(line), flush=True)


def _sustained(torch, run, min_s=1.0, min_reps=50, block=10):
    """Steps timed in blocks of ``block`` until at least ``min_s`` seconds and
    ``min_reps`` steps have run: median and spread of ms per step over the
    blocks (a steadier figure beside the K-step timed region)."""
    per, t_all, n = [], time.perf_counter(), 0
    while time.perf_counter() - t_all < min_s or n < min_reps:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(block):
            run()
        torch.cuda.synchronize()
        per.append((time.perf_counter() - t0) * 1000.0 / block)
        n += block
    per.sort()
    return dict(steps=n, seconds=round(time.perf_counter() - t_all, 2), median_ms_per_step=round(per[len(per) // 2], 4),
                min_ms_per_step=round(per[0], 4), max_ms_per_step=round(per[-1], 4))


def _queue_ahead(torch, steps, us_per_step=200.0):
    """Spin the GPU (torch's bounded busy-wait kernel) long enough for the
    host to queue ``steps`` steps behind it, so timed launches run back to
    back instead of each starting on an idle, down-clocked GPU."""
    torch.cuda.synchronize()
    torch.cuda._sleep(int(min(steps * us_per_step, 250000.0) * 2500))


def _time_graph_of_steps(torch, step, steps, n):
    """Seconds per step of ``steps`` steps captured in one HIP graph (after
    the caller's warmup has built the weight caches) and replayed once after
    one untimed replay; the last n outputs stay alive, so the outputs rotate
    over n buffers as the inputs do.  None when capture fails."""
    try:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            outs = [None] * n
            for i in range(steps):
                outs[i % n] = step(i)
        g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        g.replay()
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / steps
        del g, outs
        return dt
    except Exception as e:  # noqa: BLE001
        print(f"graph capture failed ({type(e).__name__}: {e}); timing eager launches", file=sys.stderr)
        return None


def _time_steps(torch, step, steps, warmup):
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def _roofline_of(kernels, steps, bound="hbm"):
    from src.model import _hip  # noqa: F401
    dom = max(kernels, key=lambda k: kernels[k]["ms"])
    d = kernels[dom]
    avg_ms = d["ms"] / d["launches"]
    if bound == "mfma":
        achieved = d["flops"] / d["launches"] / (avg_ms * 1e-3) / 1e12
        peak, unit = MFMA_BF16_PEAK_TFLOPS, "TFLOP/s"
    else:
        achieved = d["bytes"] / d["launches"] / (avg_ms * 1e-3) / 1e9
        peak, unit = HBM_PEAK_GBS, "GB/s"
    return dict(bound=bound, achieved=round(achieved, 1), peak=peak, unit=unit, frac=round(achieved / peak, 4),
                traffic=None, kernel=dom, avg_launch_us=round(avg_ms * 1000, 2),
                launches_per_step=d["launches"] // steps,
                algorithmic_bytes_per_launch=int(d["bytes"] / d["launches"]),
                flops_per_launch=int(d["flops"] / d["launches"]))


def _line(metric, value, unit, steps, warmup, ms, dtype, data, config, roofline, cpu, higher=True):
    return {"metric": metric, "value": round(value, 1), "unit": unit, "n_gpus": 1, "steps": steps,
            "warmup": warmup, "ms_per_step": round(ms, 4), "higher_is_better": higher, "scaling": "weak",
            "vs_baseline": None, "dtype": dtype, "data": data, "config": config, "roofline": roofline,
            "cpu_baseline": cpu}


def bench_moe(torch, args):
    """HadamardMoE forward (config 3): router N(0, 0.02), k = 6 for every token
    (the reference's top-k routing), reference output dtype (float32)."""
    from src.model import _hip
    from src.model.moe import HadamardMoE

    class Cfg:
        n_embd = 512
    torch.manual_seed(0)
    m = HadamardMoE(Cfg(), max_experts=6).cuda().eval()
    with torch.no_grad():
        for lin in (m.router.gate[0], m.router.gate[2]):
            lin.weight.normal_(0.0, 0.02)
    B, T, C = 16, 1024, 512
    nbuf = 8   # 8 x (16 MB in + 32 MB out) = 384 MB > 256 MB Infinity Cache
    gen = torch.Generator().manual_seed(0)
    xs = [torch.randn(B, T, C, generator=gen).bfloat16().cuda() for _ in range(nbuf)]

    def step(i):
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            return m(xs[i % nbuf])
    for i in range(max(args.warmup, 1)):
        step(i)
    # the step is one kernel launch, shorter than the host's cost of a
    # module call: the K timed steps run as one captured graph
    dt = None if args.eager else _time_graph_of_steps(torch, step, args.steps, nbuf)
    graphed = dt is not None
    if dt is None:
        dt = _time_steps(torch, step, args.steps, args.warmup)
    _queue_ahead(torch, args.steps)
    with _hip.LaunchTimer() as lt:
        for i in range(args.steps):
            step(i)
    roof = _roofline_of(lt.summary(), args.steps)
    cpu = None
    if not args.no_cpu:
        host = cpu_setup(torch)
        from oracle.moe import moe_forward
        sd = {k: v.detach().cpu().float().numpy() for k, v in m.state_dict().items()}
        xc = xs[0].float().cpu().numpy().reshape(-1, C)[:1024]
        t0, reps = time.perf_counter(), 0
        while time.perf_counter() - t0 < min(args.cpu_seconds, 10.0) or reps == 0:
            moe_forward(xc, sd["router.gate.0.weight"], sd["router.gate.2.weight"], sd["experts.gate_weights"],
                        sd["experts.up_weights"], sd["experts.down_weights"], 6)
            reps += 1
        el = time.perf_counter() - t0
        cpu = dict(value=round(reps * 1024 / el, 1), unit="tokens/s", cores=torch.get_num_threads(), kind="port",
                   host=host,
                   sample=f"{reps} x 1024 tokens through oracle/moe.py (numpy float64, all-expert einsum as the "
                          f"reference), {el:.1f} s")
    return _line("tokens/sec through the Hadamard MoE FFN at 1 GPU; % of HBM roofline (GB/s)", B * T / dt,
                 "tokens/s", args.steps, args.warmup, dt * 1e3, "bf16",
                 "synthetic: x N(0,1), router N(0,0.02), experts U(-1,1) latents",
                 {"workload": "HadamardMoE n_embd 512, 16 experts, k 6, expansion 4", "global_batch": B,
                  "seq_len": T, "parallelism": "single GPU", "rotated_buffers": nbuf,
                  "execution": "the timed steps as one HIP graph" if graphed else "eager launches"}, roof, cpu)


def bench_router(torch, args):
    """HadamardRouter.forward's routing (moe.py:407-447) at the n_embd-4096
    width: Linear(4096, 1024) -> SiLU -> Linear(1024, 128), softmax, top-6;
    weights N(0, 0.01) as the module's init, x [64, 1024, 4096] bf16."""
    from src.model import _hip
    from src.model.moe import HadamardRouter
    torch.manual_seed(0)
    m = HadamardRouter(4096, n_experts=128, max_experts=6).cuda().eval()
    B, T, C = 64, 1024, 4096
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(B * T, C, generator=gen).bfloat16().cuda()

    def step(i):
        with torch.no_grad():
            return m.route(x)
    dt = _time_steps(torch, step, args.steps, args.warmup)
    _queue_ahead(torch, args.steps)
    with _hip.LaunchTimer() as lt:
        for i in range(args.steps):
            step(i)
    roof = _roofline_of(lt.summary(), args.steps, bound="mfma")
    cpu = None
    if not args.no_cpu:
        host = cpu_setup(torch)
        from oracle.moe import route_from_probs, router_logits, softmax
        w1 = m.gate[0].weight.detach().float().cpu().numpy()
        w2 = m.gate[2].weight.detach().float().cpu().numpy()
        xc = x[:1024].float().cpu().numpy()
        t0, reps = time.perf_counter(), 0
        while time.perf_counter() - t0 < min(args.cpu_seconds, 10.0) or reps == 0:
            route_from_probs(softmax(router_logits(xc, w1, w2)), 6)
            reps += 1
        el = time.perf_counter() - t0
        cpu = dict(value=round(reps * 1024 / el, 1), unit="tokens/s", cores=torch.get_num_threads(), kind="port",
                   host=host,
                   sample=f"{reps} x 1024 tokens through oracle/moe.py's router (numpy), {el:.1f} s")
    line = _line("tokens/sec through the MoE router at 1 GPU; % of MFMA roofline", B * T / dt, "tokens/s",
                 args.steps, args.warmup, dt * 1e3, "bf16", "synthetic: x N(0,1), router weights N(0,0.01)",
                 {"workload": "HadamardRouter n_embd 4096, hidden 1024, 128 experts, k 6", "global_batch": B,
                  "seq_len": T, "parallelism": "single GPU"}, roof, cpu)
    line["library_gemm_reference"] = _library_gemm(torch, x, 1024)
    return line


def bench_octonion(torch, args):
    """8 octonion ternary linear layers (config 4), bf16, x [32, 2048, 1024]."""
    from src.model import _hip
    from src.model.octonion import OctonionFusedLinear
    torch.manual_seed(0)
    layers = [OctonionFusedLinear(1024, 1024).cuda() for _ in range(8)]
    with torch.no_grad():
        for l in layers:
            l.weight.normal_(0.0, 0.02)
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(32 * 2048, 1024, generator=gen).bfloat16().cuda()

    from src.model import kernels
    mats = [l.block_matrix(torch.bfloat16) for l in layers]

    def step(i):
        # each layer's bf16 output (beta folded, one rounding) is within one
        # bf16 ulp of bf16(the module's float32 output), the value the
        # reference's next layer reads (cayley_dickson_cuda.py:402)
        with torch.no_grad():
            h = x
            for l, B in zip(layers, mats):
                h = kernels.octonion_linear(h, l.in_o, l.out_o, B, l.beta)
            return h
    dt = _time_steps(torch, step, args.steps, args.warmup)
    _queue_ahead(torch, args.steps)
    with _hip.LaunchTimer() as lt:
        for i in range(args.steps):
            step(i)
    roof = _roofline_of(lt.summary(), args.steps, bound="mfma")
    cpu = None
    if not args.no_cpu:
        host = cpu_setup(torch)
        import numpy as np
        from oracle.octonion import octonion_linear_f64
        codes = np.sign(layers[0].weight.detach().cpu().numpy())  # timing only: any ternary matrix
        beta = layers[0].beta.detach().cpu().numpy()
        xp = x[:2048].float().cpu().numpy().reshape(2048, 8, 128).transpose(1, 0, 2)
        t0, reps = time.perf_counter(), 0
        while time.perf_counter() - t0 < min(args.cpu_seconds, 10.0) or reps == 0:
            octonion_linear_f64(xp, codes, beta)
            reps += 1
        el = time.perf_counter() - t0
        cpu = dict(value=round(reps * 2048 / 8 / el, 1), unit="tokens/s", cores=torch.get_num_threads(), kind="port",
                   host=host,
                   sample=f"{reps} x one layer on 2048 tokens (oracle/octonion.py, 64 block matmuls as the reference "
                          f"CPU path), {el:.1f} s; tokens/s of the 8-layer stack = layer rate / 8")
    line = _line("tokens/sec through the octonion ternary linear stack at 1 GPU; % of MFMA roofline",
                 32 * 2048 / dt, "tokens/s", args.steps, args.warmup, dt * 1e3, "bf16",
                 "synthetic: x N(0,1), weights N(0,0.02) latents",
                 {"workload": "8 x OctonionFusedLinear(1024, 1024)", "global_batch": 32, "seq_len": 2048,
                  "parallelism": "single GPU"}, roof, cpu)
    line["library_gemm_reference"] = _library_gemm(torch, x, 1024)
    return line


def _library_gemm(torch, x, n):
    """The GEMM x [M, K] @ W^T [K, n] as a plain library call (torch.matmul:
    hipBLASLt) on an independent bf16 matrix, for scale: what the platform's
    tuned GEMM reaches at the shape a hand-written kernel runs."""
    M, K = x.shape
    wt = torch.randn(n, K, device=x.device).bfloat16()
    for _ in range(3):
        x @ wt.t()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(20):
        x @ wt.t()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / 20
    return dict(what=f"torch.matmul (hipBLASLt), bf16, M {M} x N {n} x K {K}", us_per_call=round(us, 2),
                tflops=round(2.0 * M * n * K / (us * 1e-6) / 1e12, 1))


def bench_hadamard(torch, args):
    """One HadamardLinear(512, 512) in fp32 (config 1: x [4, 256, 512]) and a
    token sweep with rotated buffers (> 256 MB) for the HBM figure."""
    from src.model import _hip
    from src.model.hadamard import HadamardLinear
    torch.manual_seed(0)
    lin = HadamardLinear(512, 512).cuda()
    sweep = []
    for rows in (1024, 8192, 65536, 262144):
        nbuf = max(1, min(64, (512 << 20) // (rows * 512 * 4 * 2)))
        gen = torch.Generator().manual_seed(0)
        xs = [torch.randn(rows, 512, generator=gen).cuda() for _ in range(nbuf)]

        def step(i):
            with torch.no_grad():
                return lin(xs[i % nbuf])
        iters = max(args.steps, 200 if rows <= 8192 else 20)
        dt = _time_steps(torch, step, iters, args.warmup)
        _queue_ahead(torch, iters)
        with _hip.LaunchTimer() as lt:
            for i in range(iters):
                step(i)
        r = _roofline_of(lt.summary(), iters)
        sweep.append(dict(rows=rows, us_per_call=round(dt * 1e6, 2), kernel_us=r["avg_launch_us"],
                          kernel_gbs=r["achieved"], frac=r["frac"], rotated_buffers=nbuf))
        if rows == 1024:
            roof, dt1 = r, dt
    cpu = None
    if not args.no_cpu:
        host = cpu_setup(torch)
        import numpy as np
        from oracle.hadamard import hadamard_linear_torch32
        codes = np.sign(lin.weight.detach().cpu().numpy())
        xc = torch.randn(1024, 512)
        t0, reps = time.perf_counter(), 0
        while time.perf_counter() - t0 < min(args.cpu_seconds, 5.0) or reps == 0:
            hadamard_linear_torch32(xc, codes, lin.alpha.detach().cpu(), lin.beta.detach().cpu())
            reps += 1
        el = time.perf_counter() - t0
        cpu = dict(value=round(reps * 1024 / el, 1), unit="tokens/s", cores=torch.get_num_threads(), kind="port",
                   host=host,
                   sample=f"{reps} x [4, 256, 512] float32 through oracle/hadamard.py (the reference CPU einsums), "
                          f"{el:.1f} s")
    line = _line("tokens/sec through one Hadamard ternary linear at 1 GPU; % of HBM roofline (GB/s)",
                 1024 / dt1, "tokens/s", max(args.steps, 200), args.warmup, dt1 * 1e3, "f32",
                 "synthetic: x N(0,1), weights N(0,0.02) latents",
                 {"workload": "HadamardLinear(512, 512), x [4, 256, 512]", "global_batch": 4, "seq_len": 256,
                  "parallelism": "single GPU"}, roof, cpu)
    line["sweep"] = sweep
    # the same layer in bf16 (the dtype of the model configs) at prefill row counts
    sweep16 = []
    for rows in (65536, 262144, 1048576):
        # at least two inputs, so the inputs alone exceed the 256 MB Infinity
        # Cache (non-temporal output stores leave a lone input cached)
        nbuf = max(2, min(16, (768 << 20) // (rows * 512 * 2 * 2)))
        gen = torch.Generator(device="cuda").manual_seed(0)
        xs = [torch.randn(rows, 512, device="cuda", generator=gen).to(torch.bfloat16) for _ in range(nbuf)]

        def step16(i):
            with torch.no_grad():
                return lin(xs[i % nbuf])
        iters = max(args.steps, 20)
        dt = _time_steps(torch, step16, iters, args.warmup)
        _queue_ahead(torch, iters)
        with _hip.LaunchTimer() as lt:
            for i in range(iters):
                step16(i)
        r = _roofline_of(lt.summary(), iters)
        sweep16.append(dict(rows=rows, us_per_call=round(dt * 1e6, 2), kernel_us=r["avg_launch_us"],
                            kernel_gbs=r["achieved"], frac=r["frac"], rotated_buffers=nbuf))
        del xs
    line["sweep_bf16"] = sweep16
    return line


def bench_hadamard_bwd(torch, args):
    """Backward of one HadamardLinear(512, 512) in bf16 at the per-layer shape
    of the headline model (8 x 1024 tokens): gx, dalpha, dbeta and the STE
    weight gradient in one walsh_hadamard_linear_bwd call, plus a token sweep
    with rotated buffers (> 256 MB) for the HBM figure."""
    from src.model import _hip, kernels
    from src.model.hadamard import HadamardLinear
    torch.manual_seed(0)
    lin = HadamardLinear(512, 512).cuda()
    with torch.no_grad():
        lin.alpha.add_(0.1 * torch.randn_like(lin.alpha))
    _, _, kw = lin.ternary_state()
    kwt = lin.ternary_state_t()
    sweep = []
    for rows in (8192, 65536, 262144):
        nbuf = max(1, min(32, (768 << 20) // (rows * 512 * 2 * 3)))
        gen = torch.Generator(device="cuda").manual_seed(0)
        xs = [torch.randn(rows, 512, device="cuda", generator=gen).to(torch.bfloat16) for _ in range(nbuf)]
        gs = [torch.randn(rows, 512, device="cuda", generator=gen).to(torch.bfloat16) for _ in range(nbuf)]

        def step(i):
            return kernels.hadamard_linear_bwd(xs[i % nbuf], gs[i % nbuf], 16, 16, kw, kwt, lin.alpha, lin.beta,
                                               latent=lin.weight)
        iters = max(args.steps, 100 if rows <= 8192 else 20)
        dt = _time_steps(torch, step, iters, args.warmup)
        _queue_ahead(torch, iters)
        with _hip.LaunchTimer() as lt:
            for i in range(iters):
                step(i)
        r = _roofline_of(lt.summary(), iters)
        sweep.append(dict(rows=rows, us_per_call=round(dt * 1e6, 2), kernels_us=r["avg_launch_us"],
                          gbs=r["achieved"], frac=r["frac"], rotated_buffers=nbuf))
        if rows == 8192:
            roof, dt1 = r, dt
        del xs, gs
    roof["note"] = ("all four launches of one walsh_hadamard_linear_bwd call (dx+dalpha pass, dbeta pass, dW pass, "
                    "reduction) against the minimal traffic: x and gy read once, gx written once")
    cpu = None
    if not args.no_cpu:
        host = cpu_setup(torch)
        import numpy as np
        from oracle.hadamard import sylvester
        torch.manual_seed(1)
        M = 1024
        H = torch.tensor(sylvester(32), dtype=torch.float32)
        w = torch.tensor(np.sign(lin.weight.detach().cpu().numpy()), requires_grad=True)
        a = lin.alpha.detach().cpu().requires_grad_(True)
        b = lin.beta.detach().cpu().requires_grad_(True)
        x = torch.randn(M, 512, requires_grad=True)
        gy = torch.randn(M, 512)
        t_bwd, reps, t0 = 0.0, 0, time.perf_counter()
        while time.perf_counter() - t0 < min(args.cpu_seconds, 10.0) or reps == 0:
            # the reference's float32 CPU graph (fht_cuda.py:497-519)
            xs_ = x.view(M, 32, 16) * a
            xm = torch.einsum('mgi,gh->mhi', xs_, H)
            ym = torch.einsum('mgo,gh->mho', torch.einsum('mgi,goi->mgo', xm, w), H)
            y = (ym * b).reshape(M, 512)
            t1 = time.perf_counter()
            y.backward(gy)
            t_bwd += time.perf_counter() - t1
            x.grad = a.grad = b.grad = w.grad = None
            reps += 1
        cpu = dict(value=round(reps * M / t_bwd, 1), unit="tokens/s", cores=torch.get_num_threads(), kind="port",
                   host=host,
                   sample=f"{reps} backward passes of [1024, 512] float32 through the reference's CPU einsum graph "
                          f"(torch autograd), {t_bwd:.1f} s of backward")
    line = _line("tokens/sec through one Hadamard ternary linear backward at 1 GPU; % of HBM roofline (GB/s)",
                 8192 / dt1, "tokens/s", max(args.steps, 100), args.warmup, dt1 * 1e3, "bf16",
                 "synthetic: x, gy N(0,1); weights N(0,0.02) latents",
                 {"workload": "HadamardLinear(512, 512) backward, x and gy [8192, 512]", "global_batch": 8,
                  "seq_len": 1024, "parallelism": "single GPU"}, roof, cpu)
    line["sweep"] = sweep
    return line


def bench_chanmod(torch, args):
    """mHCLlamaBlock's channel modulation (mhc.py:528-532) at the headline
    model's stream shape: x [8, 1024, 4, 512] bf16 viewed as [32, 1024, 512],
    y = x + cm(RMSNorm(x)) with the ternary context MLP, one
    walsh_chanmod_fwd call (column sums, MLP, apply).  A sweep over more
    groups rotates buffers beyond the 256 MB Infinity Cache."""
    from src.model import _hip
    from src.model.chassis import RMSNorm
    from src.model.moe import HadamardChannelModulation
    torch.manual_seed(0)
    C = 512
    cm = HadamardChannelModulation(n_embd=C, residual_scale=0.5).cuda()
    norm = RMSNorm(C).cuda()
    sweep = []
    for G in (32, 128, 512):
        T = 1024
        nbuf = max(1, min(16, (768 << 20) // (G * T * C * 2 * 2)))
        gen = torch.Generator(device="cuda").manual_seed(0)
        xs = [torch.randn(G, T, C, device="cuda", generator=gen).to(torch.bfloat16) for _ in range(nbuf)]

        def step(i):
            with torch.no_grad():
                return cm.fused_residual(xs[i % nbuf], norm)
        iters = max(args.steps, 50)
        dt = _time_steps(torch, step, iters, args.warmup)
        _queue_ahead(torch, iters)
        with _hip.LaunchTimer() as lt:
            for i in range(iters):
                step(i)
        r = _roofline_of(lt.summary(), iters)
        sweep.append(dict(groups=G, rows=G * T, us_per_call=round(dt * 1e6, 2), kernels_us=r["avg_launch_us"],
                          gbs=r["achieved"], frac=r["frac"], rotated_buffers=nbuf))
        if G == 32:
            roof, dt1 = r, dt
        del xs
    roof["note"] = ("the three launches of one walsh_chanmod_fwd call (column sums, MLP, apply) against the "
                    "minimal traffic: x read once and y written once (the kernels read x twice)")
    cpu = None
    if not args.no_cpu:
        host = cpu_setup(torch)
        from oracle.model import Oracle
        sd = {"cm." + k: v.detach().float().cpu() for k, v in cm.state_dict().items()}
        orc = Oracle(sd, C, 1, 0)
        nw = norm.weight.detach().float().cpu()
        G, T = 32, 1024
        x = torch.randn(G, T, C)
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < min(args.cpu_seconds, 10.0) or reps == 0:
            with torch.no_grad():
                xn = orc.rmsnorm(x, nw)
                _ = x + orc.channel_mod(xn, "cm")
            reps += 1
        el = time.perf_counter() - t0
        cpu = dict(value=round(reps * G * T / el, 1), unit="rows/s", cores=torch.get_num_threads(), kind="port",
                   host=host,
                   sample=f"{reps} passes of the reference's float32 CPU graph (RMSNorm, mean, ternary MLP, "
                          f"per-block modulation, residual) over [32, 1024, 512], {el:.1f} s")
    line = _line("rows/sec through the block's channel modulation at 1 GPU; % of HBM roofline (GB/s)",
                 32 * 1024 / dt1, "rows/s", max(args.steps, 50), args.warmup, dt1 * 1e3, "bf16",
                 "synthetic: x N(0,1); context MLP N(0,0.02) / N(0,0.01) ternary latents",
                 {"workload": "mHC block channel modulation x + cm(RMSNorm(x)), streams [8, 1024, 4, 512] as "
                              "[32, 1024, 512]", "global_batch": 8, "seq_len": 1024, "parallelism": "single GPU"},
                 roof, cpu)
    line["sweep"] = sweep
    return line


def bench_train2(torch, args):
    """One training step of the headline model (n_layer 16, n_embd 512,
    hadamard + head mixing, 4 streams) at batch x seq tokens: bf16 autocast
    forward with targets, backward through the HIP backward kernels, and an
    AdamW step (torch, foreach) on every parameter."""
    from src.model import _hip
    cfg, model, idx = build_model(torch, args.batch, args.seq)
    model.train()
    gen = torch.Generator().manual_seed(2)
    tgt = torch.randint(0, cfg.vocab_size, idx.shape, generator=gen).cuda()
    opt = torch.optim.AdamW(model.parameters(), lr=1e-4, foreach=True, capturable=not args.eager)
    tokens = args.batch * args.seq

    def step(i=0):
        opt.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            _, loss = model(idx, targets=tgt)
        loss.backward()
        opt.step()
        return loss

    steps = max(1, min(args.steps, 10))
    run, execution = step, "eager launches"
    if not args.eager:
        # the whole step (forward, backward, AdamW) as one HIP graph: the
        # step is host-bound eagerly (57 ms of kernels in ~64 ms); warmup on
        # a side stream of default priority, then capture
        try:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(3):
                    step()
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            opt.zero_grad(set_to_none=True)
            with torch.cuda.graph(graph):
                with torch.autocast("cuda", dtype=torch.bfloat16):
                    _, static_loss = model(idx, targets=tgt)
                static_loss.backward()
                opt.step()
            run = lambda i=0: graph.replay()  # noqa: E731
            execution = "one HIP graph per training step (captured after warmup)"
        except Exception as e:  # capture is an optimisation: fall back to eager steps
            torch.cuda.synchronize()
            execution = f"eager launches (graph capture failed: {type(e).__name__}: {e})"[:200]
    dt = _time_steps(torch, run, steps, max(1, min(args.warmup, 2)))
    roof = None
    if not args.no_roofline:
        with _hip.LaunchTimer() as lt:
            for i in range(steps):
                step(i)
        summ = lt.summary()
        roof = _roofline_of(summ, steps)
        roof["hip_kernels"] = {k: dict(launches_per_step=v["launches"] // steps,
                                       us_per_launch=round(v["ms"] * 1000 / v["launches"], 2),
                                       ms_per_step=round(v["ms"] / steps, 3)) for k, v in summ.items()}
    cpu = None
    if not args.no_cpu:
        host = cpu_setup(torch)
        from oracle.model import Oracle
        sd = {k: v.detach().cpu() for k, v in model.state_dict().items()}
        orc = Oracle(sd, cfg.n_embd, cfg.n_head, cfg.n_layer, n_streams=4, grad=True, grad_dtype=torch.float32)
        seq = 128
        x, y = idx[:1, :seq].cpu(), tgt[:1, :seq].cpu()
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < min(args.cpu_seconds, 20.0) or reps == 0:
            orc.loss(x, y).backward()
            reps += 1
        el = time.perf_counter() - t0
        cpu = dict(value=round(reps * seq / el, 2), unit="tokens/s", cores=torch.get_num_threads(), kind="port",
                   host=host,
                   sample=f"{reps} x (1 x {seq} tokens) forward + backward of the same 16-layer model in float32 "
                          f"through the oracle (the reference's torch CPU graph, autograd), {el:.1f} s; no "
                          f"optimizer step")
    return _line("training tokens/sec of the Walsh layer stack at 1 GPU (forward + backward + AdamW)",
                 tokens / dt, "tokens/s", steps, max(1, min(args.warmup, 2)), dt * 1e3, "bf16",
                 "synthetic: random-init weights, tokens and targets uniform over 50257",
                 {"workload": "mHCWalsh training step, n_layer 16, n_head 32, n_embd 512, hadamard + head mixing, "
                              "4 mHC streams, MoE off, bf16 autocast, AdamW", "global_batch": args.batch,
                  "seq_len": args.seq, "parallelism": "single GPU"}, roof, cpu) | {"execution": execution}


def bench_walsh_load(torch, args):
    """Loading a .walsh v4 file (compress.py format) of config-5 ternary
    weights -- 24 layers of wq/wk/wv/wo [32, 128, 128] and gate/up
    [32, 342, 128], down [32, 128, 342] latents -- straight into 2-bit packed
    device buffers: the bitmask + sign decode runs on the GPU
    (walsh_ternary_from_bitmask).  value = packed ternary bytes produced per
    second by the decode kernels; the whole load (file read, host parse,
    host-to-device copies, decode) is reported beside it."""
    import tempfile
    from src.model import _hip
    from src.walsh_format import load_walsh, save_walsh
    gen = torch.Generator(device="cuda").manual_seed(0)
    sd = {}
    for l in range(24):
        for n in ("wq", "wk", "wv", "wo"):
            sd[f"layers.{l}.attention.{n}.inner.weight"] = torch.randn(32, 128, 128, device="cuda", generator=gen)
        for n, shp in (("gate_proj", (32, 342, 128)), ("up_proj", (32, 342, 128)), ("down_proj", (32, 128, 342))):
            sd[f"layers.{l}.feed_forward.{n}.inner.weight"] = torch.randn(*shp, device="cuda", generator=gen)
    values = sum(t.numel() for t in sd.values())
    path = os.path.join(tempfile.mkdtemp(), "config5.walsh")
    save_walsh(path, sd, {"n_embd": 4096, "n_layer": 24})
    fsize = os.path.getsize(path)
    load_walsh(path, packed_ternary=True)          # warm up (allocator, file cache)
    torch.cuda.synchronize()
    steps = max(1, min(args.steps, 5))
    t0 = time.perf_counter()
    for _ in range(steps):
        out, _ = load_walsh(path, packed_ternary=True)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    with _hip.LaunchTimer() as lt:
        for _ in range(steps):
            load_walsh(path, packed_ternary=True)
    k = lt.summary()["bitmask_decode"]
    dec_ms = k["ms"] / steps
    packed_bytes = sum(t.numel() for t in out.values())
    roof = _roofline_of({"bitmask_decode": k}, steps)
    roof["note"] = ("bytes per call: bitmask + sign bytes read, 2-bit packed bytes written; the three launches of "
                    "one call (word counts + scan, block-sum scan, decode) timed together")
    cpu = None
    if not args.no_cpu:
        host = cpu_setup(torch)
        import numpy as np
        from oracle import ternary as otern
        from oracle import walsh_format as owf
        name = "layers.0.feed_forward.gate_proj.inner.weight"
        codes = np.sign(sd[name].cpu().numpy()).astype(np.int8)
        bm, sg, nnz = owf.encode_codes(codes)
        reps, t1 = 0, time.perf_counter()
        while time.perf_counter() - t1 < min(args.cpu_seconds, 10.0) or reps == 0:
            otern.pack_codes(owf.decode_codes(bm, sg, codes.shape, nnz))
            reps += 1
        el = time.perf_counter() - t1
        cpu = dict(value=round(reps * codes.size / 4 / el / 1e9, 4), unit="GB/s of packed output", cores=1,
                   kind="port", sample=f"{reps} decodes of one [32, 342, 128] tensor (numpy restatement of "
                                       f"generate_compressed.py:70-105, then the 2-bit pack), {el:.1f} s")
    line = _line("packed ternary bytes per second decoded from .walsh v4 on 1 GPU", packed_bytes / (dec_ms * 1e-3) / 1e9,
                 "GB/s", steps, 1, dec_ms, "u8", "synthetic: N(0,1) latents, absmean codes (about 1/3 zeros)",
                 {"workload": ".walsh v4 load, config-5 ternary weights (24 layers x 7 matrices, "
                              f"{values / 1e6:.0f} M values, file {fsize / 1e6:.1f} MB)", "global_batch": 1,
                  "seq_len": 0, "parallelism": "single GPU"}, roof, cpu)
    line["whole_load_ms"] = round(dt * 1e3, 2)
    line["decode_kernel_ms"] = round(dec_ms, 3)
    return line


def _config5(torch, block_size):
    from src.model import WalshConfig, mHCWalsh
    torch.manual_seed(0)
    cfg = WalshConfig(block_size=block_size, vocab_size=50257, n_layer=24, n_head=32, n_embd=4096,
                      algebra="hadamard", head_mixing=True, use_moe=True, moe_max_experts=6, use_channel_mod=False)
    with torch.device("cuda"):
        model = mHCWalsh(cfg, n_streams=4).eval()
    return cfg, model


def _config5_cpu(torch, model, cfg, args, tokens):
    """Oracle float32 forward of the first layer on a bounded token sample,
    scaled to the 24-layer stack (layers cost the same)."""
    from oracle.model import Oracle
    host = cpu_setup(torch)
    keep = ("tok_embeddings.", "output.", "stream_proj.", "stream_merge.", "norm.", "freqs_cis", "layers.0.")
    sd = {k: v.detach().cpu() for k, v in model.state_dict().items() if k.startswith(keep)}
    orc = Oracle(sd, cfg.n_embd, cfg.n_head, 1, n_streams=4, use_moe=True, moe_max_experts=6)
    idx = torch.randint(0, cfg.vocab_size, (1, tokens), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        orc.forward(idx[:, :8])
        t0, reps = time.perf_counter(), 0
        while time.perf_counter() - t0 < min(args.cpu_seconds, 15.0) or reps == 0:
            orc.forward(idx)
            reps += 1
    el = time.perf_counter() - t0
    rate = reps * tokens / el / cfg.n_layer
    return dict(value=round(rate, 2), unit="tokens/s", cores=torch.get_num_threads(), kind="port", host=host,
                sample=f"{reps} x (1 x {tokens} tokens) through one layer of the oracle float32 forward "
                       f"(oracle/model.py) in {el:.1f} s; rate divided by the 24 layers (extrapolated)")


def bench_prefill5(torch, args):
    from src.model import _hip
    cfg, model = _config5(torch, 1024)
    B, T = 64, 1024
    idx = torch.randint(0, cfg.vocab_size, (B, T), generator=torch.Generator().manual_seed(0)).cuda()

    def step(i):
        with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
            return model(idx)[0]
    steps, warm = min(args.steps, 3), min(args.warmup, 1)
    dt = _time_steps(torch, step, steps, warm)
    with _hip.LaunchTimer() as lt:
        step(0)
    roof = _roofline_of(lt.summary(), 1)
    cpu = None if args.no_cpu else _config5_cpu(torch, model, cfg, args, 64)
    line = _line("tokens/sec through Walsh layer stack at 1 GPU; % of HBM roofline (GB/s)", B * T / dt, "tokens/s",
                 steps, warm, dt * 1e3, "bf16", "synthetic: random-init weights, tokens uniform over 50257",
                 {"workload": "mHCWalsh prefill, n_layer 24, n_embd 4096, n_head 32 (head_dim 128), hadamard + head "
                              "mixing, MoE 128 experts k 6, 4 mHC streams", "global_batch": B, "seq_len": T,
                  "parallelism": "single GPU"}, roof, cpu)
    line["kernels"] = {k: dict(launches=v["launches"], us_per_launch=round(v["ms"] * 1000 / v["launches"], 2),
                               gbs=round(v["bytes"] / (v["ms"] * 1e-3) / 1e9, 1), ms=round(v["ms"], 3))
                       for k, v in lt.summary().items()}
    return line


def bench_decode5(torch, args):
    from src.model import KVCache, _hip
    cfg, model = _config5(torch, 4096)
    kv_len = 4095     # cached tokens; the decoded token is position 4096
    bmax = 64
    kv = KVCache(cfg.n_layer, 4096, cfg.n_head, cfg.n_embd // cfg.n_head, torch.device("cuda"),
                 dtype=torch.bfloat16, batch=bmax)
    sweep = []
    for b in (1, 16, 64):
        idx = torch.randint(0, cfg.vocab_size, (b, 1), generator=torch.Generator().manual_seed(b)).cuda()

        def eager(i=0):
            kv.cached_len = kv_len   # synthetic cache content; every step decodes position kv_len
            with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
                return model(idx, kv_cache=kv, start_pos=kv_len)[0]
        steps = max(args.steps, 10)
        dt_eager = _time_steps(torch, eager, steps, args.warmup)
        with _hip.LaunchTimer() as lt:
            for i in range(steps):
                eager(i)
        k = lt.summary()
        hot_ms = sum(v["ms"] for v in k.values()) / steps
        # the step as one HIP graph: removes the per-launch host cost of the
        # ~40 launches per layer (the eager step is launch-bound at small batch)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                eager()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            eager()
        dt = _time_steps(torch, lambda i: graph.replay(), steps, args.warmup)
        del graph
        sweep.append(dict(batch=b, ms_per_step=round(dt * 1e3, 3), tokens_per_s=round(b / dt, 1),
                          eager_ms_per_step=round(dt_eager * 1e3, 3),
                          hot_path_kernel_ms_per_step=round(hot_ms, 3),
                          kernels={n: round(v["ms"] * 1000 / v["launches"], 2) for n, v in k.items()}))
        if b == bmax:
            roof = _roofline_of(k, steps)
            dt64 = dt
    cpu = None if args.no_cpu else _config5_cpu(torch, model, cfg, args, 16)
    line = _line("tokens/sec through Walsh layer stack at 1 GPU; % of HBM roofline (GB/s)", bmax / dt64, "tokens/s",
                 max(args.steps, 10), args.warmup, dt64 * 1e3, "bf16",
                 "synthetic: random-init weights, zero KV cache of length 4095",
                 {"workload": "mHCWalsh decode, n_layer 24, n_embd 4096, MoE 128 experts, KV 4096", "global_batch": bmax,
                  "seq_len": 1, "parallelism": "single GPU"}, roof, cpu)
    line["sweep"] = sweep
    return line


if __name__ == "__main__":
    main()
