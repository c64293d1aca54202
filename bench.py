"""Benchmark of the packed-state GDN decode step on one MI355X.

Workload: STEPQuant@6 GDN decode, one layer,
B=256 requests, 16 key heads shared GQA-style by 32 value heads, dk=dv=128,
q/k/v bf16 column views of one mixed_qkv row (as the serving adapter passes
them), raw gates a ~ N(0,1) with A_log = 0, dt_bias = 0 (g = -softplus(a)),
beta = sigmoid(N(0,1)), L2-normalised q/k in the kernel.  Per-head widths
{4, 6, 8} averaging 6 (page = 409,600 B).  Initial state ~ N(0, 0.05^2)
encoded into slots 1..B.  One step = one decode step of the layer including
the writeback of the requantised page; steps are replayed from a HIP graph
and the state evolves from step to step.  Consecutive steps use disjoint
sets of B slots of one pool in turn (``--slot-sets``, 4 by default: 1,025
pages, 420 MB), so the pages a step reads were last touched four steps
earlier, with 315 MB of other pages read and written in between, and come
from HBM rather than from the 256 MB Infinity Cache.

Prints one JSON line (metric, value = state-head updates/s, roofline of the
dominant kernel, CPU baseline from the oracle on a bounded sample).

Timing: the GPU clocks ramp up under load and fall back within a fraction
of a second of idling, so steps are replayed for ``--warm-seconds`` (2 s)
before the counted warm-up.  Decode steps are captured ``--graph-steps`` per
graph (the largest divisor of ``--steps`` up to 16): a serving graph runs its
layers' kernels back to back, without a host launch between them.  Every
timed step is a whole decode step of all B requests.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "state-head updates/sec at B=256 decode; achieved HBM GB/s vs peak"
PEAK_GBS = 8000.0


def parse():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=1024)
    p.add_argument("--warmup", type=int, default=32)
    p.add_argument("--batch", type=int, default=None, help="requests (default 256; prefill: 8)")
    p.add_argument("--heads", type=int, default=32)
    p.add_argument("--key-heads", type=int, default=16)
    p.add_argument("--arch", choices=["gdn", "kda"], default="gdn")
    p.add_argument("--nominal", type=int, choices=[4, 6], default=6)
    p.add_argument("--async-writeback", action="store_true",
                   help="split readout (foreground) and writer (writeback stream); under graphs the writers "
                        "are deferred and forked at attention windows, joined at the end of the step")
    p.add_argument("--slot-sets", type=int, default=4,
                   help="disjoint sets of B slots in each pool, used by consecutive steps in turn, so a set's "
                        "pages have left the 256 MB Infinity Cache before the set comes round again (4 sets: "
                        "315 MB of other pages read and written in between)")
    p.add_argument("--foreground-gflop", type=float, default=0.0,
                   help="stand-in for a layer's other work (attention, MLP): a bf16 matmul [B, 4096] x "
                        "[4096, n] of about this many GFLOP after each attention window, on the foreground "
                        "stream; with --async-writeback the previous layer's writer can run beside it")
    p.add_argument("--writer-cus", type=int, default=-1,
                   help="with --async-writeback: -1 a plain stream for the writers, 0 or more the stream of "
                        "writeback_resources (a CU-masked stream over that many compute units; 0 unrestricted)")
    p.add_argument("--layers", type=int, default=1,
                   help="recurrent layers per step, each with its own pool (an attention window before each)")
    p.add_argument("--cpu-sample", type=int, default=-1,
                   help="requests in the CPU-baseline sample (-1: auto, 0: skip)")
    p.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "traffic_gdn6_b256.json"),
                   help="json with HBM bytes per launch measured by rocprofv3 (see profiles/)")
    p.add_argument("--no-graph", action="store_true",
                   help="launch steps eagerly (for rocprofv3 --pmc runs, which count per dispatch)")
    p.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                   help="only run a device-to-device copy of MIB MiB five times (counter calibration)")
    p.add_argument("--workload", choices=["decode", "prefill"], default="decode",
                   help="prefill: configs[4], chunked GDN prefill into 5 prefix slots per request")
    p.add_argument("--seq-len", type=int, default=2048, help="prefill tokens per sequence")
    p.add_argument("--state-format", default="stepquant",
                   help="decode on a baseline-format pool (fp32, sym_int{4,6,8}_g128, dsq_int{4,6}) instead")
    p.add_argument("--checkpoints", type=int, default=5, help="prefill prefix slots per request")
    p.add_argument("--warm-seconds", type=float, default=2.0,
                   help="replay steps for this long before the counted warm-up: the GPU clocks ramp up "
                        "under load and drop again within a fraction of a second of idling")
    p.add_argument("--graph-steps", type=int, default=0,
                   help="consecutive decode steps captured per graph (0: the largest divisor of --steps "
                        "up to 16), as a serving graph runs its layers back to back")
    p.add_argument("--cpu-threads", type=int, default=0,
                   help="threads of the CPU baseline (0: the cores this process may use, at most 16)")
    p.add_argument("--cpu-steps", type=int, default=4, help="full decode steps of the CPU baseline sample")
    a = p.parse_args()
    if a.batch is None:
        a.batch = 8 if a.workload == "prefill" else 256
    return a


def make_plan(torch, arch, H, K, nominal, seed=0):
    g = torch.Generator().manual_seed(seed)
    if arch == "gdn":
        if nominal == 6:
            widths = torch.tensor([4] * (H // 4) + [6] * (H // 2) + [8] * (H - H // 4 - H // 2))
        else:  # {2,4,6,8} averaging 4 (the reference has no 3-bit width)
            n2 = n4 = 3 * H // 8
            n6 = (H - n2 - n4) // 2
            widths = torch.tensor([2] * n2 + [4] * n4 + [6] * n6 + [8] * (H - n2 - n4 - n6))
        widths = widths[torch.randperm(H, generator=g)]
        bits = widths[:, None].expand(H, K).contiguous()
    else:
        if nominal == 6:
            bits = torch.tensor([4, 6, 8])[torch.randint(0, 3, (H, K), generator=g)]
        else:
            bits = torch.tensor([2, 2, 2, 4, 4, 4, 6, 8])[torch.randint(0, 8, (H, K), generator=g)]
        bits[torch.rand(H, K, generator=g) < .01] = 16
    impact = torch.rand(H, K, generator=g) + .5
    return bits, impact


def host_cores():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_baseline(bits, impact, arch, B, H, HK, K, V, sample, steps=4, threads=0, group=32):
    """Oracle (C restatement of the reference CPU path) on a bounded sample:
    ``steps`` full decode steps of ``sample`` requests, the requests split
    over ``threads`` host threads (the oracle's C calls release the GIL and
    every (request, head) tile is independent)."""
    import numpy as np
    from concurrent.futures import ThreadPoolExecutor
    from oracle import oracle as O
    threads = threads or min(16, host_cores())
    threads = max(1, min(threads, sample))
    rng = np.random.default_rng(1)
    plan = O.Plan(arch, bits.numpy(), impact.numpy(), group)
    lay = O.layout(plan, V)
    pages = np.zeros((sample + 1, lay.page_bytes), np.uint8)
    slots = np.arange(1, sample + 1)
    q = rng.standard_normal((sample, HK * K)).astype(np.float32)
    k = rng.standard_normal((sample, HK * K)).astype(np.float32)
    v = rng.standard_normal((sample, H, V)).astype(np.float32)
    a = rng.standard_normal((sample, H, K) if arch == "kda" else (sample, H)).astype(np.float32)
    b = rng.standard_normal((sample, H)).astype(np.float32)
    zeros_h = np.zeros(H, np.float32)
    bias = np.zeros(H * K if arch == "kda" else H, np.float32)
    parts = [p for p in np.array_split(np.arange(sample), threads) if p.size]

    def init(idx):
        x = (np.random.default_rng(2 + int(idx[0])).standard_normal((idx.size, H, K, V)) * .05).astype(np.float32)
        O.encode_page(x, slots[idx], plan, lay, pages)

    def one(idx):
        s = slots[idx]
        state = O.decode_page(pages, s, plan, lay, V)
        qp, kp, ld, bt = O.prepare(q[idx], k[idx], a[idx], b[idx], H, K, arch == "kda", True, K ** -.5,
                                   zeros_h, bias)
        _, upd = O.delta_step(state, qp, kp, v[idx], ld, bt)
        O.encode_page(upd, s, plan, lay, pages)  # each thread writes only its own requests' pages

    with ThreadPoolExecutor(len(parts)) as ex:
        list(ex.map(init, parts))
        t0 = time.perf_counter()
        for _ in range(steps):
            list(ex.map(one, parts))
        dt = time.perf_counter() - t0
    return dict(value=steps * sample * H / dt, unit="updates/s", cores=len(parts), kind="port",
                sample=f"{steps} decode steps of {sample} requests x {H} heads of the same workload (decode page, "
                       f"prepare, delta_step, fit_state + page store), requests split over {len(parts)} threads, "
                       f"{dt:.2f} s wall")


PEAK_BF16_TFLOPS = 2500.0


def timed_steps(torch, one, block, per_block, steps, warmup, warm_seconds):
    """Warm by wall time, then ``warmup`` single steps, then exactly ``steps``
    steps as ``steps / per_block`` launches of ``block``, timed with HIP
    events on the launching stream between two synchronisations.
    Returns (ms per step, wall seconds of the timed region)."""
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < warm_seconds:
        block()
        torch.cuda.synchronize()  # keeps the launch queue shallow: the timed region starts from no backlog
    for _ in range(warmup):
        one()
    torch.cuda.synchronize()
    cur = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(cur)
    for _ in range(steps // per_block):
        block()
    end.record(cur)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps, time.perf_counter() - t0


def prefill_flops(n_chunks, C=64, K=128, V=128):
    """Algorithmic FLOPs of the chunked recurrence (chunks of C tokens) per chunk-head:
    K K^T and Q K^T (2 x 2C^2K), the triangular inverse (C^3/3 x 2), W and U
    (2C^2K + 2C^2V), W S and Q S (2 x 2CKV), (M o QK^T) Delta (2C^2V) and
    K^T Delta (2CKV)."""
    per = 6 * C * C * K + 4 * C * C * V + 6 * C * K * V + (2 * C ** 3) // 3
    return n_chunks * per


def bench_prefill(a, torch):
    from stepquant_amd.kernels.pool import PackedStatePool
    from stepquant_amd.quantization import QuantizationPlan
    dev = torch.device("cuda:0")
    B, H, HK, K, V, T = a.batch, a.heads, a.key_heads, 128, 128, a.seq_len
    NC = a.checkpoints
    kda = a.arch == "kda"
    bits, impact = make_plan(torch, a.arch, H, K, 6)
    plan = QuantizationPlan(a.arch, bits.to(dev), impact.to(dev))
    pool = PackedStatePool(plan, B * (NC + 1) + 1, V)
    g = torch.Generator(device=dev).manual_seed(0)
    tot = B * T
    q = torch.randn(tot, HK * K, device=dev, generator=g).to(torch.bfloat16)
    k = torch.randn(tot, HK * K, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(tot, H * V, device=dev, generator=g).to(torch.bfloat16)
    # raw gates with A_log = 0, dt_bias = 0: g = -softplus(a); KDA a = 0.5 N(0,1) per channel
    gate = torch.randn(tot, H, K, device=dev, generator=g) * .5 if kda else torch.randn(tot, H, device=dev, generator=g)
    beta = torch.randn(tot, H, device=dev, generator=g)
    a_log = torch.zeros(H, device=dev)
    dt_bias = torch.zeros(H * K if kda else H, device=dev)
    cu = torch.arange(0, tot + 1, T, dtype=torch.int32)  # sequence offsets known on the host
    init = torch.arange(1, B + 1, device=dev)
    pool.encode(torch.randn(B, H, K, V, device=dev, generator=g) * .05, init)
    # prefix slots at evenly spaced chunk boundaries, the last at the sequence end
    pos = [((T * (c + 1)) // NC + 63) // 64 * 64 for c in range(NC)]
    pos[-1] = T
    ck = torch.tensor(pos, dtype=torch.int32).repeat(B, 1)  # on the host, as the scheduler holds them
    ck_slots = torch.arange(B + 1, B + 1 + B * NC).reshape(B, NC)

    def step(events=None):
        return pool.extend(q, k, v, gate, beta, init, cu, checkpoints=ck, checkpoint_slots=ck_slots,
                           init_slots=init, normalize=True, scale=K ** -.5, a_log=a_log, dt_bias=dt_bias,
                           events=events)

    # the recurrence kernel timed in every step on the launching stream: a
    # ring of event pairs, one per timed step, which the timed region's steps
    # (the last ones launched) fill completely
    ring = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(a.steps)]
    for e0, e1 in ring:
        e0.record()
        e1.record()
    turn = [0]

    def timed_step():
        step(ring[turn[0] % len(ring)])
        turn[0] += 1

    step()
    torch.cuda.synchronize()
    ms_step, wall = timed_steps(torch, step, timed_step, 1, a.steps, a.warmup, a.warm_seconds)
    kernel_ms = sum(e0.elapsed_time(e1) for e0, e1 in ring) / len(ring) if ring else ms_step
    gate_bytes = tot * H * (K if kda else 1) * 4 + tot * H * 4
    hbm = (2 * tot * HK * K * 2 + tot * H * V * 2 + tot * H * V * 2 + gate_bytes + B * pool.page_bytes
           + B * NC * pool.page_bytes)
    chunk = 32 if kda else 64
    workload = (f"{a.arch.upper()} prefill STEPQuant@6, B={B}, T={T}, H={H}, HK={HK}, dk=dv={K}, "
                + f"chunk {chunk}" + (" (per-channel decay)" if kda else "")
                + f", bf16 q/k/v, raw gates, {NC} prefix slots per request")
    n_chunks = B * H * ((T + chunk - 1) // chunk)
    flops = prefill_flops(n_chunks, C=chunk)
    tflops = flops / (kernel_ms * 1e-3) / 1e12
    roof = dict(bound="mfma", achieved=round(tflops, 2), peak=PEAK_BF16_TFLOPS, unit="TFLOP/s",
                frac=round(tflops / PEAK_BF16_TFLOPS, 4), traffic=None,
                kernel="kc::kda_chunk_kernel" if kda else "pf::prefill_kernel",
                kernel_ms=round(kernel_ms, 6), step_frac=round(flops / (ms_step * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                algorithmic_flops_per_step=flops,
                hbm_fraction=round(hbm / (ms_step * 1e-3) / 1e9 / PEAK_GBS, 4),
                algorithmic_bytes_per_step=hbm)
    line = dict(metric=f"prefill tokens/sec ({a.arch.upper()} prefill into prefix slots)",
                value=round(tot / (ms_step * 1e-3), 1), unit="tokens/s", n_gpus=1, steps=a.steps,
                warmup=a.warmup, ms_per_step=round(ms_step, 6), higher_is_better=True, scaling="weak",
                vs_baseline=None, dtype="bf16", data="synthetic",
                config=dict(workload=workload, global_batch=B, seq_len=T, wall_s=round(wall, 3),
                            warm_seconds=a.warm_seconds),
                roofline=roof, cpu_baseline=None)
    print(json.dumps(line), flush=True)


def main():
    a = parse()
    if a.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {a.gpus} is not supported (the path shards by heads "
              "with no exchange between GPUs)", file=sys.stderr)
        sys.exit(2)
    import torch
    if a.calibrate_copy:
        n = a.calibrate_copy << 20
        src = torch.randint(0, 255, (n,), dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps(dict(calibrate_copy_bytes=n, launches=5)), flush=True)
        return
    if a.workload == "prefill":
        return bench_prefill(a, torch)
    from stepquant_amd.kernels.pool import PackedStatePool
    from stepquant_amd.quantization import QuantizationPlan

    dev = torch.device("cuda:0")
    B, H, HK, K, V = a.batch, a.heads, a.key_heads, 128, 128
    bits, impact = make_plan(torch, a.arch, H, K, a.nominal)
    # The foreground runs on a stream of its own, created right before the
    # writer's: a CU-masked stream is a blocking stream (the legacy default
    # stream would wait for it), and streams take the hardware queues in
    # creation order, so consecutive streams can run side by side.
    foreground = torch.cuda.Stream()
    torch.cuda.set_stream(foreground)
    stream = None
    if a.async_writeback:
        if a.writer_cus >= 0:
            from stepquant_amd.kernels.resources import writeback_resources
            stream = writeback_resources(dev, a.writer_cus).stream
        else:
            stream = torch.cuda.Stream()
    if a.state_format != "stepquant":
        from stepquant_amd.formats import FormatPlan, get_format
        from stepquant_amd.kernels.format_pool import FormatStatePool
        spec = get_format(a.state_format)
        bits = torch.full((H, K), spec.bits, dtype=torch.long)
        impact = torch.ones(H, K)
        fplan = FormatPlan(a.arch, bits.to(dev), impact.to(dev))

        def make_pool():
            return FormatStatePool(fplan, a.slot_sets * B + 1, V, spec)
        stream = None
        a.cpu_sample = 0  # the CPU port restates the STEPQuant path only
    else:
        plan = QuantizationPlan(a.arch, bits.to(dev), impact.to(dev))

        def make_pool():
            return PackedStatePool(plan, a.slot_sets * B + 1, V, writeback_stream=stream)
    if a.slot_sets < 1:
        raise SystemExit("--slot-sets must be positive")
    pools = [make_pool() for _ in range(a.layers)]
    pool = pools[0]
    g = torch.Generator(device=dev).manual_seed(0)
    slot_sets = [torch.arange(1 + r * B, 1 + (r + 1) * B, device=dev, dtype=torch.int32) for r in range(a.slot_sets)]
    for layer in pools:
        for slots in slot_sets:
            if a.nominal == 4:
                # key-row and value-column scales log-normal(0, 0.5)
                r = torch.exp(torch.randn(B, H, K, 1, device=dev, generator=g) * .5)
                c = torch.exp(torch.randn(B, H, 1, V, device=dev, generator=g) * .5)
                layer.encode(r * torch.randn(B, H, K, V, device=dev, generator=g) * c, slots)
                del r, c
            else:
                layer.encode(torch.randn(B, H, K, V, device=dev, generator=g) * .05, slots)
    mixed = torch.randn(B, 2 * HK * K + H * V, device=dev, generator=g).to(torch.bfloat16)
    q, k, v = mixed.split([HK * K, HK * K, H * V], -1)
    # raw gates with A_log = 0, dt_bias = 0: g = -softplus(a); KDA a = 0.5 N(0,1) per channel
    gate = torch.randn(B, H, K, device=dev, generator=g) * .5 if a.arch == "kda" else \
        torch.randn(B, H, device=dev, generator=g)
    beta = torch.randn(B, H, device=dev, generator=g)
    a_log = torch.zeros(H, device=dev)
    dt_bias = torch.zeros(H * K if a.arch == "kda" else H, device=dev)

    from stepquant_amd.kernels.writeback import attention_window, defer_writeback

    gemm = None
    if a.foreground_gflop > 0:
        d = 4096
        n = max(256, int(round(a.foreground_gflop * 1e9 / (2 * B * d) / 256)) * 256)
        x_fg = torch.randn(B, d, device=dev, generator=g).to(torch.bfloat16)
        w_fg = (torch.randn(d, n, device=dev, generator=g) * d ** -.5).to(torch.bfloat16)
        y_fg = torch.empty(B, n, device=dev, dtype=torch.bfloat16)
        gemm = (x_fg, w_fg, y_fg, 2.0 * B * d * n)

    def layers(slots):
        outs = []
        for layer in pools:
            attention_window()
            if gemm is not None:
                torch.matmul(gemm[0], gemm[1], out=gemm[2])
            outs.append(layer.step(q, k, v, gate, beta, slots, normalize=True, scale=K ** -.5, a_log=a_log,
                                   dt_bias=dt_bias))
        return outs

    turn = [0]

    def step(slots=None):
        if slots is None:  # eager steps take the slot sets in turn
            slots = slot_sets[turn[0] % len(slot_sets)]
            turn[0] += 1
        if stream is not None and torch.cuda.is_current_stream_capturing():
            # writers forked at attention windows, joined when the step ends
            with defer_writeback(pools, attention_windows=True, joined=True):
                outs = layers(slots)
        else:
            outs = layers(slots)
        for layer in pools:
            layer.wait()
        return outs

    for _ in range(3):
        step()
    torch.cuda.synchronize()
    if a.no_graph:
        one, block, per_block = step, step, 1
    else:
        per_block = a.graph_steps or max(d for d in range(1, 17) if a.steps % d == 0)
        if a.steps % per_block:
            raise SystemExit(f"--graph-steps {per_block} must divide --steps {a.steps}")
        # a launch of the multi-step graph takes the slot sets in turn; a
        # single-step graph per set, replayed in turn, for the warm-up steps
        singles = [torch.cuda.CUDAGraph() for _ in slot_sets]
        for graph, slots in zip(singles, slot_sets):
            with torch.cuda.graph(graph, pool=singles[0].pool() if graph is not singles[0] else None):
                step(slots)
        multi = torch.cuda.CUDAGraph()
        with torch.cuda.graph(multi, pool=singles[0].pool()):
            for i in range(per_block):
                step(slot_sets[i % len(slot_sets)])

        def one():
            singles[turn[0] % len(singles)].replay()
            turn[0] += 1
        block = multi.replay
    ms_step, wall = timed_steps(torch, one, block, per_block, a.steps, a.warmup, a.warm_seconds)
    page = pool.page_bytes
    alg_bytes = 2 * B * page * a.layers
    achieved = alg_bytes / (ms_step * 1e-3) / 1e9
    updates = B * H * a.layers / (ms_step * 1e-3)
    # measured HBM bytes per launch apply only to the workload they were taken on
    key = f"{a.arch}-{a.nominal}-b{B}-h{H}-hk{HK}-{'async' if stream is not None else 'fused'}"
    if a.layers != 1:
        key += f"-l{a.layers}"
    if a.state_format != "stepquant":
        key = f"{a.state_format}-{a.arch}-b{B}-h{H}-hk{HK}"
    key += f"-sets{a.slot_sets}"
    if gemm is not None:
        key += f"-fg{a.foreground_gflop:g}"
    traffic = None
    if a.traffic and os.path.exists(a.traffic):
        meas = json.load(open(a.traffic))
        if meas.get("workload_key") == key:
            traffic = meas.get("bytes_per_launch")
    roof = dict(bound="hbm", achieved=round(achieved, 1), peak=PEAK_GBS, unit="GB/s",
                frac=round(achieved / PEAK_GBS, 4), traffic=traffic,
                kernel=("readout + writeback kernels" if stream is not None
                        else "format_kernel (fused step)" if a.state_format != "stepquant"
                        else f"{a.arch}128_kernel (fused read+update+readout+requant+store)"),
                algorithmic_bytes_per_launch=alg_bytes)
    cpu = None
    if a.cpu_sample != 0:
        sample = a.cpu_sample if a.cpu_sample > 0 else B
        cpu = cpu_baseline(bits, impact, a.arch, B, H, HK, K, V, sample, a.cpu_steps, a.cpu_threads)
    line = dict(metric=METRIC, value=round(updates, 1), unit="state-head updates/s", n_gpus=1, steps=a.steps,
                warmup=a.warmup, ms_per_step=round(ms_step, 6), higher_is_better=True, scaling="weak",
                vs_baseline=None, dtype="f32", data="synthetic",
                config=dict(workload=(f"{a.arch.upper()} decode STEPQuant@{a.nominal}" if a.state_format == "stepquant"
                                      else f"{a.arch.upper()} decode {a.state_format} pages")
                                     + (", one layer" if a.layers == 1 else f", {a.layers} layers")
                                     + f", B={B}, H={H}, "
                                     f"HK={HK}, dk=dv={K}, bf16 q/k/v, raw gates, "
                                     + (f"{per_block} steps per graph launch" if not a.no_graph else "eager steps")
                                     + (", async writeback" if stream is not None else ", fused writeback")
                                     + f", steps rotate over {a.slot_sets} disjoint sets of B slots "
                                       f"({a.slot_sets * B * page * a.layers / 1e6:.0f} MB of pages)"
                                     + ("" if gemm is None else
                                        f", a {gemm[3] / 1e9:.1f} GFLOP bf16 matmul per layer as stand-in "
                                        f"foreground work (inside the timed step)")
                                     + ("" if stream is None or a.writer_cus < 0 else
                                        f", writers on a stream over {a.writer_cus or 'all'} CUs"),
                            page_bytes=page, global_batch=B, wall_s=round(wall, 3),
                            warm_seconds=a.warm_seconds),
                roofline=roof, cpu_baseline=cpu)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
