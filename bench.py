"""Benchmark of the sparse-KV decode read path on one MI355X.

Workload (HiSparse Top-K decode read at one GPU's shard): 128 requests x
65,536-token context, 60 layers, 2 KV heads x head_dim 128 bf16 (512 B per K
or V row), Top-K = 2048 per (request, layer) with 80 % of the indices drawn
from the last 4096 tokens and 20 % uniform over the rest, hot capacity 4096
slots per request holding the 4096 most recent tokens (a seeded permutation
of the request's slots). The KV pool is a VMM Backing of 2 MiB chunks.

One step = resident lookup + miss compaction over all 60 layers (one launch)
followed by the Top-K K/V gather of all 60 layers (one launch) into a dense
[128, 60, 2, 2048, 256] bf16 output. `value` is the gather's algorithmic
bytes per step (512 B written per row, plus 512 B read per resident row, plus
the 4 B slot) divided by the measured step time (lookup included).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--capacity C]
"""

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for entry in (str(ROOT / "elastic-kv-vmm_amd"), str(ROOT)):
    if entry not in sys.path:
        sys.path.insert(0, entry)

METRIC = "sparse KV gather GB/s (% of HBM peak) + Top-K lookups/s at K=2048, 1 GPU"
HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = ROOT / "profiles" / "gather_kv_hisparse_decode.md"


def log(message):
    print(f"[bench] {message}", file=sys.stderr, flush=True)


def parse_args():
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--requests", type=int, default=128)
    parser.add_argument("--context", type=int, default=65536)
    parser.add_argument("--layers", type=int, default=60)
    parser.add_argument("--topk", type=int, default=2048)
    parser.add_argument("--capacity", type=int, default=4096)
    parser.add_argument("--recent", type=int, default=4096, help="recency window of the 80 %% share")
    parser.add_argument("--seed", type=int, default=2024)
    parser.add_argument("--cpu-seconds", type=float, default=12.0, help="bound of the CPU baseline sample")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    return parser.parse_args()


def make_inputs(torch, args, device):
    """Seeded synthetic Top-K indices and hot-slot tables, generated on the device."""
    L, R, T, K, C, W = args.layers, args.requests, args.context, args.topk, args.capacity, args.recent
    gen = torch.Generator(device=device).manual_seed(args.seed)
    recent_count = (K * 4) // 5                     # 1638 of 2048
    uniform_count = K - recent_count                # 410 of 2048
    recent = torch.rand((L, R, W), generator=gen, device=device).argsort(-1)[..., :recent_count]
    recent = (recent + (T - W)).to(torch.int32)
    uniform = torch.rand((L, R, T - W), generator=gen, device=device).topk(uniform_count, dim=-1).indices
    topk = torch.cat([recent, uniform.to(torch.int32)], dim=-1)
    del recent, uniform
    order = torch.rand((L, R, K), generator=gen, device=device).argsort(-1)
    topk = torch.gather(topk, -1, order).contiguous()
    del order
    # Hot set: the C most recent tokens of every (layer, request), mapped to a
    # seeded permutation of the request's slots r*C+1 .. r*C+C (0 = not resident).
    table = torch.zeros((L, R, T), dtype=torch.int32, device=device)
    hot = min(C, T)
    perm = torch.rand((L, R, hot), generator=gen, device=device).argsort(-1).to(torch.int32)
    base = (torch.arange(R, device=device, dtype=torch.int32) * C + 1).view(1, R, 1)
    table[:, :, T - hot:] = perm + base
    del perm
    rows = torch.arange(R, device=device, dtype=torch.int64)
    lengths = torch.full((R,), T, device=device, dtype=torch.int32)
    return topk, table, rows, lengths


def time_copy_ceiling(torch, device, nbytes=8 << 30, reps=10):
    """Device-to-device copy bandwidth (read + write bytes / time)."""
    src = torch.empty(nbytes, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    src.fill_(1)
    dst.copy_(src)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        dst.copy_(src)
    stop.record()
    stop.synchronize()
    seconds = start.elapsed_time(stop) / 1000.0 / reps
    del src, dst
    torch.cuda.empty_cache()
    return 2 * nbytes / seconds / 1e9


def read_traffic():
    """HBM bytes per gather launch from the committed rocprof counter summary."""
    if not TRAFFIC_FILE.exists():
        return None
    for line in TRAFFIC_FILE.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def cpu_baseline(torch, args, topk, table, pool_layout, raw, slots, output, budget_s):
    """Time the C oracle (one core) on layer 0 of the same workload; check parity too."""
    import numpy as np

    from oracle.oracle import COracle

    oracle = COracle()
    R, K, T = args.requests, args.topk, args.context
    topk0 = topk[0:1].cpu().numpy()
    table0 = table[0].cpu().numpy()
    rows = np.arange(R)
    lengths = np.full(R, T)
    # Layer 0's K and V planes, copied to host.
    plane = pool_layout.plane_stride
    pool0 = raw.narrow(0, 0, 2 * plane).cpu().numpy()
    init = np.zeros((1, R, K), np.int32)
    want_slots, _, want_counts = oracle.resolve_resident(topk0, table0, None, rows, lengths, rows, 1, init,
                                                         with_misses=True)
    parity_lookup = bool(np.array_equal(slots[0:1].cpu().numpy(), want_slots))
    want_rows = oracle.gather_kv(pool0, 2 * plane, plane, pool_layout.row_bytes, pool_layout.row_bytes,
                                 pool_layout.rows, want_slots, 2)
    got_rows = output[:, 0:1].contiguous().view(torch.uint8).reshape(want_rows.shape).cpu().numpy()
    parity_gather = bool(np.array_equal(got_rows, want_rows))
    del got_rows
    hits = int((want_slots > 0).sum())
    sample_bytes = R * K * 2 * pool_layout.row_bytes + hits * 2 * pool_layout.row_bytes + R * K * 4
    durations = []
    started = time.perf_counter()
    while not durations or (time.perf_counter() - started < budget_s and len(durations) < 1000):
        t0 = time.perf_counter()
        s, _, _ = oracle.resolve_resident(topk0, table0, None, rows, lengths, rows, 1, init, with_misses=True)
        oracle.gather_kv(pool0, 2 * plane, plane, pool_layout.row_bytes, pool_layout.row_bytes,
                         pool_layout.rows, s, 2)
        durations.append(time.perf_counter() - t0)
    median = statistics.median(durations)
    cpu_model = ""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(sample_bytes / median / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"layer 0 of the same workload ({R} requests x {K} lookups + {2 * R * K} gathered "
                   f"{pool_layout.row_bytes} B rows, {sample_bytes / 1e6:.1f} MB algorithmic), C oracle "
                   f"single-threaded, median of {len(durations)} runs ({median * 1e3:.1f} ms each) "
                   f"on {cpu_model or platform.processor()} ({len(os.sched_getaffinity(0))} cores visible)"),
        "parity_layer0": {"lookup": parity_lookup, "gather": parity_gather},
    }


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported by this build "
              "(the path has no cross-GPU step; see the sharding notes)", file=sys.stderr)
        return 2
    import torch

    from adaptive_sparse.kv_pool import PlanePoolLayout
    from adaptive_sparse.resident_lookup import resolve_resident
    from adaptive_sparse.sparse_read import gather_kv
    from elastic_kv.backing import Backing

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    L, R, K, C = args.layers, args.requests, args.topk, args.capacity
    row_bytes = 2 * 128 * 2
    log("measuring device copy ceiling")
    copy_gbs = time_copy_ceiling(torch, device)
    log(f"copy ceiling {copy_gbs:.0f} GB/s")

    layout = PlanePoolLayout(layers=L, kv=2, rows=1 + R * C, row_bytes=row_bytes)
    backing = Backing(layout.capacity_bytes, layout.chunk_bytes, device=0)
    t0 = time.perf_counter()
    backing.ensure(range(backing.chunk_count))
    commit_s = time.perf_counter() - t0
    log(f"committed {backing.chunk_count} chunks ({layout.capacity_bytes / 1e9:.1f} GB) in {commit_s:.2f} s")
    raw = backing.raw
    gen = torch.Generator(device=device).manual_seed(args.seed + 1)
    for plane in range(layout.planes):
        raw.narrow(0, plane * layout.plane_stride, layout.plane_bytes).view(torch.bfloat16).normal_(generator=gen)
    planes = layout.kv_planes(backing.base, 0, owner=backing)
    topk, table, rows, lengths = make_inputs(torch, args, device)
    selected = rows
    slots = torch.empty((L, R, K), dtype=torch.int32, device=device)
    misses = torch.empty_like(slots)
    counts = torch.empty((L, R), dtype=torch.int32, device=device)
    output = torch.empty((R, L, 2, K, 256), dtype=torch.bfloat16, device=device)
    torch.cuda.synchronize()
    log("inputs ready")

    def lookup():
        resolve_resident(topk, table, None, rows, lengths, selected, slots, 1, misses=misses, miss_count=counts)

    def gather():
        gather_kv(planes, slots, output)

    for _ in range(args.warmup):
        lookup()
        gather()
    torch.cuda.synchronize()
    hits = int((slots > 0).sum().item())
    miss_total = int(counts.sum().item())
    lanes = L * R * K
    lookup_bytes = 12 * lanes + 4 * miss_total + 4 * L * R
    gather_bytes = lanes * 2 * row_bytes + hits * 2 * row_bytes + lanes * 4

    events = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    for step in range(args.steps):
        e0, e1, e2 = events[step]
        e0.record()
        lookup()
        e1.record()
        gather()
        e2.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    lookup_ms = [events[i][0].elapsed_time(events[i][1]) for i in range(args.steps)]
    gather_ms = [events[i][1].elapsed_time(events[i][2]) for i in range(args.steps)]
    step_ms = wall * 1e3 / args.steps
    gather_avg_ms = statistics.mean(gather_ms)
    lookup_avg_ms = statistics.mean(lookup_ms)
    value = gather_bytes / (step_ms / 1e3) / 1e9
    achieved = gather_bytes / (gather_avg_ms / 1e3) / 1e9
    log(f"step {step_ms:.3f} ms, gather {gather_avg_ms:.3f} ms ({achieved:.0f} GB/s), "
        f"lookup {lookup_avg_ms * 1e3:.1f} us")

    baseline = None
    if not args.no_cpu_baseline:
        log("CPU baseline (C oracle, one core, layer 0) + layer-0 parity")
        baseline = cpu_baseline(torch, args, topk, table, layout, raw, slots, output, args.cpu_seconds)
        log(f"cpu baseline {baseline['value']} GB/s, parity {baseline['parity_layer0']}")

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded; bf16 ~N(0,1) KV, Top-K 80% last-4096 / 20% uniform)",
        "config": {"workload": "hisparse-topk-decode-read", "requests": R, "context": args.context,
                   "layers": L, "kv_heads": 2, "head_dim": 128, "topk": K, "hot_capacity": C,
                   "pool_bytes": layout.capacity_bytes, "chunk_bytes": layout.chunk_bytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": read_traffic(),
                     "kernel": "copy_small_rows<KvGather,16> (ekv_gather_kv)",
                     "algorithmic_bytes_per_launch": gather_bytes, "avg_launch_ms": round(gather_avg_ms, 4)},
        "cpu_baseline": baseline,
        "lookups_per_s": round(lanes / (lookup_avg_ms / 1e3), 1),
        "lookup_us_per_step": round(lookup_avg_ms * 1e3, 2),
        "lookup_gbs": round(lookup_bytes / (lookup_avg_ms / 1e3) / 1e9, 1),
        "hit_rate": round(hits / lanes, 4),
        "copy_ceiling_gbs": round(copy_gbs, 1),
        "pool_commit_s": round(commit_s, 3),
    }
    print(json.dumps(result), flush=True)
    del raw, output
    torch.cuda.synchronize()
    backing.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
