"""Benchmarks of the sparse-KV residency path on one MI355X.

Default workload (--workload decode-read), HiSparse Top-K decode read at one
GPU's shard: 128 requests x 65,536-token context, 60 layers, 2 KV heads x
head_dim 128 bf16 (512 B per K or V row), Top-K = 2048 per (request, layer)
with 80 % of the indices from the last 4096 tokens and 20 % uniform over the
rest, hot capacity 4096 slots per request holding the 4096 most recent tokens
(a seeded permutation of the request's slots). The KV pool is a VMM Backing of
2 MiB chunks. One step = resident lookup + miss compaction over all 60 layers
(one launch; int16 local-slot table behind a line summary, one bit per 64
positions) + the Top-K K/V gather of all 60 layers (one launch) into a dense
[128, 60, 2, 2048, 256] bf16 output. `value` = the gather's algorithmic bytes
per step (512 B written per row, + 512 B read per resident row, + 4 B slot)
divided by the measured step time, lookup included.

The default line also carries, as extra keys, the streaming ceilings of this
box (own read / write / copy kernels), the lookup variants timed in
alternating arms, configs 1, 2 and 4 (topk-gather, block-gather, migration
below), each with its own roofline, parity flags and CPU baseline, configs 4
and 5 also with the VMM spare pool (--spare-chunks: reclaimed chunks' memory
kept for the next commits), the decode read at hot capacity 8192 (81 % hits,
the lookup's longest default case), and the reference's two microbenchmarks
(lookup-micro, virtual-addressing).
The CPU baseline is the reference's torch CPU path restated
(oracle/torch_path.py: adaptive_sparse/request_residency.py:819-825, nonzero,
index_select) at all visible host threads and at one thread.

Other workloads (same JSON contract):
  topk-gather   8 requests x 8192 context, 28 layers x 8 heads x 128, two-level
                lookup (req_to_token -> logical -> slot), Top-K 2048 shared by
                all layers, hot capacity 4096 (~50 % misses)
  block-gather  64 requests x 256 blocks of 16 tokens, 36 layers x 8 heads x
                128, block tables from a permutation of a 20k-block pool
  migration     per tick: 512 scattered 2.25 MiB blocks packed, copied to
                pinned host and back, unpacked into freshly mapped chunks
  composite     elastic decode step: 128 requests with contexts uniform in
                [4096, 32768], 60 layers x 2 heads x 128, Top-K 2048 with the
                decode-read locality mix, hot capacity 4096 (LRU); per step
                5 % of pool chunks are unmapped and remapped (their hot slots
                invalidated), then lookup + compaction, LRU swap-in, promote
                of misses from pinned host, gather
  hisparse-swap SGLang-convention swap-in (load_blocks_to_device_buffer_mha)
                of one layer: 128 requests x 65,536-token context, 4096 hot
                slots each, 16 Top-K blocks of 128 tokens (newest block, 12
                recent, 3 older), 512 B K and V rows promoted from pinned host
  lookup-micro  the reference's resident-lookup microbenchmark
                (tests/bench_resident_lookup.py): batch 1/2/4, 8192-token rows,
                16 Top-K blocks of 128 tokens, two-level int64 lookup, per-call
                p50/p95 with the host launch included (time-like: lower is
                better; vs_baseline against the reference's A100 Triton p50)
  virtual-addressing  the reference's gather microbenchmark
                (scripts/bench_virtual_addressing.py): gather_rows over a VMM
                arena of 4 x 65,536 rows of 256 bf16, 2048 positions per
                request from three support sets, direct and software-table
                addressing; host-launched p50 per call and HIP-graph GB/s
  residency-summary  rebuild of the residency summary (ekv_residency_bits) of
                the decode-read int16 table (60 x 128 x 65,536) at shifts 6
                and 0, checked against a torch restatement

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
"""

import argparse
import dataclasses
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
PCIE_PEAK_GBS = 64.0   # PCIe Gen5 x16, per direction, theoretical
PROFILES = ROOT / "profiles"


def log(message):
    print(f"[bench] {message}", file=sys.stderr, flush=True)


def parse_args():
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--workload", default="decode-read",
                        choices=["decode-read", "topk-gather", "block-gather", "migration", "composite",
                                 "hisparse-swap", "lookup-micro", "virtual-addressing",
                                 "residency-summary"])
    parser.add_argument("--remap-fraction", type=float, default=0.05,
                        help="share of pool chunks unmapped and remapped per composite step")
    parser.add_argument("--capacity", type=int, default=4096, help="hot slots per request (decode-read)")
    parser.add_argument("--spare-chunks", type=int, default=0,
                        help="VMM spare pool of the migration and composite pools (0: release at once)")
    parser.add_argument("--serial-remap", action="store_true",
                        help="composite: remap with the GPU idle before the step's kernels (no overlap)")
    parser.add_argument("--remap-groups", type=int, default=2,
                        help="composite: remap the chunks in this many groups, each followed by the promote of "
                             "the items whose hot buffers it completes (1: promote after the whole remap)")
    parser.add_argument("--seed", type=int, default=2024)
    parser.add_argument("--cpu-seconds", type=float, default=8.0,
                        help="bound of each CPU baseline sample (per thread count)")
    parser.add_argument("--extras-cpu-seconds", type=float, default=3.0,
                        help="bound of each CPU baseline sample of the extra configs")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-copy-ceiling", action="store_true")
    parser.add_argument("--profile-ranges", action="store_true",
                        help="keep EKV_PROFILE_RANGES=1 (ekv/* profiler and roctx ranges); timed runs drop it")
    parser.add_argument("--no-extras", action="store_true",
                        help="decode-read only: skip configs 1, 2 and 4 in the default line")
    return parser.parse_args()


# ------------------------------------------------------------------ shared helpers


def cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def time_cpu(fn, budget_s):
    """Median wall time of fn() over repeated runs within the budget."""
    durations = []
    started = time.perf_counter()
    while not durations or (time.perf_counter() - started < budget_s and len(durations) < 1000):
        t0 = time.perf_counter()
        fn()
        durations.append(time.perf_counter() - t0)
    return statistics.median(durations), len(durations)


def cpu_rates(torch, fn, nbytes, budget_s):
    """GB/s of fn() (moving `nbytes` algorithmic bytes) at every visible host thread and at one thread."""
    threads = len(os.sched_getaffinity(0))
    before = torch.get_num_threads()
    result = {}
    try:
        for label, count in (("all", threads), ("one", 1)):
            torch.set_num_threads(count)
            median, runs = time_cpu(fn, budget_s)
            result[label] = {"gbs": round(nbytes / median / 1e9, 3), "threads": count, "runs": runs,
                             "ms": round(median * 1e3, 2)}
    finally:
        torch.set_num_threads(before)
    return result


def cpu_budget(args, workload):
    """Seconds per CPU-baseline sample: the full budget for the workload asked for, less for extras."""
    return args.cpu_seconds if args.workload == workload else args.extras_cpu_seconds


def cpu_baseline_entry(rates, sample, parity):
    """The cpu_baseline object: the all-thread rate as `value`, the one-thread rate beside it."""
    return {"value": rates["all"]["gbs"], "unit": "GB/s", "cores": rates["all"]["threads"], "kind": "port",
            "value_1_thread": rates["one"]["gbs"],
            "sample": (f"{sample}; torch CPU restatement of the reference path (oracle/torch_path.py), median of "
                       f"{rates['all']['runs']} runs at {rates['all']['threads']} threads ({rates['all']['ms']} ms) "
                       f"and {rates['one']['runs']} at 1 thread ({rates['one']['ms']} ms), {cpu_model()}"),
            "parity": parity}


PROBE_NT_LOAD, PROBE_HALF_TILE = 0x10, 0x20      # include/ekv_kernels.h: EKV_PROBE_NT_LOAD, EKV_PROBE_HALF_TILE


def stream_ceilings(torch, device, nbytes=8 << 30, reps=10):
    """GB/s of this box's own streaming kernels (ekv_stream_probe): read-only, write-only and copy, each in its
    variants (32 or 16 KiB tiles; temporal or non-temporal loads) without a workgroup cap and at 2, 3 and 4
    workgroups per CU; the best of each mode is its ceiling. Plus torch's device copy."""
    from elastic_kv import _native

    lib = _native.kernel_library()
    src = torch.empty(nbytes, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    src.fill_(1)
    result = {}
    for name, mode, moved in (("read", 0, nbytes), ("write", 1, nbytes), ("copy", 2, 2 * nbytes)):
        loads = (0,) if name == "write" else (0, PROBE_NT_LOAD)
        per = {}
        for tile in (0, PROBE_HALF_TILE):
            for load in loads:
                label = ("16k" if tile else "32k") + ("_nt_load" if load else "")
                for per_cu in (0, 2, 3, 4):
                    def probe(flags=mode | tile | load, per_cu=per_cu):
                        status = lib.ekv_stream_probe(flags, src.data_ptr(), dst.data_ptr(), nbytes, per_cu,
                                                      _native.stream_handle(device))
                        _native.check(lib, status, "stream probe")

                    ms = back_to_back_ms(torch, probe, reps)
                    cap = "max_per_cu" if per_cu == 0 else f"{per_cu}_per_cu"
                    per[f"{label}_{cap}"] = round(moved / (ms / 1e3) / 1e9, 1)
        best = max(per, key=per.get)
        result[name] = {"best_gbs": per[best], "best_variant": best, **per}
    torch.cuda.synchronize()
    ms = back_to_back_ms(torch, lambda: dst.copy_(src), reps)
    result["torch_copy_gbs"] = round(2 * nbytes / (ms / 1e3) / 1e9, 1)
    del src, dst
    torch.cuda.empty_cache()
    return result


def read_traffic(name):
    """HBM bytes per launch from a committed rocprof counter summary, if any."""
    path = PROFILES / name
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def timed_steps(torch, steps, phases):
    """Run `steps` steps of the given (name, fn) phases; per-phase event times (ms) and wall ms/step."""
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(len(phases) + 1)] for _ in range(steps)]
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    for step in range(steps):
        marks = events[step]
        marks[0].record()
        for i, (_, fn) in enumerate(phases):
            fn()
            marks[i + 1].record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - wall0) * 1e3 / steps
    samples = {name: [events[s][i].elapsed_time(events[s][i + 1]) for s in range(steps)]
               for i, (name, _) in enumerate(phases)}
    per_phase = {name: statistics.mean(values) for name, values in samples.items()}
    LAST_SAMPLES.clear()
    LAST_SAMPLES.update(samples)
    return wall_ms, per_phase


LAST_SAMPLES = {}   # per-phase event times (ms) of the latest timed_steps call


def spread(values_ms, scale=1.0, digits=4):
    """Median and 95th percentile of event times (scaled, e.g. 1e3 for us)."""
    ordered = sorted(values_ms)
    p95 = ordered[min(len(ordered) - 1, int(round(0.95 * (len(ordered) - 1))))]
    return {"median": round(statistics.median(ordered) * scale, digits), "p95": round(p95 * scale, digits)}


def back_to_back_ms(torch, fn, reps=20, lead=None):
    """Mean event time (ms) of `reps` consecutive calls of fn on the current stream.

    With `lead`, a longer kernel is queued first, so the host has queued the
    timed calls before the GPU reaches them (no host launch gaps inside).
    """
    fn()
    torch.cuda.synchronize()
    if lead is not None:
        lead()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        fn()
    stop.record()
    stop.synchronize()
    return start.elapsed_time(stop) / reps


def in_step_events(torch, steps, phases, lead):
    """Per-phase event times (ms) of `steps` steps queued behind `lead`, so no host launch gap is timed."""
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(len(phases) + 1)] for _ in range(steps)]
    torch.cuda.synchronize()
    lead()
    for marks in events:
        marks[0].record()
        for i, (_, fn) in enumerate(phases):
            fn()
            marks[i + 1].record()
    torch.cuda.synchronize()
    return {name: [marks[i].elapsed_time(marks[i + 1]) for marks in events] for i, (name, _) in enumerate(phases)}


def alternating_arms(torch, arms, rounds=6, reps=10, lead=None):
    """Per-launch event times (ms) of each (name, fn) arm: every round times each arm `reps` times back to
    back, starting from a different arm each round (scripts/bench_virtual_addressing.py:93-103 alternates
    its arms the same way)."""
    samples = {name: [] for name, _ in arms}
    for r in range(rounds):
        for name, fn in arms[r % len(arms):] + arms[:r % len(arms)]:
            samples[name].append(back_to_back_ms(torch, fn, reps, lead))
    return samples


def graph_replay_ms(torch, fn, reps=10):
    """Mean event time (ms) of one replay of a HIP graph capturing fn."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    ms = back_to_back_ms(torch, graph.replay, reps)
    del graph
    return ms


def roofline(achieved_gbs, kernel, algorithmic_bytes, avg_ms, traffic):
    return {"bound": "hbm", "achieved": round(achieved_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved_gbs / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": kernel,
            "algorithmic_bytes_per_launch": algorithmic_bytes, "avg_launch_ms": round(avg_ms, 4)}


def envelope(args, value, step_ms, config, roof, baseline, extra, unit="GB/s", metric=METRIC):
    result = {
        "metric": metric, "value": round(value, 2), "unit": unit, "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(step_ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded inputs; bf16 ~N(0,1) or random-byte KV payload)",
        "config": config, "roofline": roof, "cpu_baseline": baseline,
    }
    result.update(extra)
    return result


def make_pool(torch, layout, device, seed):
    """A fully committed VMM pool of the layout, filled with bf16 ~N(0,1)."""
    from elastic_kv.backing import Backing

    backing = Backing(layout.capacity_bytes, layout.chunk_bytes, device=device.index or 0)
    t0 = time.perf_counter()
    backing.ensure(range(backing.chunk_count))
    commit_s = time.perf_counter() - t0
    log(f"committed {backing.chunk_count} chunks ({layout.capacity_bytes / 1e9:.1f} GB) in {commit_s:.2f} s")
    raw = backing.raw
    gen = torch.Generator(device=device).manual_seed(seed)
    for plane in range(layout.planes):
        raw.narrow(0, plane * layout.plane_stride, layout.plane_bytes).view(torch.bfloat16).normal_(generator=gen)
    return backing, raw, commit_s


# ------------------------------------------------------------------ decode-read (HiSparse Top-K decode)


def decode_inputs(torch, device, L, R, T, K, C, W, seed):
    """Seeded Top-K indices (80 % recent / 20 % uniform) and hot-slot tables, on the device."""
    gen = torch.Generator(device=device).manual_seed(seed)
    recent_count = (K * 4) // 5
    uniform_count = K - recent_count
    if not (recent_count <= W <= T and uniform_count <= T - W and C <= T):
        # The index gathers below would read past their sources.
        raise ValueError(f"decode inputs need {recent_count} <= W <= T, {uniform_count} <= T - W and C <= T")
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


def run_decode_read(torch, args, device):
    import numpy as np

    from adaptive_sparse.kv_pool import PlanePoolLayout
    from adaptive_sparse.resident_lookup import build_residency_bits, resolve_resident
    from adaptive_sparse.sparse_read import gather_kv

    L, R, T, K, C, W = 60, 128, 65536, 2048, args.capacity, 4096
    row_bytes = 2 * 128 * 2
    layout = PlanePoolLayout(layers=L, kv=2, rows=1 + R * C, row_bytes=row_bytes)
    backing, raw, commit_s = make_pool(torch, layout, device, args.seed + 1)
    planes = layout.kv_planes(backing.base, 0, owner=backing)
    topk, table, rows, lengths = decode_inputs(torch, device, L, R, T, K, C, W, args.seed)
    slots = torch.empty((L, R, K), dtype=torch.int32, device=device)
    misses = torch.empty_like(slots)
    counts = torch.empty((L, R), dtype=torch.int32, device=device)
    output = torch.empty((R, L, 2, K, 256), dtype=torch.bfloat16, device=device)
    bits = build_residency_bits(table)          # maintained with the table; built once here
    # The same residency as an int16 table of local slots (request r's hot slots start at r * C + 1),
    # which holds hot buffers of up to 32767 slots; larger ones keep the int32 form.
    slot_base = torch.arange(R, device=device, dtype=torch.int64) * C + 1
    local_form = C < 1 << 15
    if local_form:
        table16 = torch.where(table > 0, table - slot_base.view(1, R, 1).to(torch.int32) + 1, 0).to(torch.int16)
        bits16 = build_residency_bits(table16)
    else:
        table16, bits16, slot_base = table, bits, None
    # The decode default: a line summary (one bit per 64 positions = one 128-byte
    # line of the int16 table) in front of the table instead of the per-position bitmap.
    SHIFT = 6
    lines16 = build_residency_bits(table16, shift=SHIFT)

    def lookup_plain():
        resolve_resident(topk, table, None, rows, lengths, rows, slots, 1, misses=misses, miss_count=counts)

    def lookup_global():
        resolve_resident(topk, table, None, rows, lengths, rows, slots, 1, misses=misses, miss_count=counts,
                         resident_bits=bits)

    def lookup_bitmap():
        resolve_resident(topk, table16, None, rows, lengths, rows, slots, 1, misses=misses, miss_count=counts,
                         resident_bits=bits16, slot_base=slot_base)

    def lookup():
        resolve_resident(topk, table16, None, rows, lengths, rows, slots, 1, misses=misses, miss_count=counts,
                         resident_bits=lines16, bits_shift=SHIFT, slot_base=slot_base)

    def gather():
        gather_kv(planes, slots, output)

    # Every lookup variant must give the same slots, counts and miss lists.
    lane = torch.arange(K, device=device).view(1, 1, K)
    lookup_plain()
    plain = (slots.clone(), counts.clone(), torch.where(lane < counts.unsqueeze(-1), misses, -1))
    same = True
    for variant in (lookup_global, lookup_bitmap, lookup):
        variant()
        same = same and torch.equal(plain[0], slots) and torch.equal(plain[1], counts) and torch.equal(
            plain[2], torch.where(lane < counts.unsqueeze(-1), misses, -1))
    same = bool(same)
    del plain
    for _ in range(args.warmup):
        lookup()
        gather()
    torch.cuda.synchronize()
    hits = int((slots > 0).sum().item())
    miss_total = int(counts.sum().item())
    lanes = L * R * K
    lookup_bytes = 10 * lanes + 4 * miss_total + 4 * L * R   # 4 B index + 2 B table entry + 4 B slot per lookup
    gather_bytes = lanes * 2 * row_bytes + hits * 2 * row_bytes + lanes * 4
    # The timed steps: wall clock, bracketed by synchronizations.
    step_ms, _ = timed_steps(torch, args.steps, [("lookup", lookup), ("gather", gather)])
    # The same steps queued behind one gather (the host runs ahead, so no launch gap is timed):
    # per-kernel event times inside the step, the lookup right after the previous step's gather.
    phase_samples = in_step_events(torch, args.steps, [("lookup", lookup), ("gather", gather)], gather)
    phase = {name: statistics.mean(values) for name, values in phase_samples.items()}
    step_spread = {"gather_ms": spread(phase_samples["gather"]), "lookup_us": spread(phase_samples["lookup"], 1e3, 2)}
    # The lookup variants alone, back to back, in alternating arms.
    arm_samples = alternating_arms(torch, [("line_summary", lookup), ("position_bitmap", lookup_bitmap),
                                           ("int32_table_bitmap", lookup_global), ("int32_table_plain", lookup_plain)],
                                   rounds=6, reps=10, lead=gather)
    arms = {name: {"median_us": round(statistics.median(v) * 1e3, 2), "min_us": round(min(v) * 1e3, 2)}
            for name, v in arm_samples.items()}
    # Reference points of the same engine on the same shapes: sequential slots
    # (every row read, contiguous) and all-miss slots (write-only zero fill).
    seq = (torch.arange(K, device=device, dtype=torch.int32).view(1, 1, K) + 1
           + torch.arange(R, device=device, dtype=torch.int32).view(1, R, 1) * C).expand(L, R, K).contiguous()
    none = torch.zeros_like(slots)
    engine = {}
    for name, probe, nbytes in (("sequential_all_hit", seq, lanes * 2048 + lanes * 4),
                                ("all_miss_write_only", none, lanes * 1024 + lanes * 4)):
        ms = back_to_back_ms(torch, lambda s=probe: gather_kv(planes, s, output), 5)
        engine[name] = round(nbytes / (ms / 1e3) / 1e9, 1)
    del seq, none
    # The 20 back-to-back 60-layer launches replayed from one HIP graph, and one
    # launch per layer (as a decode step interleaved with attention issues them).
    lookup_graph_ms = graph_replay_ms(torch, lambda: [lookup() for _ in range(20)], reps=5) / 20
    per_layer = [(topk[l:l + 1], table16[l:l + 1], lines16[l:l + 1], slots[l:l + 1], misses[l:l + 1],
                  counts[l:l + 1]) for l in range(L)]

    def lookup_by_layer():
        for tk, tb, bt, sl, ms, ct in per_layer:
            resolve_resident(tk, tb, None, rows, lengths, rows, sl, 1, misses=ms, miss_count=ct, resident_bits=bt,
                             bits_shift=SHIFT, slot_base=slot_base)

    per_layer_graph_ms = graph_replay_ms(torch, lookup_by_layer)
    del per_layer
    lookup()
    gather()  # the probes above overwrote the output
    torch.cuda.synchronize()
    achieved = gather_bytes / (phase["gather"] / 1e3) / 1e9
    log(f"step {step_ms:.3f} ms, gather {phase['gather']:.3f} ms ({achieved:.0f} GB/s), lookup "
        f"{phase['lookup'] * 1e3:.1f} us in the step (median {step_spread['lookup_us']['median']} us; "
        f"int16 table + line summary), arms {arms}, {lookup_graph_ms * 1e3:.1f} us back to back from a graph, "
        f"{per_layer_graph_ms * 1e3 / L:.2f} us per one-layer launch in a graph, identical results {same}")

    baseline = None
    if not args.no_cpu_baseline:
        from oracle import torch_path

        # Layer 0 of the step on the host, as the reference's CPU path computes it:
        # req_to_token -> mapping (here the hot-slot table), nonzero, index_select.
        topk0 = topk[0].cpu()
        mapping = table[0].reshape(-1).cpu()
        req_to_token = torch.arange(R * T, dtype=torch.int64).view(R, T)
        rows_c, lengths_c = rows.cpu(), lengths.cpu()
        planes0 = raw.narrow(0, 0, 2 * layout.plane_stride).view(2, layout.plane_stride)
        planes0 = planes0[:, :layout.plane_bytes].reshape(2, layout.rows, row_bytes).cpu()

        def sample():
            s, m = torch_path.lookup(topk0, req_to_token, mapping, rows_c, lengths_c, rows_c, 1)
            return s, m, torch_path.gather(planes0, s.reshape(-1))

        want_slots, want_misses, want_rows = sample()
        got_misses = misses[0].cpu()
        got_counts = counts[0].cpu()
        parity = {"lookup": bool(torch.equal(slots[0].cpu(), want_slots)),
                  "misses": bool(torch.equal(got_counts, torch.bincount(want_misses[:, 0], minlength=R).to(torch.int32))
                                 and all(torch.equal(got_misses[r, :int(got_counts[r])],
                                                     want_misses[want_misses[:, 0] == r, 1].to(torch.int32))
                                         for r in range(R))),
                  "gather": bool(torch.equal(output[:, 0].contiguous().view(torch.uint8).cpu(),
                                             want_rows.view(2, R, K, row_bytes).transpose(0, 1)))}
        del want_rows
        layer_hits = int((want_slots > 0).sum())
        sample_bytes = R * K * 2 * row_bytes + layer_hits * 2 * row_bytes + R * K * 4
        rates = cpu_rates(torch, sample, sample_bytes, args.cpu_seconds)
        baseline = cpu_baseline_entry(
            rates, f"layer 0 of the same step ({R} x {K} lookups, miss list, {2 * R * K} gathered {row_bytes} B "
                   f"rows: {sample_bytes / 1e6:.1f} MB algorithmic); x{L} layers extrapolated: "
                   f"{rates['all']['ms'] * L / 1e3:.2f} s per step at {rates['all']['threads']} threads, "
                   f"{rates['one']['ms'] * L / 1e3:.2f} s at 1", parity)
        baseline["step_ms_extrapolated"] = {"all_threads": round(rates["all"]["ms"] * L, 1),
                                            "one_thread": round(rates["one"]["ms"] * L, 1), "layers": L}
        log(f"cpu baseline {rates}, parity {parity}")

    config = {"workload": "hisparse-topk-decode-read", "requests": R, "context": T, "layers": L, "kv_heads": 2,
              "head_dim": 128, "topk": K, "hot_capacity": C, "pool_bytes": layout.capacity_bytes,
              "chunk_bytes": layout.chunk_bytes}
    # Committed counter summaries exist for hot capacities 4096 and 8192; other capacities move other bytes.
    suffix = {4096: "", 8192: "_capacity8192"}.get(C)
    profiled = suffix is not None
    lookup_traffic = read_traffic(f"resolve_resident_hisparse_decode{suffix}.md") if profiled else None
    extra = {"lookups_per_s": round(lanes / (phase["lookup"] / 1e3), 1),
             "lookup_us_per_step": round(phase["lookup"] * 1e3, 2),
             "lookup_us_per_layer": round(phase["lookup"] * 1e3 / L, 2),
             "lookup_gbs": round(lookup_bytes / (phase["lookup"] / 1e3) / 1e9, 1),
             "lookup_roofline": roofline(lookup_bytes / (phase["lookup"] / 1e3) / 1e9,
                                         "resolve_runs_pipe2_kernel<compact, int16> (ekv_resolve_resident_local: "
                                         "int16 table, line summary), in the step", lookup_bytes, phase["lookup"],
                                         lookup_traffic),
             "lookup_arms_back_to_back": arms,
             "lookup_us_back_to_back_graph": round(lookup_graph_ms * 1e3, 2),
             "lookup_us_per_layer_launch_graph": round(per_layer_graph_ms * 1e3 / L, 2),
             "lookup_table": ("int16 local slots + slot_base, line summary (1 bit per 64 positions)" if local_form
                              else "int32 global slots, line summary (1 bit per 64 positions)"),
             "lookup_variants_identical": same,
             "engine_gbs_same_shapes": engine,
             "event_spread": step_spread,
             "hit_rate": round(hits / lanes, 4), "pool_commit_s": round(commit_s, 3)}
    roof = roofline(achieved, "copy_small_rows<KvGather,16> (ekv_gather_kv)", gather_bytes, phase["gather"],
                    read_traffic(f"gather_kv_hisparse_decode{suffix}.md") if profiled else None)
    result = envelope(args, gather_bytes / (step_ms / 1e3) / 1e9, step_ms, config, roof, baseline, extra)
    del raw, output
    torch.cuda.synchronize()
    backing.close()
    return result


# ------------------------------------------------------------------ topk-gather (two-level lookup + shared Top-K)


def run_topk_gather(torch, args, device):
    import numpy as np

    from adaptive_sparse.kv_pool import PlanePoolLayout
    from adaptive_sparse.resident_lookup import resolve_resident
    from adaptive_sparse.sparse_read import gather_kv

    R, T, L, K, C = 8, 8192, 28, 2048, 4096
    row_bytes = 8 * 128 * 2
    rng = np.random.default_rng(args.seed)
    table = (np.arange(R * T, dtype=np.int64).reshape(R, T) + 1)       # req_to_token: logical ids
    mapping = np.zeros(R * T + 1, dtype=np.int64)                       # logical -> global hot slot
    for r in range(R):
        resident = rng.choice(T, C, replace=False)
        mapping[r * T + resident + 1] = r * C + rng.permutation(C) + 1
    topk = np.stack([rng.choice(T, K, replace=False) for _ in range(R)])[None].astype(np.int32)
    layout = PlanePoolLayout(layers=L, kv=2, rows=1 + R * C, row_bytes=row_bytes)
    backing, raw, commit_s = make_pool(torch, layout, device, args.seed + 1)
    planes = layout.kv_planes(backing.base, 0, owner=backing)
    t = lambda a, dt: torch.tensor(a, dtype=dt, device=device)  # noqa: E731
    topk_d, table_d, map_d = t(topk, torch.int32), t(table, torch.int64), t(mapping, torch.int64)
    rows = torch.arange(R, device=device)
    lengths = torch.full((R,), T, dtype=torch.int32, device=device)
    slots = torch.empty((1, R, K), dtype=torch.int32, device=device)
    misses = torch.empty_like(slots)
    counts = torch.empty((1, R), dtype=torch.int32, device=device)
    output = torch.empty((R, L, 2, K, row_bytes // 2), dtype=torch.bfloat16, device=device)

    def lookup():
        resolve_resident(topk_d, table_d, map_d, rows, lengths, rows, slots, 1, misses=misses, miss_count=counts)

    def gather():
        gather_kv(planes, slots.expand(L, R, K), output)

    for _ in range(args.warmup):
        lookup()
        gather()
    torch.cuda.synchronize()
    hits = int((slots > 0).sum().item())
    lanes = R * K
    gather_bytes = lanes * L * 2 * row_bytes + hits * L * 2 * row_bytes + lanes * L * 4
    step_ms, phase = timed_steps(torch, args.steps, [("lookup", lookup), ("gather", gather)])
    achieved = gather_bytes / (phase["gather"] / 1e3) / 1e9
    log(f"step {step_ms:.3f} ms, gather {phase['gather']:.3f} ms ({achieved:.0f} GB/s), "
        f"lookup {phase['lookup'] * 1e3:.1f} us, hit rate {hits / lanes:.3f}")
    baseline = None
    if not args.no_cpu_baseline:
        from oracle import torch_path

        # The whole step on the host: the reference's two-level torch resolver once,
        # then index_select of the 28 layers' K and V planes.
        host_planes = raw.view(-1)[:L * 2 * layout.plane_stride].view(L, 2, layout.plane_stride)
        host_planes = host_planes[..., :layout.plane_bytes].reshape(L, 2, layout.rows, row_bytes).cpu()
        topk_c, table_c, map_c = torch.tensor(topk[0]), torch.tensor(table), torch.tensor(mapping)
        idx, full = torch.arange(R), torch.full((R,), T)

        def sample():
            s, m = torch_path.lookup(topk_c, table_c, map_c, idx, full, idx, 1)
            return s, m, [torch_path.gather(host_planes[l], s.reshape(-1)) for l in range(L)]

        want_slots, want_misses, want_rows = sample()
        got_counts = counts[0].cpu()
        got = output.view(torch.uint8).cpu()        # [R, L, 2, K, row]
        parity = {"lookup": bool(torch.equal(slots[0].cpu(), want_slots)),
                  "misses": bool(torch.equal(got_counts, torch.bincount(want_misses[:, 0], minlength=R)
                                             .to(torch.int32))),
                  "gather": all(torch.equal(got[:, l], want_rows[l].view(2, R, K, row_bytes).transpose(0, 1))
                                for l in range(L))}
        del want_rows, got
        rates = cpu_rates(torch, sample, gather_bytes, cpu_budget(args, "topk-gather"))
        baseline = cpu_baseline_entry(rates, f"the full step (two-level lookup + {L}-layer gather, "
                                             f"{gather_bytes / 1e9:.2f} GB algorithmic)", parity)
        del host_planes
        log(f"cpu baseline {rates}, parity {parity}")
    config = {"workload": "resident-lookup-topk-gather", "requests": R, "context": T, "layers": L, "kv_heads": 8,
              "head_dim": 128, "topk": K, "hot_capacity": C, "lookup": "two-level (req_to_token -> mapping)"}
    extra = {"lookups_per_s": round(lanes / (phase["lookup"] / 1e3), 1),
             "lookup_us_per_step": round(phase["lookup"] * 1e3, 2), "hit_rate": round(hits / lanes, 4),
             "pool_commit_s": round(commit_s, 3)}
    roof = roofline(achieved, "copy_small_rows<KvGather,16> (ekv_gather_kv)", gather_bytes, phase["gather"],
                    read_traffic("gather_kv_topk_gather.md"))
    result = envelope(args, gather_bytes / (step_ms / 1e3) / 1e9, step_ms, config, roof, baseline, extra)
    del raw, output
    torch.cuda.synchronize()
    backing.close()
    return result


# ------------------------------------------------------------------ block-gather (vLLM-style)


def run_block_gather(torch, args, device):
    import numpy as np

    from adaptive_sparse.kv_pool import PlanePoolLayout
    from adaptive_sparse.sparse_read import gather_kv

    R, NB, L, POOL = 64, 256, 36, 20000
    row_bytes = 16 * 8 * 128 * 2                 # one 16-token block of one plane
    rng = np.random.default_rng(args.seed)
    tables = rng.permutation(POOL)[: R * NB].reshape(R, NB)
    layout = PlanePoolLayout(layers=L, kv=2, rows=POOL, row_bytes=row_bytes)
    backing, raw, commit_s = make_pool(torch, layout, device, args.seed + 1)
    planes = layout.kv_planes(backing.base, 0, owner=backing)
    tables_d = torch.tensor(tables, dtype=torch.int32, device=device)
    output = torch.empty((R, L, 2, NB, row_bytes // 2), dtype=torch.bfloat16, device=device)

    def gather():
        gather_kv(planes, tables_d.unsqueeze(0).expand(L, R, NB), output, zero_below=0)

    for _ in range(args.warmup):
        gather()
    torch.cuda.synchronize()
    units = R * NB * L * 2
    gather_bytes = units * 2 * row_bytes + units * 4
    step_ms, phase = timed_steps(torch, args.steps, [("gather", gather)])
    achieved = gather_bytes / (phase["gather"] / 1e3) / 1e9
    log(f"step {step_ms:.3f} ms, gather {phase['gather']:.3f} ms ({achieved:.0f} GB/s)")
    baseline = None
    if not args.no_cpu_baseline:
        from oracle import torch_path

        planes0 = raw.narrow(0, 0, 2 * layout.plane_stride).view(2, layout.plane_stride)
        planes0 = planes0[:, :layout.plane_bytes].reshape(2, POOL, row_bytes).cpu()
        blocks = torch.tensor(tables, dtype=torch.int32).reshape(-1)

        def sample():
            return torch_path.gather(planes0, blocks, zero_below=0)

        want = sample()
        parity = {"gather": bool(torch.equal(output[:, 0].contiguous().view(torch.uint8).cpu(),
                                             want.view(2, R, NB, row_bytes).transpose(0, 1)))}
        del want
        sample_bytes = R * NB * 2 * (2 * row_bytes + 4)
        rates = cpu_rates(torch, sample, sample_bytes, cpu_budget(args, "block-gather"))
        baseline = cpu_baseline_entry(rates, f"layer 0 of the same step ({R * NB * 2} block-planes of {row_bytes} B, "
                                             f"{sample_bytes / 1e9:.2f} GB algorithmic)", parity)
        del planes0
        log(f"cpu baseline {rates}, parity {parity}")
    config = {"workload": "vllm-block-gather", "requests": R, "blocks_per_request": NB, "block_tokens": 16,
              "layers": L, "kv_heads": 8, "head_dim": 128, "pool_blocks": POOL, "pool_bytes": layout.capacity_bytes}
    roof = roofline(achieved, "copy_small_rows<KvGather,16> (ekv_gather_kv, 32 KiB rows)", gather_bytes,
                    phase["gather"], read_traffic("gather_kv_block_gather.md"))
    result = envelope(args, gather_bytes / (step_ms / 1e3) / 1e9, step_ms, config, roof, baseline,
                      {"pool_commit_s": round(commit_s, 3)}, metric="block gather GB/s (% of HBM peak), 1 GPU")
    del raw, output
    torch.cuda.synchronize()
    backing.close()
    return result


# ------------------------------------------------------------------ migration (demote/promote round trip)


def run_migration(torch, args, device):
    import numpy as np

    from adaptive_sparse.kv_pool import BlockMajorLayout
    from adaptive_sparse.migration_engine import MigrationEngine, PagedKVPool

    BLOCKS, LIVE, MOVE = 2048, 1024, 512
    layout = BlockMajorLayout(blocks=BLOCKS, layers=36, kv=2, row_bytes=16 * 8 * 128 * 2)
    pool = PagedKVPool(layout, device=device.index or 0)
    if args.spare_chunks:
        pool.backing.set_spare_chunks(args.spare_chunks)   # the sources' chunks serve the next tick's targets
    rng = np.random.default_rng(args.seed)
    live = sorted(rng.choice(np.arange(1, BLOCKS), size=LIVE, replace=False).tolist())
    pool.allocate(live)
    gen = torch.Generator(device=device).manual_seed(args.seed)
    for page in live:
        pool.page_view(page).view(torch.bfloat16).normal_(generator=gen)
    # The tick runs on a non-blocking stream: a HIP VMM unmap waits for the work queued on the legacy
    # null stream, not for other streams', so the sources' unmaps then overlap the PCIe legs and unpacks
    # (which never touch the unmapped chunks) instead of waiting for them.
    stream = torch.cuda.Stream(device)
    torch.cuda.set_stream(stream)
    engine = MigrationEngine(pool, max_pages=MOVE, sub_batch=64)
    snapshot = torch.empty((MOVE, layout.block_bytes), dtype=torch.uint8, device=device)
    moved = 2 * MOVE * layout.block_bytes
    ticks, verified = [], True
    phases = {"map_s": [], "move_s": [], "trim_s": [], "mapped": [], "unmapped": []}
    for tick in range(args.warmup + args.steps):
        sources = rng.choice(live, size=MOVE, replace=False).tolist()
        free = sorted(set(range(1, BLOCKS)) - set(live))
        targets = rng.choice(free, size=MOVE, replace=False).tolist()
        engine.pack(sources, snapshot)                  # reference copy, outside the timed tick
        torch.cuda.synchronize()
        backed_before = len(pool.backing.mapped_chunks)
        t0 = time.perf_counter()
        pool.allocate(targets)                          # hipMemMap-commit + zero the destination chunks
        t1 = time.perf_counter()
        mapped_now = len(pool.backing.mapped_chunks)
        host = engine.round_trip(sources, targets)      # pack -> D2H -> H2D -> unpack, pipelined
        pool.release(sources)
        unmapped = pool.trim(after=host.packed, pages=sources) // layout.chunk_bytes
        t2 = time.perf_counter()                        # unmap chunks only the sources used, once packed,
        torch.cuda.synchronize()                        # while the PCIe legs and unpacks still run
        t3 = time.perf_counter()
        engine.release_host(host)
        check = torch.empty_like(snapshot)
        engine.pack(targets, check)
        verified &= bool(torch.equal(check, snapshot))
        del check
        live = sorted(set(live) - set(sources) | set(targets))
        if tick >= args.warmup:
            ticks.append(t3 - t0)
            phases["map_s"].append(t1 - t0)
            phases["move_s"].append(t3 - t1)            # round trip, with the unmap overlapped
            phases["trim_s"].append(t2 - t1)            # issue + wait for the packs + release and unmap
            phases["mapped"].append(mapped_now - backed_before)
            phases["unmapped"].append(unmapped)
    tick_s = statistics.mean(ticks)
    map_chunks, unmap_chunks = statistics.mean(phases["mapped"]), statistics.mean(phases["unmapped"])
    # GPU-only time of one pipelined round trip (no VMM call beside it), to set against the tick.
    sources = rng.choice(live, size=MOVE, replace=False).tolist()
    ev_rt = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    torch.cuda.synchronize()
    ev_rt[0].record()
    host = engine.round_trip(sources, sources)          # back into the same pages: the bytes do not change
    ev_rt[1].record()
    torch.cuda.synchronize()
    engine.release_host(host)
    gpu_round_trip_ms = ev_rt[0].elapsed_time(ev_rt[1])
    # Phase breakdown of one non-pipelined move (events per stream).
    sources = torch.tensor(rng.choice(live, size=MOVE, replace=False).tolist(), device=device)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(5)]
    torch.cuda.synchronize()
    engine.pack(sources, engine.out_staging)   # keeps the GPU busy while the timed launches are queued
    ev[0].record()
    engine.pack(sources, engine.out_staging)
    ev[1].record()
    engine.host.copy_(engine.out_staging, non_blocking=True)
    ev[2].record()
    engine.in_staging.copy_(engine.host, non_blocking=True)
    ev[3].record()
    engine.unpack(sources, engine.in_staging)
    ev[4].record()
    torch.cuda.synchronize()
    pack_ms, d2h_ms, h2d_ms, unpack_ms = (ev[i].elapsed_time(ev[i + 1]) for i in range(4))
    one_way = MOVE * layout.block_bytes
    pack_bytes = 2 * one_way + MOVE * 4
    log(f"tick {tick_s * 1e3:.1f} ms ({moved / tick_s / 1e9:.1f} GB/s migrated), pack {pack_ms:.2f} ms, "
        f"D2H {d2h_ms:.1f} ms, H2D {h2d_ms:.1f} ms, unpack {unpack_ms:.2f} ms, verified {verified}")
    baseline = None
    if not args.no_cpu_baseline:
        # Pack + unpack of 64 blocks in host memory with torch (index_select into
        # staging, index_copy_ back): the byte movement without a PCIe leg.
        count = 64
        page_ids = torch.tensor(sorted(rng.choice(live, size=count, replace=False).tolist()))
        host_pool = torch.zeros((BLOCKS, layout.block_bytes), dtype=torch.uint8)
        for p in page_ids.tolist():
            host_pool[p] = pool.page_view(p).cpu()
        original = host_pool[page_ids].clone()

        def sample():
            staging = host_pool.index_select(0, page_ids)
            host_pool.index_copy_(0, page_ids, staging)
            return staging

        parity = {"round_trip": bool(torch.equal(sample(), original) and torch.equal(host_pool[page_ids], original))}
        sample_bytes = 2 * 2 * count * layout.block_bytes
        rates = cpu_rates(torch, sample, sample_bytes, cpu_budget(args, "migration"))
        baseline = cpu_baseline_entry(rates, f"pack + unpack of {count} blocks in host memory ({sample_bytes / 1e9:.2f}"
                                             f" GB read + written; no PCIe leg exists on the CPU path)", parity)
        del host_pool
    config = {"workload": "page-migration-round-trip", "blocks_per_tick": MOVE, "block_bytes": layout.block_bytes,
              "layers": 36, "kv_heads": 8, "head_dim": 128, "block_tokens": 16, "pool_blocks": BLOCKS,
              "spare_chunks": args.spare_chunks}
    roof = roofline(pack_bytes / (pack_ms / 1e3) / 1e9, "copy_small_rows<KvGather,16> (pack, 32 KiB rows)",
                    pack_bytes, pack_ms, read_traffic("pack_page_migration.md"))
    extra = {"verified_round_trip": verified, "tick_ms": round(tick_s * 1e3, 3),
             "phase_ms": {"map_and_zero": round(statistics.mean(phases["map_s"]) * 1e3, 3),
                          "pipelined_move_with_unmap": round(statistics.mean(phases["move_s"]) * 1e3, 3),
                          "release_and_unmap_overlapped": round(statistics.mean(phases["trim_s"]) * 1e3, 3),
                          "pack": round(pack_ms, 3), "d2h": round(d2h_ms, 3), "h2d": round(h2d_ms, 3),
                          "unpack": round(unpack_ms, 3)},
             "gpu_round_trip_ms": round(gpu_round_trip_ms, 3),
             "vmm_chunks_per_tick": {"mapped": round(map_chunks, 1), "unmapped": round(unmap_chunks, 1)},
             "vmm_us_per_chunk": {
                 "map_and_zero": round(statistics.mean(phases["map_s"]) * 1e6 / max(map_chunks, 1), 1),
                 "release_and_unmap": round(statistics.mean(phases["trim_s"]) * 1e6 / max(unmap_chunks, 1), 1)},
             "link_gbs": {"d2h": round(one_way / (d2h_ms / 1e3) / 1e9, 2),
                          "h2d": round(one_way / (h2d_ms / 1e3) / 1e9, 2), "peak_per_direction": PCIE_PEAK_GBS},
             "pack_gbs": round(pack_bytes / (pack_ms / 1e3) / 1e9, 1),
             "unpack_gbs": round(pack_bytes / (unpack_ms / 1e3) / 1e9, 1)}
    result = envelope(args, moved / tick_s / 1e9, tick_s * 1e3, config, roof, baseline, extra,
                      metric="migrated GB/s (D2H + H2D bytes per tick / tick time), 1 GPU")
    torch.cuda.synchronize()
    torch.cuda.set_stream(torch.cuda.default_stream(device))
    pool.close()
    return result


# ------------------------------------------------------------------ hisparse-swap (SGLang convention)


def run_hisparse_swap(torch, args, device):
    import numpy as np

    from adaptive_sparse.hisparse_swap import load_blocks_to_device_buffer_mha

    R, T, H, K, BS = 128, 65536, 4096, 16, 128
    ROW = 2 * 128 * 2                        # 2 KV heads x head_dim 128, bf16
    HOST_ROWS = 1 << 21                      # 1 GiB per plane of pinned host rows
    W = K * BS
    total = args.warmup + args.steps
    rng = np.random.default_rng(args.seed)
    # Step i: length T - total + i + 1; 13 of the 32 blocks holding the last 4096 tokens (the newest
    # block included) and 3 older blocks - the 80 % / 20 % locality mix in 128-token blocks.
    blocks = np.empty((total, R, K), np.int32)
    lengths = T - total + np.arange(total) + 1
    for step, length in enumerate(lengths):
        last = (int(length) - 1) // BS
        recent = last - np.argsort(rng.random((R, 31)), axis=1)[:, :12] - 1
        older = np.argsort(rng.random((R, last - 31)), axis=1)[:, :3]
        picked = np.concatenate([np.full((R, 1), last), recent, older], axis=1)
        blocks[step] = np.take_along_axis(picked, np.argsort(rng.random((R, K)), axis=1), axis=1)
    host_locs = (np.arange(T)[None, :] + np.arange(R)[:, None] * 7919) % HOST_ROWS
    dev_locs = np.arange(R * (H + 1), dtype=np.int64).reshape(R, H + 1) + 1
    host = torch.empty((2, HOST_ROWS, ROW), dtype=torch.uint8).pin_memory()
    host.copy_(torch.randint(0, 256, host.shape, dtype=torch.uint8, device=device))
    device_k = torch.zeros((R * (H + 1) + 1, ROW), dtype=torch.uint8, device=device)
    device_v = torch.zeros_like(device_k)
    tokens = torch.full((R, H + 1), -1, dtype=torch.int32, device=device)
    lru = torch.arange(H, dtype=torch.int16, device=device).repeat(R, 1)
    blocks_d = torch.tensor(blocks, device=device)
    seq_d = torch.tensor(np.repeat(lengths[:, None], R, axis=1), dtype=torch.int32, device=device)
    host_locs_d = torch.tensor(host_locs, device=device)
    dev_locs_d = torch.tensor(dev_locs, dtype=torch.int32, device=device)
    req = torch.arange(R, device=device)
    out = torch.empty((R, W), dtype=torch.int32, device=device)

    def call(step, state):
        load_blocks_to_device_buffer_mha(
            top_k_blocks=blocks_d[step], device_buffer_tokens=state[0], host_cache_locs=host_locs_d,
            device_buffer_locs=dev_locs_d, host_cache_k=host[0], host_cache_v=host[1], device_buffer_k=state[2],
            device_buffer_v=state[3], top_k_device_locs=out, req_pool_indices=req, seq_lens=seq_d[step],
            lru_slots=state[1], item_size_bytes=ROW, hot_buffer_size=H, sparse_block_size=BS)

    live = (tokens, lru, device_k, device_v)
    for step in range(args.warmup):
        call(step, live)
    torch.cuda.synchronize()
    saved = tuple(t.clone() for t in live)
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    torch.cuda.synchronize()
    host_us = []   # host time of each call (it returns once queued: the per-layer launch cost of a serving loop)
    wall0 = time.perf_counter()
    marks[0].record()
    for i in range(args.steps):
        h0 = time.perf_counter()
        call(args.warmup + i, live)
        host_us.append((time.perf_counter() - h0) * 1e6)
        marks[i + 1].record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - wall0) * 1e3 / args.steps
    call_ms = [marks[i].elapsed_time(marks[i + 1]) for i in range(args.steps)]
    # Replay the timed steps from the saved state: misses per call from the slots that took new tokens,
    # and the first timed call's results for the parity check.
    replay = tuple(t.clone() for t in saved)
    misses, first = [], None
    for i in range(args.steps):
        before = replay[0].clone()
        call(args.warmup + i, replay)
        misses.append(int((replay[0] != before).sum().item()))
        if i == 0:
            first = (out.cpu().numpy(), replay[0].cpu().numpy(), replay[1].cpu().numpy())
    promoted = [m * 2 * ROW for m in misses]
    mean_ms = statistics.mean(call_ms)
    achieved = statistics.mean(promoted) / (mean_ms / 1e3) / 1e9
    length = int(lengths[args.warmup])
    looked_up = R * ((K - 1) * BS + (length - (length - 1) // BS * BS) - 1)   # selected tokens but the newest
    hit_rate = 1 - statistics.mean(misses) / looked_up
    log(f"swap-in call {mean_ms:.3f} ms, {statistics.mean(misses):.0f} misses per call (hit rate {hit_rate:.3f}), "
        f"{achieved:.1f} GB/s promoted over PCIe")
    baseline = None
    parity = None
    if not args.no_cpu_baseline:
        from oracle import oracle as ref

        host_np = host.numpy()
        s_tokens, s_lru = saved[0].cpu().numpy(), saved[1].cpu().numpy()
        s_k, s_v = saved[2].cpu().numpy(), saved[3].cpu().numpy()
        step = args.warmup

        def sample():
            return ref.hisparse_swap(blocks[step], s_tokens, host_locs, dev_locs, host_np[0], host_np[1], s_k, s_v,
                                     np.arange(R), np.full(R, lengths[step]), s_lru, H, BS)

        want = sample()
        rows = want[0][want[0] >= 0]
        parity = {"locations": bool(np.array_equal(first[0], want[0])),
                  "hot_state": bool(np.array_equal(first[1], want[1]) and np.array_equal(first[2], want[2]))}
        # Rows of the first call, read back from a replay of that call alone.
        check = tuple(t.clone() for t in saved)
        call(step, check)
        rows_t = torch.tensor(rows, device=device)
        parity["rows"] = bool(np.array_equal(check[2][rows_t].cpu().numpy(), want[3][rows])
                              and np.array_equal(check[3][rows_t].cpu().numpy(), want[4][rows]))
        del check, want
        median, runs = time_cpu(sample, args.cpu_seconds)
        baseline = {"value": round(promoted[0] / median / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
                    "sample": (f"the first timed call ({R} requests, {misses[0]} misses): the Python oracle on one "
                               f"thread, median of {runs} runs ({median * 1e3:.0f} ms), {cpu_model()}"),
                    "parity": parity}
        log(f"cpu baseline {baseline['value']} GB/s, parity {parity}")
    config = {"workload": "hisparse-swap-sglang-convention", "requests": R, "context": T, "hot_buffer_size": H,
              "topk_blocks": K, "block_tokens": BS, "row_bytes": ROW, "host_rows": HOST_ROWS,
              "selection": "newest block + 12 of the other 31 recent blocks + 3 older blocks per call"}
    roof = {"bound": "pcie", "achieved": round(achieved, 2), "peak": PCIE_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / PCIE_PEAK_GBS, 4), "traffic": None,
            "kernel": "hisparse_swap_kernel<16> (ekv_hisparse_swap_in)",
            "algorithmic_bytes_per_launch": round(statistics.mean(promoted)), "avg_launch_ms": round(mean_ms, 4)}
    extra = {"call_ms": spread(call_ms), "misses_per_call": round(statistics.mean(misses), 1),
             "hit_rate": round(hit_rate, 4), "tokens_per_s": round(R * W / (mean_ms / 1e3), 1),
             "host_us_per_call": round(statistics.median(host_us), 2)}
    result = envelope(args, achieved, wall_ms, config, roof, baseline, extra,
                      metric="HiSparse swap-in promoted GB/s (host rows copied per call / call time), 1 GPU")
    return result


# ------------------------------------------------------------------ lookup-micro (the reference's microbenchmark)

# The reference's published figures for this microbenchmark (results/lookup-micro/results.json, A100-SXM4-80GB):
# p50 microseconds per call of its Triton resolver and of its torch indexing sequence, batch 1 / 2 / 4.
REFERENCE_LOOKUP_MICRO_US = {"triton_p50": {1: 30.54, 2: 30.00, 4: 30.08}, "torch_p50": {1: 213.80, 2: 211.06, 4: 211.88}}


def run_lookup_micro(torch, args, device):
    """tests/bench_resident_lookup.py of the reference, on this library's resolve_resident.

    Per batch of 1, 2 and 4 requests: a two-level lookup (int64 table -> int64
    mapping) of 16 Top-K blocks of 128 tokens (2048 lanes per row) over
    8192-token rows, the closed form ((B-1-row)*8192 + block*512 + off + 1)*3 + 5
    checked first; then 100 warm-up calls of each path and 40 rounds of 100
    calls, the two paths alternating, HIP events per round (time per call,
    host launch included, as the reference measures). The torch path is the
    reference's indexing sequence on the GPU. Also the same 100 calls replayed
    from one HIP graph (no host launch).
    """
    from adaptive_sparse.resident_lookup import resolve_resident

    per_batch = {}
    for batch in (1, 2, 4):
        selected = torch.arange(batch, device=device)
        rows = selected.flip(0)
        lengths = torch.full((batch,), 8192, dtype=torch.int32, device=device)
        table = torch.arange(batch * 8192, device=device).reshape(batch, 8192) + 1
        mapping = torch.arange(batch * 8192 + 1, device=device) * 3 + 5
        topk = (torch.arange(16, device=device) * 4).int().expand(1, batch, 16).contiguous()
        lane = torch.arange(128, device=device)

        def torch_lookup():
            result = torch.empty((batch, 2048), device=device, dtype=torch.int32)
            blocks = topk[0, selected].long()
            positions = (blocks.unsqueeze(-1) * 128 + lane).flatten(1)
            valid = (positions >= 0) & (positions < lengths[selected, None])
            logical = table[rows[selected, None], positions.masked_fill(~valid, 0)]
            result[selected] = mapping[logical].masked_fill(~valid, -1).int()
            return result.unsqueeze(0)

        def hip_lookup(out=None):
            result = torch.empty((1, batch, 2048), device=device, dtype=torch.int32) if out is None else out
            resolve_resident(topk, table, mapping, rows, lengths, selected, result, 128)
            return result

        expected = torch.tensor([[((batch - 1 - row) * 8192 + block * 512 + offset + 1) * 3 + 5
                                  for block in range(16) for offset in range(128)] for row in range(batch)],
                                dtype=torch.int32, device=device).unsqueeze(0)
        correct = bool(torch.equal(torch_lookup(), expected) and torch.equal(hip_lookup(), expected))
        timings = {"hip": [], "torch": []}
        methods = [("hip", hip_lookup), ("torch", torch_lookup)]
        for _, call in methods:
            for _ in range(100):
                call()
        torch.cuda.synchronize()
        for round_number in range(40):
            for name, call in methods[::(-1 if round_number % 2 else 1)]:
                begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                begin.record()
                for _ in range(100):
                    call()
                end.record()
                end.synchronize()
                timings[name].append(begin.elapsed_time(end) * 10)     # us per call
        # The same 100 calls replayed from one HIP graph.
        out = torch.empty((1, batch, 2048), device=device, dtype=torch.int32)
        hip_lookup(out)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(100):
                hip_lookup(out)
        graph.replay()
        torch.cuda.synchronize()
        correct &= bool(torch.equal(out, expected))
        replays = []
        for _ in range(20):
            begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            begin.record()
            graph.replay()
            end.record()
            end.synchronize()
            replays.append(begin.elapsed_time(end) * 10)
        del graph
        stats = {name: {"p50_us": round(statistics.median(v), 2),
                        "p95_us": round(statistics.quantiles(v, n=20, method="inclusive")[18], 2)}
                 for name, v in timings.items()}
        per_batch[batch] = {"correct": correct, **stats, "graph_us_per_call": round(statistics.median(replays), 2),
                            "reference_a100_triton_p50_us": REFERENCE_LOOKUP_MICRO_US["triton_p50"][batch],
                            "reference_a100_torch_p50_us": REFERENCE_LOOKUP_MICRO_US["torch_p50"][batch]}
        log(f"lookup micro batch {batch}: {per_batch[batch]}")
    value = per_batch[1]["hip"]["p50_us"]
    config = {"workload": "resident-lookup-micro", "context": 8192, "topk_blocks": 16, "block_size": 128,
              "lanes_per_row": 2048, "batches": [1, 2, 4], "lookup": "two-level (int64 table -> int64 mapping)",
              "rounds": 40, "calls_per_round": 100, "warmup_calls": 100}
    result = envelope(args, value, value / 1e3, config, None, None,
                      {"per_batch": {str(b): v for b, v in per_batch.items()},
                       "correct": all(v["correct"] for v in per_batch.values())},
                      unit="us", metric="resident lookup us per call (p50, batch 1, host launch included)")
    result["higher_is_better"] = False
    result["vs_baseline"] = round(value / REFERENCE_LOOKUP_MICRO_US["triton_p50"][1], 4)
    result["dtype"] = "int64"
    result["data"] = "the reference microbenchmark's closed-form inputs"
    result["steps"], result["warmup"] = 40 * 100, 100   # per path and batch: 40 rounds of 100 calls
    return result


def reference_support_sets(length, selected, seed=137):
    """The three position sets of scripts/analyze_virtual_layout.py:11-27: the first `selected` positions, a
    uniform sample, and runs of selected // 8 positions from random starts (the same generator calls, so the same
    sets)."""
    import random

    draw = random.Random(seed)
    run = max(1, selected // 8)
    clustered = set()
    while len(clustered) < selected:
        start = draw.randrange(length)
        clustered.update((start + i) % length for i in range(min(run, selected - len(clustered))))
    return {"contiguous": list(range(selected)), "uniform_random": draw.sample(range(length), selected),
            "synthetic_clustered": sorted(clustered)}


def run_virtual_addressing(torch, args, device):
    """scripts/bench_virtual_addressing.py of the reference, on this library's gather_rows.

    4 requests x 65,536 positions of 256 bf16 (512 B rows) in a VMM arena, 2048 positions gathered per request
    from each of the three support sets, direct (layout arithmetic) and software-table (two dependent lookups)
    addressing over identical payload addresses; every result checked against the closed-form payload
    (pos * 256 + col + req * 17) % 97, invalid lanes too; then 30 rounds of 20 host-launched calls, the two modes
    alternating (HIP events, us per call, as the reference measures), and 20 calls replayed from a HIP graph.
    """
    from experimental.resident_arena import VmmResidentArena
    from experimental.sparse_read import gather_rows
    from experimental.virtual_layout import VirtualKVLayout

    batch, length, selected, width, rounds, calls = 4, 65536, 2048, 256, 30, 20
    layout = VirtualKVLayout(batch, length, width)
    arena = VmmResidentArena(layout)
    results = {}
    try:
        for req in range(batch):
            arena.reserve(req, length)
            view = arena.row_view(req, length, torch.bfloat16)
            view.copy_(((torch.arange(length * width, device=device) + req * 17) % 97).reshape(length, width))
        del view
        raw = arena.backing.raw.view(torch.bfloat16)
        request_ids = torch.arange(batch, device=device, dtype=torch.int64).flip(0)
        lengths = torch.full((batch,), length, device=device, dtype=torch.int64)
        count = batch * length
        table = torch.arange(count, 0, -1, device=device, dtype=torch.int64).reshape(batch, length)
        flat = torch.arange(count, device=device, dtype=torch.int64)
        offsets = torch.zeros(count + 1, device=device, dtype=torch.int64)
        offsets[table.flatten()] = (layout.chunk_bytes // layout.itemsize
                                    + (flat // length) * (layout.request_bytes // layout.itemsize)
                                    + (flat % length) * width)
        del flat
        output = torch.empty((batch, selected, width), device=device, dtype=torch.bfloat16)
        lanes = batch * selected
        moved = {False: lanes * (2 * width * 2 + 8),                  # row read + row written + position
                 True: lanes * (2 * width * 2 + 8 + 8 + 8)}           # + table entry + element offset
        correct = True
        for name, support in reference_support_sets(length, selected).items():
            positions = torch.tensor(support, device=device, dtype=torch.int64).expand(batch, -1).contiguous()
            columns = torch.arange(width, device=device)
            expected = ((positions[..., None] * width + columns + request_ids[:, None, None] * 17) % 97).to(
                torch.bfloat16)

            def call(indirect, read=positions):
                gather_rows(raw, read, request_ids, lengths, table, offsets, output, layout, indirect=indirect)

            for indirect in (False, True):
                call(indirect)
                correct &= bool(torch.equal(output, expected))
                for invalid in (-1, length):
                    bad = positions.clone()
                    bad[:, 0] = invalid
                    call(indirect, bad)
                    correct &= bool(torch.equal(output[:, 1:], expected[:, 1:])) and not output[:, 0].any()
                for _ in range(30):
                    call(indirect)
            torch.cuda.synchronize()
            timings = {False: [], True: []}
            for repeat in range(rounds):
                for indirect in ((False, True) if repeat % 2 == 0 else (True, False)):
                    begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    begin.record()
                    for _ in range(calls):
                        call(indirect)
                    end.record()
                    end.synchronize()
                    timings[indirect].append(begin.elapsed_time(end) * 1e3 / calls)
            entry = {}
            for indirect, label in ((False, "direct"), (True, "software_table")):
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    for _ in range(calls):
                        call(indirect)
                graph.replay()
                torch.cuda.synchronize()
                correct &= bool(torch.equal(output, expected))
                replays = []
                for _ in range(10):
                    begin, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    begin.record()
                    graph.replay()
                    end.record()
                    end.synchronize()
                    replays.append(begin.elapsed_time(end) * 1e3 / calls)
                del graph
                p50, graph_us = statistics.median(timings[indirect]), statistics.median(replays)
                entry[label] = {"p50_us": round(p50, 2), "graph_us_per_call": round(graph_us, 2),
                                "graph_gbs": round(moved[indirect] / (graph_us / 1e6) / 1e9, 1)}
            results[name] = entry
            log(f"virtual addressing {name}: {entry}")
        del raw, output
        torch.cuda.synchronize()
    finally:
        arena.close()
    value = results["uniform_random"]["direct"]["graph_gbs"]
    config = {"workload": "virtual-addressing-gather", "batch": batch, "length": length, "selected": selected,
              "width_bf16": width, "rounds": rounds, "calls_per_round": calls,
              "support_sets": list(results), "modes": ["direct", "software_table"]}
    result = envelope(args, value, results["uniform_random"]["direct"]["graph_us_per_call"] / 1e3, config, None,
                      None, {"per_support_set": results, "correct": bool(correct)},
                      metric="gather_rows GB/s per call from a HIP graph (uniform-random positions, direct)")
    result["data"] = "the reference gather benchmark's closed-form payload"
    result["steps"], result["warmup"] = rounds * calls, 30
    return result


# ------------------------------------------------------------------ composite (config 5)


def composite_topk(torch, device, L, R, K, lengths, gen, recent_window=4096):
    """Per (layer, request): K unique tokens, 80 % from the last 4096 of the request's context, 20 % from the rest."""
    T = int(lengths.max())
    uniform_want = K - (K * 4) // 5
    if recent_window < K or T < uniform_want:
        raise ValueError("composite Top-K needs recent_window >= K and contexts of at least the uniform picks")
    older = (lengths - recent_window).clamp_min(0)                               # [R]
    u_count = torch.minimum(older, torch.full_like(older, uniform_want))         # uniform picks per request
    r_count = K - u_count
    recent = torch.rand((L, R, recent_window), generator=gen, device=device).argsort(-1)[..., :K]
    recent = recent + older.view(1, R, 1)
    keys = torch.rand((L, R, T), generator=gen, device=device)
    keys.masked_fill_(torch.arange(T, device=device).view(1, 1, T) >= older.view(1, R, 1), 2.0)
    uniform = keys.topk(uniform_want, dim=-1, largest=False).indices              # valid where < older
    del keys
    lane = torch.arange(K, device=device).view(1, 1, K)
    take_recent = lane < r_count.view(1, R, 1)
    pick = torch.where(take_recent, recent, torch.gather(uniform, -1, (lane - r_count.view(1, R, 1)).clamp(0, uniform_want - 1)))
    order = torch.rand((L, R, K), generator=gen, device=device).argsort(-1)
    return torch.gather(pick, -1, order).to(torch.int32).contiguous()


def run_composite(torch, args, device):
    import numpy as np

    from adaptive_sparse.host_arena import HostArena
    from adaptive_sparse.kv_pool import KVPlanes, PlanePoolLayout
    from adaptive_sparse.resident_lookup import build_residency_bits, resolve_resident
    from adaptive_sparse.sparse_read import gather_kv
    from adaptive_sparse.swap_in import INT32_MIN, HotBuffers, move_kv, swap_in

    L, R, K, C, HOST_ROWS = 60, 128, 2048, 4096, 65536
    row_bytes = 512
    gen = torch.Generator(device=device).manual_seed(args.seed)
    lengths = torch.randint(4096, 32769, (R,), generator=gen, device=device)
    T = int(lengths.max())
    layout = PlanePoolLayout(layers=L, kv=2, rows=1 + R * C, row_bytes=row_bytes)
    backing, raw, commit_s = make_pool(torch, layout, device, args.seed + 1)
    planes = layout.kv_planes(backing.base, 0, owner=backing)
    # Pinned, device-mapped host copy: 65,536 rows per plane; token t of request r lives at row (r*T + t) % rows.
    host_plane = HOST_ROWS * row_bytes
    arena = HostArena(2 * L * host_plane)
    fill = torch.empty(host_plane, dtype=torch.uint8, device=device)
    for p in range(2 * L):
        fill.view(torch.bfloat16).normal_(generator=gen)
        arena.host.narrow(0, p * host_plane, host_plane).copy_(fill)
    del fill
    host_planes = KVPlanes(base=arena.device_ptr, device=0, layers=L, kv=2, layer_stride=2 * host_plane,
                           kv_stride=host_plane, row_stride=row_bytes, row_bytes=row_bytes, rows=HOST_ROWS, owner=arena)
    host_table = ((torch.arange(R, device=device).view(R, 1) * T + torch.arange(T, device=device).view(1, T))
                  % HOST_ROWS).to(torch.int32)
    # Graph-replayable swap-in; int16 local-slot table, as the decode-read lookup uses.
    buffers = HotBuffers(L, R, T, C, device, step_counter=True, table_dtype=torch.int16)
    recent = (lengths.view(1, R, 1) - C + torch.arange(C, device=device).view(1, 1, C)).expand(L, R, C)
    local = torch.rand((L, R, C), generator=gen, device=device).argsort(-1)
    buffers.install(recent, local)
    rows = torch.arange(R, device=device)
    lengths32 = lengths.to(torch.int32)
    # Prefill the hot rows from the host copy.
    all_lanes = torch.full((L, R), C, dtype=torch.int32, device=device)
    move_kv(host_planes, host_table[rows.view(1, R, 1), recent].to(torch.int32).contiguous(), planes,
            (local + buffers.slot_base.view(1, R, 1)).to(torch.int32).contiguous(), all_lanes)
    slots = torch.empty((L, R, K), dtype=torch.int32, device=device)
    misses = torch.empty_like(slots)
    counts = torch.empty((L, R), dtype=torch.int32, device=device)
    promote_src = torch.empty_like(slots)
    promote_dst = torch.empty_like(slots)
    output = torch.empty((R, L, 2, K, 256), dtype=torch.bfloat16, device=device)
    chunk_rows = layout.chunk_bytes // row_bytes
    remap_count = int(round(args.remap_fraction * backing.chunk_count))
    if args.spare_chunks:
        backing.set_spare_chunks(args.spare_chunks)   # reclaimed chunks' memory kept for the re-ensure
    rng = np.random.default_rng(args.seed)
    torch.cuda.synchronize()
    log(f"composite ready: T={T}, host arena {arena.nbytes / 1e9:.1f} GB, remap {remap_count} chunks/step")

    remap_parts = {"invalidate_ms": [], "unmap_ms": [], "map_ms": []}
    # Device-resident fill values: a Python scalar in an indexed assignment is copied from pageable host
    # memory, a copy that blocks the host until the stream's queued work (the summary rebuild) has run.
    fill = {"table": torch.zeros((), dtype=buffers.table.dtype, device=device),
            "slot_token": torch.full((), -1, dtype=torch.int32, device=device),
            "stamps": torch.full((), INT32_MIN, dtype=torch.int32, device=device),
            "zero_counts": torch.zeros_like(counts)}

    def invalidate(groups=1):
        """Choose `remap_count` random chunks (never chunk 0) and empty their hot slots (queued, no wait).

        Returns the chunk ids, split in `groups` consecutive groups, and the [L, R] group of the (layer,
        request) items whose slots they hold (the last group holding any of its slots; -1: none): a 2 MiB
        chunk of a plane is 4096 rows of 512 B, so it holds (most of) one request's hot buffer.
        """
        chosen = rng.choice(np.arange(1, backing.chunk_count), size=remap_count, replace=False)
        ids = torch.tensor(chosen, device=device)
        plane, within = ids // layout.plane_chunks, ids % layout.plane_chunks
        slot = (within.view(-1, 1) * chunk_rows + torch.arange(chunk_rows, device=device).view(1, -1))
        layer = (plane // 2).view(-1, 1).expand_as(slot)
        assignment = np.arange(len(chosen)) * groups // len(chosen)     # the group of each chosen chunk
        group = torch.tensor(assignment, device=device).view(-1, 1).expand_as(slot)
        keep = (slot >= 1) & (slot < layout.rows)
        slot, layer, group = slot[keep], layer[keep], group[keep]
        req, loc = (slot - 1) // C, (slot - 1) % C
        token = buffers.slot_token[layer, req, loc].long()
        held = token >= 0
        buffers.table[layer[held], req[held], token[held]] = fill["table"]
        buffers.slot_token[layer, req, loc] = fill["slot_token"]
        buffers.stamps[layer, req, loc] = fill["stamps"]
        build_residency_bits(buffers.table, out=buffers.bits)
        item_group = torch.full((L * R,), -1, dtype=torch.int64, device=device)
        item_group.scatter_reduce_(0, layer * R + req, group, reduce="amax")
        return [chosen[assignment == g].tolist() for g in range(groups)], item_group.view(L, R)

    def remap_chunks(chosen):
        r1 = time.perf_counter()
        backing.reclaim(chosen, synchronize=False)   # hipMemUnmap + release (or keep); no kernel uses them
        r2 = time.perf_counter()
        backing.ensure(chosen)                       # hipMemCreate + map + access + zero fill
        r3 = time.perf_counter()
        return r2 - r1, r3 - r2

    def remap():
        """Unmap + remap the chosen chunks with the GPU idle (the form the graph replays below use)."""
        r0 = time.perf_counter()
        (chosen,), _ = invalidate()
        torch.cuda.synchronize()
        r1 = time.perf_counter()
        unmap_s, map_s = remap_chunks(chosen)
        for key, value in zip(remap_parts, (r1 - r0, unmap_s, map_s)):
            remap_parts[key].append(value * 1e3)

    topk = torch.zeros((L, R, K), dtype=torch.int32, device=device)   # refilled in place every step

    def lookup():
        resolve_resident(topk, buffers.table, None, rows, lengths32, rows, slots, 1, misses=misses,
                         miss_count=counts, resident_bits=buffers.bits, slot_base=buffers.slot_base)

    def swap():
        swap_in(topk, 1, rows, rows, slots, misses, counts, buffers, host_table, promote_src, promote_dst)

    def promote():
        move_kv(host_planes, promote_src, planes, promote_dst, counts)

    def gather():
        gather_kv(planes, slots, output)

    phases = {name: [] for name in ("remap_ms", "lookup_ms", "swap_ms", "promote_ms", "gather_ms", "step_ms",
                                    "gpu_beside_remap_ms", "after_remap_ms")}
    promoted, verified = [], True

    def verify():
        """Every lane is resident after the step: its gathered rows must be its token's host rows.

        Checked in every layer on the GPU: the expected rows are gathered from the pinned host copy
        (device-mapped) by the token's host row, ten layers at a time, and compared bit for bit.
        """
        host_rows = torch.gather(host_table.expand(L, R, T), 2, topk.long())               # [L, R, K]
        ok = True
        for first in range(0, L, 10):
            last = min(L, first + 10)
            part = dataclasses.replace(host_planes, base=host_planes.base + first * host_planes.layer_stride,
                                       layers=L - first)
            expect = torch.empty((R, last - first, 2, K, 256), dtype=torch.bfloat16, device=device)
            gather_kv(part, host_rows[first:last].contiguous(), expect, zero_below=0)
            ok &= bool(torch.equal(output[:, first:last].view(torch.int16), expect.view(torch.int16)))
        return ok

    # The step runs on a non-blocking stream. A HIP VMM unmap waits for the work queued on the legacy null
    # stream but not for other streams' (measured: 50 unmaps took 55.6 ms behind a 42 ms kernel on the null
    # stream, 12.4 ms behind one on a side stream, 13.2 ms idle), so the remap's driver calls run on the
    # host while kernels that never touch the chunks being remapped run on the GPU:
    #   queue: invalidate the chosen chunks' slots -> lookup -> swap-in -> promote of the items whose
    #          hot buffers the chunks do not hold
    #   host:  per group of the chosen chunks, unmap (+ release) and re-commit (map + zero fill, waited
    #          for) them, then queue the promote of the items whose hot buffers that group completes (into
    #          the fresh chunks): an item's group is the last one holding any of its slots, so no queued
    #          promote touches a chunk of a later group, and those promotes run while the later groups'
    #          driver calls do
    #   queue: gather
    # The chunks' last readers are the previous step's kernels, which the step boundary has drained.
    groups = 1 if args.serial_remap else max(1, args.remap_groups)
    stream = torch.cuda.Stream(device)
    torch.cuda.set_stream(stream)
    counts_part = torch.empty_like(counts)      # rewritten and read in stream order
    no_items = torch.full((L, R), -1, dtype=torch.int64, device=device)
    step_remap = {"queue_ms": [], "unmap_ms": [], "map_ms": []}
    for step in range(args.warmup + args.steps):
        topk.copy_(composite_topk(torch, device, L, R, K, lengths, gen))
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(6)]
        t0 = time.perf_counter()
        chunk_groups, item_group = invalidate(groups) if remap_count else ([[]] * groups, no_items)
        ev[0].record()
        lookup()
        ev[1].record()
        swap()
        ev[2].record()
        torch.where(item_group < 0, counts, fill["zero_counts"], out=counts_part)
        move_kv(host_planes, promote_src, planes, promote_dst, counts_part)
        ev[3].record()
        if args.serial_remap:
            torch.cuda.synchronize()            # the comparison form: the driver calls with the GPU idle
        t1 = time.perf_counter()
        unmap_s = map_s = 0.0
        group_events = []
        for group, chunks in enumerate(chunk_groups):
            if chunks:
                unmap_g, map_g = remap_chunks(chunks)
                unmap_s, map_s = unmap_s + unmap_g, map_s + map_g
            pair = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            pair[0].record()
            torch.where(item_group == group, counts, fill["zero_counts"], out=counts_part)
            move_kv(host_planes, promote_src, planes, promote_dst, counts_part)
            pair[1].record()
            group_events.append(pair)
        t2 = time.perf_counter()
        ev[4].record()
        gather()
        ev[5].record()
        torch.cuda.synchronize()
        t3 = time.perf_counter()
        promoted.append(int(counts.sum().item()))
        if step == args.warmup + args.steps - 1 or step == 0:
            verified &= verify()
        if step >= args.warmup:
            phases["remap_ms"].append((t2 - t1) * 1e3)
            step_remap["queue_ms"].append((t1 - t0) * 1e3)
            step_remap["unmap_ms"].append(unmap_s * 1e3)
            step_remap["map_ms"].append(map_s * 1e3)
            phases["lookup_ms"].append(ev[0].elapsed_time(ev[1]))
            phases["swap_ms"].append(ev[1].elapsed_time(ev[2]))
            phases["promote_ms"].append(ev[2].elapsed_time(ev[3]) + sum(a.elapsed_time(b) for a, b in group_events))
            phases["gather_ms"].append(ev[4].elapsed_time(ev[5]))
            phases["gpu_beside_remap_ms"].append(ev[0].elapsed_time(ev[3]))
            phases["after_remap_ms"].append((t3 - t2) * 1e3)
            phases["step_ms"].append((t3 - t0) * 1e3)
    torch.cuda.synchronize()
    torch.cuda.set_stream(torch.cuda.default_stream(device))
    # The same step replayed from one HIP graph (the swap-in reads its LRU step from
    # the device counter), with the chunk remap between replays.
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        lookup()
        swap()
        promote()
        gather()
    graph_ms, graph_verified = [], True
    for replay in range(max(2, min(args.steps, 5))):
        topk.copy_(composite_topk(torch, device, L, R, K, lengths, gen))
        torch.cuda.synchronize()
        if remap_count:
            remap()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        graph.replay()
        stop.record()
        stop.synchronize()
        graph_ms.append(start.elapsed_time(stop))
        graph_verified &= verify()
    del graph
    log(f"graph replays: {statistics.mean(graph_ms):.2f} ms of GPU time per step, verified {graph_verified}")
    mean = {k: statistics.mean(v) for k, v in phases.items()}
    lanes = L * R * K
    misses_per_step = statistics.mean(promoted[args.warmup:])
    gather_bytes = lanes * 2 * row_bytes * 2 + lanes * 4             # every lane resident after promotion
    promote_bytes = misses_per_step * 2 * row_bytes
    # Swap-in, per (layer, request): the C int32 stamps read and written back and the K lookup slots read; per miss
    # its list entry, Top-K id, host row and victim's token read, the patched slot, the victim's token, the two int16
    # table entries, the two summary words and the two promotion entries written (44 B).
    swap_bytes = L * R * (8 * C + 4 * K + 4) + misses_per_step * 44
    serial_gpu = mean["lookup_ms"] + mean["swap_ms"] + mean["promote_ms"] + mean["gather_ms"]
    log(f"step {mean['step_ms']:.1f} ms: remap {mean['remap_ms']:.1f} ms (unmap "
        f"{statistics.mean(step_remap['unmap_ms'] or [0]):.1f} + map {statistics.mean(step_remap['map_ms'] or [0]):.1f})"
        f" beside {mean['gpu_beside_remap_ms']:.1f} ms of GPU work, then {mean['after_remap_ms']:.1f} ms; GPU work "
        f"lookup {mean['lookup_ms']:.3f} + swap {mean['swap_ms']:.3f} + promote {mean['promote_ms']:.2f} + gather "
        f"{mean['gather_ms']:.2f} = {serial_gpu:.1f} ms; {misses_per_step / lanes:.3f} of lanes promoted; "
        f"verified {verified}")
    config = {"workload": "composite-elastic-decode", "requests": R, "context": "uniform [4096, 32768]", "layers": L,
              "kv_heads": 2, "head_dim": 128, "topk": K, "hot_capacity": C, "remap_fraction": args.remap_fraction,
              "spare_chunks": args.spare_chunks,
              "host_rows_per_plane": HOST_ROWS}
    achieved = gather_bytes / (mean["gather_ms"] / 1e3) / 1e9
    roof = roofline(achieved, "copy_small_rows<KvGather,16> (ekv_gather_kv)", gather_bytes, mean["gather_ms"], None)
    extra = {"verified_against_host_copy": verified, "phase_ms": {k: round(v, 3) for k, v in mean.items()},
             "promoted_rows_per_step": round(misses_per_step), "promoted_fraction": round(misses_per_step / lanes, 4),
             "promote_gbs_over_pcie": round(promote_bytes / (mean["promote_ms"] / 1e3) / 1e9, 2),
             "swap_in": {"algorithmic_bytes": round(swap_bytes),
                         "gbs": round(swap_bytes / (mean["swap_ms"] / 1e3) / 1e9, 1),
                         "frac_of_hbm_peak": round(swap_bytes / (mean["swap_ms"] / 1e3) / 1e9 / HBM_PEAK_GBS, 4)},
             "lookups_per_s": round(lanes / (mean["lookup_ms"] / 1e3), 1),
             "gpu_work_ms": round(serial_gpu, 3), "serial_remap": bool(args.serial_remap),
             "overlap": "the remap's unmap + map run on the host beside the lookup, swap-in and the promote of the "
                        "items whose hot buffers the remapped chunks do not hold (a non-blocking stream); the chunks "
                        "are remapped in groups, each followed by the promote of the items it completes, which "
                        "runs beside the later groups' driver calls; the gather follows",
             "remap_groups": groups,
             "remap_parts_ms": {k: round(statistics.mean(v), 2) if v else 0.0 for k, v in step_remap.items()},
             "vmm_us_per_chunk": {
                 "unmap_and_release" if not args.spare_chunks else "unmap":
                     round(statistics.mean(step_remap["unmap_ms"]) * 1e3 / remap_count, 1) if remap_count else None,
                 "map_and_zero": round(statistics.mean(step_remap["map_ms"]) * 1e3 / remap_count, 1)
                 if remap_count else None},
             "remapped_chunks_per_step": remap_count, "pool_commit_s": round(commit_s, 3),
             "graph_replay": {"replays": len(graph_ms), "gpu_ms_per_step": round(statistics.mean(graph_ms), 3),
                              "verified_against_host_copy": graph_verified}}
    result = envelope(args, gather_bytes / (mean["step_ms"] / 1e3) / 1e9, mean["step_ms"], config, roof, None, extra,
                      metric="composite decode step: gathered GB/s per step (lookup, LRU swap-in, promote, gather, remap)")
    del raw, output
    torch.cuda.synchronize()
    backing.close()
    arena.close()
    return result


def run_residency_summary(torch, args, device):
    """Residency-summary rebuild (ekv_residency_bits) of the config-3 int16 table, shifts 6 and 0."""
    from adaptive_sparse.resident_lookup import build_residency_bits, summary_words

    L, R, T, C = 60, 128, 65536, 4096
    gen = torch.Generator(device=device).manual_seed(args.seed)
    table = torch.zeros((L, R, T), dtype=torch.int16, device=device)
    table[..., T - C:] = torch.randint(1, C + 1, (L, R, C), dtype=torch.int16, device=device, generator=gen)
    results, verified = {}, True
    for shift in (6, 0):
        out = torch.zeros((L, R, summary_words(T, shift)), dtype=torch.int32, device=device)
        for _ in range(max(1, args.warmup)):
            build_residency_bits(table, out=out, shift=shift)
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(args.steps):
            build_residency_bits(table, out=out, shift=shift)
        stop.record()
        stop.synchronize()
        ms = start.elapsed_time(stop) / args.steps
        words = -(-(T >> shift) // 32)
        nbytes = table.numel() * 2 + L * R * words * 4            # table read + summary words written
        # torch restatement on the first and last layer: bit j of word w = any(table[p] != 0) over its group
        picked = table[[0, L - 1]]
        groups = (picked != 0).view(2, R, T >> shift, 1 << shift).any(-1).view(2, R, words, 32).to(torch.int64)
        want = (groups << torch.arange(32, device=device)).sum(-1)
        verified &= bool(torch.equal(out[[0, L - 1]][..., :words].to(torch.int64) & 0xffffffff, want))
        results[shift] = {"ms": ms, "bytes": nbytes, "gbs": nbytes / (ms / 1e3) / 1e9}
        log(f"residency summary shift {shift}: {ms * 1e3:.1f} us, {nbytes / 1e9:.3f} GB, "
            f"{results[shift]['gbs']:.0f} GB/s, verified {verified}")
    main_run = results[6]
    roof = roofline(main_run["gbs"], "residency_pieces_kernel<int16> (ekv_residency_bits, shift 6)", main_run["bytes"],
                    main_run["ms"], read_traffic("residency_summary_config3.md"))
    config = {"workload": "residency-summary-rebuild", "layers": L, "requests": R, "context": T, "hot_capacity": C,
              "table": "int16 local slots", "bits_shift": 6}
    extra = {"verified_against_torch": verified,
             "shift0": {"ms": round(results[0]["ms"], 4), "gbs": round(results[0]["gbs"], 1),
                        "frac": round(results[0]["gbs"] / HBM_PEAK_GBS, 4), "bytes": results[0]["bytes"]}}
    return envelope(args, main_run["gbs"], main_run["ms"], config, roof, None, extra,
                    metric="residency summary rebuild GB/s (int16 table read + summary written), 1 GPU")


WORKLOADS = {"decode-read": run_decode_read, "topk-gather": run_topk_gather, "lookup-micro": run_lookup_micro,
             "virtual-addressing": run_virtual_addressing, "residency-summary": run_residency_summary,
             "block-gather": run_block_gather, "migration": run_migration, "composite": run_composite,
             "hisparse-swap": run_hisparse_swap}


# (key, workload, argument overrides) of the other configurations the default line carries.
MIGRATION_SPARE_CHUNKS = 700   # > the ~500 chunks a 512-block tick frees and maps
COMPOSITE_SPARE_CHUNKS = 800   # > the 774 chunks (5 % of the pool) a composite step remaps
EXTRA_CONFIGS = (("config1_topk_gather", "topk-gather", {}), ("config2_block_gather", "block-gather", {}),
                 ("config4_migration", "migration", {}),
                 ("config4_migration_spare_pool", "migration",
                  {"spare_chunks": MIGRATION_SPARE_CHUNKS, "no_cpu_baseline": True}),
                 # About one second per step (the remap's VMM calls): 3 timed steps after 1 warm-up.
                 ("config5_composite", "composite", {"steps": 3, "warmup": 1, "no_cpu_baseline": True}),
                 ("config5_composite_spare_pool", "composite",
                  {"steps": 3, "warmup": 1, "spare_chunks": COMPOSITE_SPARE_CHUNKS, "no_cpu_baseline": True}),
                 # The decode read at twice the hot capacity (81 % hits): the lookup's longest default case.
                 ("config3_capacity_8192", "decode-read", {"capacity": 8192, "no_cpu_baseline": True}),
                 ("lookup_micro", "lookup-micro", {}),
                 ("virtual_addressing", "virtual-addressing", {}),
                 ("residency_summary", "residency-summary", {}))


def apply_profile_switch(environment, keep):
    """Diagnostic ranges cost host time per call: a timed run has none unless asked."""
    if keep:
        environment["EKV_PROFILE_RANGES"] = "1"
    else:
        environment.pop("EKV_PROFILE_RANGES", None)


def summary(result):
    """The fields of another workload's line that the default line carries for it."""
    keys = ("metric", "value", "unit", "ms_per_step", "roofline", "cpu_baseline", "config", "lookup_us_per_step",
            "hit_rate", "verified_round_trip", "tick_ms", "link_gbs", "pack_gbs", "unpack_gbs", "phase_ms",
            "higher_is_better", "vs_baseline", "per_batch", "correct", "verified_against_host_copy",
            "gpu_work_ms", "overlap", "remap_parts_ms", "vmm_us_per_chunk", "vmm_chunks_per_tick",
            "gpu_round_trip_ms", "promote_gbs_over_pcie", "swap_in", "graph_replay",
            "per_support_set", "verified_against_torch", "shift0", "lookup_roofline", "event_spread",
            "lookup_arms_back_to_back", "lookup_variants_identical")
    return {key: result[key] for key in keys if key in result}


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported: this path has no "
              "cross-GPU step (each GPU runs its own shard independently)", file=sys.stderr)
        return 2
    apply_profile_switch(os.environ, args.profile_ranges)
    import torch

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    ceilings = None
    if not args.no_copy_ceiling:
        log("measuring streaming ceilings (own read / write / copy kernels)")
        ceilings = stream_ceilings(torch, device)
        log(f"ceilings {ceilings}")
    result = WORKLOADS[args.workload](torch, args, device)
    result["copy_ceiling_gbs"] = None if ceilings is None else ceilings["copy"]["best_gbs"]
    result["stream_ceilings_gbs"] = ceilings
    result["profile_ranges"] = args.profile_ranges
    if args.workload == "decode-read" and not args.no_extras:
        torch.cuda.empty_cache()
        for key, workload, overrides in EXTRA_CONFIGS:
            log(f"extra: {key}")
            result[key] = summary(WORKLOADS[workload](torch, argparse.Namespace(**{**vars(args), **overrides}),
                                                      device))
            torch.cuda.empty_cache()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
