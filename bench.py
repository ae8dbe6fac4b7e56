#!/usr/bin/env python3
"""Page16 decode benchmark on one MI355X.

Workload: B=16 sequences at ctx=32768 (2048 pages each), H_q=32, H_kv=8,
D=128, bf16 K/V pool of 40960 pages with fully fragmented (permuted) block
tables, q/K/V ~ N(0,1), scale 1/sqrt(128). One step = one Page16 decode call
(one layer-step) through the drop-in ``page16_decode_attention`` -> libukv.so,
with every input already resident in HBM.

Prints ONE JSON line:
  value        achieved HBM GB/s = algorithmic bytes / (measured ms per step)
  ms_per_step  wall time per call from HIP events around the K timed calls
  roofline     the decode kernel's achieved GB/s against MI355X's 8 TB/s
  cpu_baseline the reference's Page16 page loop restated in C (oracle/),
               timed on this host's cores on a bounded sample of the workload
Algorithmic bytes per step: each attended token's K and V once (4096 B per
token), q, out, block table and lengths = 2,147,876,928 B.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBPS = 8000.0
METRIC = "Page16 decode µs/step + achieved HBM GB/s (%peak), B=16 ctx=32K, 1×MI355X"
PMC_SUMMARY = ROOT / "profiles" / "page16_decode_longctx_pmc.txt"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def pmc_traffic_bytes():
    """HBM bytes per decode launch from the committed rocprofv3 --pmc summary, if any."""
    if not PMC_SUMMARY.exists():
        return None
    for line in PMC_SUMMARY.read_text().splitlines():
        if line.startswith("traffic_bytes_per_step:"):
            try:
                return int(float(line.split(":", 1)[1].split()[0]))
            except ValueError:
                return None
    return None


def cpu_baseline(tc, layout, budget_s: float):
    """Time the C page-loop oracle on the host on the first S sequences (bounded)."""
    import numpy as np
    import torch

    from oracle import oracle
    from unifiedkv_amd import workloads

    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or len(os.sched_getaffinity(0))
    os.environ["OMP_NUM_THREADS"] = str(threads)
    bt = layout["block_table"]
    lens = layout["seqlens"]
    D, Hq, Hkv = layout["D"], layout["Hq"], layout["Hkv"]
    dt = workloads.DTYPE_CODES[layout["dtype"]]

    def host_sample(nseq):
        rows, o, ids = [], 0, []
        for b in range(nseq):
            n = (int(lens[b]) + 15) // 16
            ids.append(bt[b, :n])
            rows.append(np.arange(o, o + n, dtype=np.int32))
            o += n
        idx = torch.from_numpy(np.concatenate(ids).astype(np.int64)).to(tc["k_cache"].device)
        k = tc["k_cache"].index_select(0, idx).view(torch.int16).cpu().numpy().view(np.uint16)
        v = tc["v_cache"].index_select(0, idx).view(torch.int16).cpu().numpy().view(np.uint16)
        q = tc["q"][:nseq].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
        return q, k, v, workloads.tables_from_pages(rows), np.ascontiguousarray(lens[:nseq])

    def run(sample):
        q, k, v, t, l = sample
        t0 = time.perf_counter()
        oracle.page16_decode_pageloop(q, k, v, t, l, softmax_scale=tc["scale"], n_rep=tc["n_rep"], dtype=dt)
        return time.perf_counter() - t0

    s1 = host_sample(1)
    t1 = run(s1)
    nseq = int(max(1, min(layout["B"], round(2.0 / max(t1, 1e-3)))))
    sample = s1 if nseq == 1 else host_sample(nseq)
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < budget_s and len(times) < 20):
        times.append(run(sample))
    med = sorted(times)[len(times) // 2]
    sbytes = workloads.decode_bytes(sample[4], nseq, Hq, Hkv, D, sample[3].shape[1])
    gbps = sbytes / med / 1e9
    return {
        "value": round(gbps, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"C restatement of core/page16_native.py:34-80 (fp32 page loop, OpenMP over "
                   f"(seq, q head)) on the first {nseq} of {layout['B']} config-2 sequences "
                   f"({int(np.sum(sample[4]))} tokens), median of {len(times)} runs"),
        "us_per_step_equiv": None,
        "seconds_per_sample_run": round(med, 4),
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--seed", type=int, default=2024)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="budget of the CPU baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device copy (known bytes) for scaling PMC counters")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: --gpus {args.gpus} requested, but this build measures the Page16 decode path on one "
              "GPU only (no sharding or collectives are built); run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from unifiedkv_amd import page16_native, workloads

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    if not page16_native.HAS_TRITON:
        raise RuntimeError("libukv.so is not built/loadable; run __graft_entry__.build() first")
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)

    if args.calibrate_copy:
        # A plain device copy of exactly 1 GiB read + 1 GiB written per dispatch.
        src = torch.ones(1 << 29, dtype=torch.bfloat16, device=dev)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes_read": src.numel() * 2, "calibrate_copy_bytes_written": dst.numel() * 2,
                          "dispatches": args.steps}), flush=True)
        return

    layout = workloads.layout_longctx(np.random.default_rng(args.seed))
    log(f"[bench] building config 2 on {torch.cuda.get_device_name(dev)}: B={layout['B']} "
        f"ctx=32768 pool={layout['N']} pages bf16")
    tc = workloads.torch_decode_case(layout, args.seed, device=dev)
    torch.cuda.synchronize()
    step_bytes = workloads.decode_bytes(layout["seqlens"], layout["B"], layout["Hq"], layout["Hkv"], layout["D"],
                                        layout["block_table"].shape[1])

    def step():
        return page16_native.page16_decode_attention(tc["q"], tc["k_cache"], tc["v_cache"], tc["block_table"],
                                                     tc["seqlens"], softmax_scale=tc["scale"], n_rep=tc["n_rep"])

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"[bench] warmup {args.warmup} done; timing {args.steps} steps")

    # whole timed region
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps):
        step()
    end.record()
    torch.cuda.synchronize()
    ms_per_step = start.elapsed_time(end) / args.steps

    # per-launch durations of the decode call on the stream it runs on
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for a, b in evs:
        a.record()
        step()
        b.record()
    torch.cuda.synchronize()
    per_launch_ms = [a.elapsed_time(b) for a, b in evs]
    kern_ms = sum(per_launch_ms) / len(per_launch_ms)
    log(f"[bench] region {ms_per_step * 1e3:.1f} us/step, per-launch mean {kern_ms * 1e3:.1f} us, "
        f"min {min(per_launch_ms) * 1e3:.1f} us")

    gbps = step_bytes / (ms_per_step * 1e-3) / 1e9
    kern_gbps = step_bytes / (kern_ms * 1e-3) / 1e9
    traffic = pmc_traffic_bytes()

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] timing the CPU baseline sample")
        cpu = cpu_baseline(tc, layout, args.cpu_seconds)
        cpu["us_per_step_equiv"] = round(step_bytes / (cpu["value"] * 1e9) * 1e6, 1)
        log(f"[bench] cpu baseline {cpu['value']} GB/s on {cpu['cores']} threads")

    rec = {
        "metric": METRIC,
        "value": round(gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/K/V, random-permutation block tables)",
        "config": {
            "workload": "page16_decode_config2_longctx",
            "batch": layout["B"], "ctx": 32768, "num_q_heads": layout["Hq"], "num_kv_heads": layout["Hkv"],
            "head_dim": layout["D"], "page_size": 16, "pool_pages": layout["N"], "kv_dtype": "bf16",
        },
        "us_per_step": round(ms_per_step * 1e3, 2),
        "pct_of_peak_hbm": round(100.0 * gbps / PEAK_HBM_GBPS, 2),
        "tokens_per_s_32_layers": round(layout["B"] / (32 * ms_per_step * 1e-3), 1),
        "algorithmic_bytes_per_step": step_bytes,
        "roofline": {
            "bound": "hbm",
            "achieved": round(kern_gbps, 2),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(kern_gbps / PEAK_HBM_GBPS, 4),
            "traffic": traffic,
            "kernel_us": round(kern_ms * 1e3, 2),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
