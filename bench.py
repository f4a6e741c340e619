"""Benchmark: ms per Pairformer pair-stack block at N = 512 (bf16) on one MI355X, with the
triangle-attention core's TFLOP/s against the bf16 MFMA peak.

Workload (one step): one Pairformer pair-stack block -- LayerNorm-fed triangle
multiplication outgoing + incoming (c_hidden 128), triangle attention starting + ending
node (4 heads x 32), pair transition (x4) -- on z [1, 512, 512, 128] bf16 ~N(0,1), fp32
parameters (seeded init), ragged padding: the real length is drawn from U{300..512}
(seed 0) and the key mask zeroes the padded tokens. Inputs are resident in HBM before
the timed region; every step runs the full block through the native ``hip`` backend.

Reported beside it, in the same JSON line:
* ``roofline``: the triangle-attention flash core (the block's dominant MFMA kernel),
  launched on operands of the workload's exact shape between HIP events on the stream it
  runs on; achieved = 4 N^3 H D FLOP per launch / average launch time, against the
  2.5 PFLOP/s dense bf16 peak. ``kernels`` adds the LayerNorm's HBM rate the same way.
* ``cpu_baseline``: the fp32 CPU oracle (``oracle/pairstack.py``, kind "port") timed on the
  host's cores on the same block and input (1 warm-up, median of 3), with the GPU
  result's rel-RMS against it.

``python bench.py [--steps K] [--warmup W] [--n 512] [--no-cpu-baseline]``; one GPU only.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "ms per Pairformer block @N=512 bf16; triangle-attn TFLOP/s & % MFMA peak"
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--n", type=int, default=512)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-runs", type=int, default=3)
    ap.add_argument("--copy-reference-mb", type=int, default=0,
                    help="also run a plain device copy of this many MiB (the HBM-counter calibration)")
    return ap.parse_args()


def real_length(n: int, seed: int) -> int:
    import torch

    g = torch.Generator().manual_seed(seed)
    lo = min(300, n)
    return int(torch.randint(lo, n + 1, (1,), generator=g).item())


def event_time_ms(fn, reps: int) -> float:
    """Average ms of ``fn`` over ``reps`` launches between two events on the current stream."""
    import torch

    fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        fn()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / reps


def flash_roofline(n: int, length: int, reps: int) -> dict:
    """The flash core on the workload's operand shapes: [1, 4 heads, n rows, n, 32]."""
    import torch

    from foldforge_amd import kernels

    heads, d = 4, 32
    np_ = (n + 127) // 128 * 128
    g = torch.Generator(device="cuda").manual_seed(1)
    q = (torch.randn(1, heads, n, np_, d, device="cuda", generator=g) * 0.25).bfloat16()
    k = torch.randn(1, heads, n, np_, d, device="cuda", generator=g).bfloat16()
    vt = torch.randn(1, heads, n, d, np_, device="cuda", generator=g).bfloat16()
    bias = torch.randn(1, heads, np_, np_, device="cuda", generator=g)
    keep = torch.arange(np_, device="cuda") < length
    bias = torch.where(keep[None, None, None, :], bias, torch.tensor(float("-inf"), device="cuda"))
    bias = kernels.blocked_bias(bias)
    out = torch.empty(1, n, n, heads * d, device="cuda", dtype=torch.bfloat16)

    def launch():
        kernels.flash_attention_bias(q, k, vt, bias, out, rows_valid=n, n_valid=n)

    ms = event_time_ms(launch, reps)
    flops = 4.0 * n**3 * heads * d
    achieved = flops / (ms * 1e-3) / 1e12
    return {"bound": "mfma", "kernel": "flash_attn_bias", "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": recorded_traffic("flash_attn_bias_n512"), "us_per_launch": round(ms * 1e3, 2),
            "flop_per_launch": flops}


def layernorm_roofline(n: int, reps: int) -> dict:
    import torch

    from foldforge_amd import kernels

    x = torch.randn(n * n, 128, device="cuda").bfloat16()
    w = torch.ones(128, device="cuda")
    b = torch.zeros(128, device="cuda")
    ms = event_time_ms(lambda: kernels.layer_norm(x, w, b, 1e-5), reps)
    nbytes = 2.0 * n * n * 128 * 2
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"kernel": "layer_norm_bf16_128", "bound": "hbm", "achieved": round(gbs, 1),
            "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
            "us_per_launch": round(ms * 1e3, 2), "bytes_per_launch": nbytes}


def copy_reference(mib: int, reps: int = 3) -> dict:
    """A plain device-to-device copy of known size: what the HBM read / write counters report
    for it calibrates the counters of the kernels above (bytes per counted KiB)."""
    import torch

    src = torch.empty(mib << 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    ms = event_time_ms(lambda: dst.copy_(src), reps)
    return {"bytes_each_way": mib << 20, "us_per_copy": round(ms * 1e3, 2),
            "gbs": round(2.0 * (mib << 20) / (ms * 1e-3) / 1e9, 1)}


def recorded_traffic(kernel: str) -> float | None:
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3 counter summary
    (``profiles/<kernel>_traffic.md``, line ``traffic_bytes_per_launch: <n>``), else None."""
    path = ROOT / "profiles" / f"{kernel}_traffic.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.strip().startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def cpu_baseline(z, mask, state, gpu_out, runs: int) -> dict:
    import platform

    import torch

    from oracle import pairstack as ps

    threads = min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    ps.pairformer_block(z, mask, state)  # warm-up
    times = []
    out = None
    for _ in range(runs):
        t0 = time.perf_counter()
        out = ps.pairformer_block(z, mask, state)
        times.append(time.perf_counter() - t0)
    where = mask[:, :, None] & mask[:, None, :]
    rr = ps.rel_rms(gpu_out.double() - z.double(), out.double() - z.double(), where)
    cpu = platform.processor() or platform.machine()
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(statistics.median(times) * 1e3, 1), "unit": "ms per block",
            "cores": threads, "kind": "port",
            "sample": f"the full timed workload: one block at N={z.shape[1]}, fp32, oracle/pairstack.py, "
                      f"median of {runs} after 1 warm-up; {cpu}",
            "gpu_vs_cpu_update_rel_rms": round(rr, 5)}


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the pair stack's "
              "multi-GPU sharding is a design note, not part of this build", file=sys.stderr)
        return 2
    import torch

    from foldforge_amd import factories, serving
    from foldforge_amd.policy import guard
    from foldforge_amd.trunk import randomise

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    n = args.n
    length = real_length(n, args.seed)
    g = torch.Generator().manual_seed(args.seed)
    z_cpu = torch.randn(1, n, n, 128, generator=g).bfloat16()
    mask_cpu = torch.ones(1, n, dtype=torch.bool)
    mask_cpu[0, length:] = False
    block = randomise(factories.pairformer_block(d_pair=128, triangle_model="af3"), seed=args.seed).to(dev)
    block.set_backend("hip")
    for m in block.children_ops():
        guard(m, "error")  # a refused call would raise instead of running torch ops
    z, mask = z_cpu.to(dev), mask_cpu.to(dev)

    with torch.no_grad():
        for _ in range(args.warmup):
            out = block(z, mask)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        start.record()
        for _ in range(args.steps):
            out = block(z, mask)
        end.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    ms_per_step = start.elapsed_time(end) / args.steps
    served = serving.report_observations(block)["modules"]
    hip_calls = sum(v["served_host_calls"].get("hip", 0) for v in served.values())
    print(f"timed {args.steps} steps: {ms_per_step:.3f} ms/step (wall {wall * 1e3 / args.steps:.3f}); "
          f"hip op calls {hip_calls}", file=sys.stderr, flush=True)

    roof = flash_roofline(n, length, args.kernel_reps)
    ln = layernorm_roofline(n, args.kernel_reps)
    print(f"flash core {roof['us_per_launch']} us {roof['achieved']} TFLOP/s; "
          f"layernorm {ln['us_per_launch']} us {ln['achieved']} GB/s", file=sys.stderr, flush=True)
    gpu_out = out.cpu()
    copy = copy_reference(args.copy_reference_mb) if args.copy_reference_mb > 0 else None

    base = None
    if not args.no_cpu_baseline:
        base = cpu_baseline(z_cpu, mask_cpu, block.state_dict(), gpu_out, args.cpu_runs)
        print(f"cpu baseline {base['value']} ms/block on {base['cores']} threads", file=sys.stderr, flush=True)

    gflop = (2 * (2 * n**3 * 128 + n * n * (8 * 128 * 128 + 2 * 128 * 128 + 2 * 128 * 128))
             + 2 * (4 * n**3 * 4 * 32 + n * n * (8 * 128 * 128 + 2 * 128 * 4 + 2 * 128 * 128))
             + n * n * (4 * 128 * 512 + 2 * 512 * 128)) / 1e9
    line = {
        "metric": METRIC,
        "value": round(ms_per_step, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"Pairformer pair-stack block, N={n}, ragged real length {length} (key mask), "
                        "c_z=128, trimul hidden 128, triangle attention 4x32, transition x4, batch 1",
            "n_tokens": n, "real_length": length, "batch": 1, "c_z": 128,
            "block_gflop": round(gflop, 1), "block_tflops": round(gflop / ms_per_step, 1),
        },
        "roofline": roof,
        "kernels": {"layer_norm": ln, **({"copy_reference": copy} if copy else {})},
        "cpu_baseline": base,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
