"""Benchmark: ms per Pairformer pair-stack block at N = 512 (bf16) on one MI355X, with the
triangle-attention core's TFLOP/s against the bf16 MFMA peak.

Workload (one step): one Pairformer pair-stack block -- LayerNorm-fed triangle
multiplication outgoing + incoming (c_hidden 128), triangle attention starting + ending
node (4 heads x 32), pair transition (x4) -- on z [1, 512, 512, 128] bf16 ~N(0,1), fp32
parameters (seeded init), ragged padding: the real length is drawn from U{300..512}
(seed 0) and the key mask zeroes the padded tokens. Inputs are resident in HBM before
the timed region; every step runs the full block through the native ``hip`` backend.
After the W warm-up steps, untimed steps continue until ``--settle-ms`` (500) of wall
time has passed since the first warm-up step: an idle MI355X needs a few hundred ms of
load to reach its steady clock, and a timed region of 20 blocks (~25 ms) started from a
cold clock has measured up to 2.8x slow. ``config.clock_settle`` reports those steps.

Reported beside it, in the same JSON line:
* ``roofline``: the triangle-attention flash core (the block's dominant MFMA kernel),
  launched on operands of the workload's exact shape between HIP events on the stream it
  runs on; achieved = 4 N^3 H D FLOP per launch / average launch time, against the
  2.5 PFLOP/s dense bf16 peak. ``kernels`` adds the LayerNorm's HBM rate the same way.
  ``roofline.logit_regimes``: the same launch with q scaled x0.25 / x2 / x8.5 (x8.5: logits up
  to about 100 nats above the offset, the trained-weight scale), time per launch and the share
  of softmax rows that take the lazy rescale or the exact path.
* ``cpu_baseline``: the fp32 CPU oracle (``oracle/pairstack.py``, kind "port") timed on the
  host's cores on the same block and input (1 warm-up, median of 3), with the GPU
  result's rel-RMS against it.

* ``shapes``: the same block at its other widths, N = 384: the template stacks of AF3 (pair 64,
  4 x 16 heads, hidden 64, transition x 2), Protenix-1 (4 x 32 heads, hidden 128) and Boltz-2
  (4 x 32 heads, transition x 4), 4 templates each, and the confidence head (pair 128 + single
  384, 5 samples), ms per block on ``hip`` and on the engine ``pytorch`` backend.
* ``trunk``: the 48-block trunk with its single track (c_s 384, 16 x 24 attention with
  pair bias) at N = 512, all-ones mask, z and s ~N(0,1), 3 passes (144 block evaluations),
  every op on ``hip``: ms per trunk run, ms per block, the single track's share, and the
  residual-stream RMS after the last block. ``trunk.parity`` (with the CPU baseline): block
  evaluations 1, 72 and 144 of the hip trunk re-run on the fp32 CPU oracle from the same
  input (update rel-RMS), and the final state against the fp32 reference trunk.
* ``ladder``: the same trunk at N = 768, 1024, 1536 and 2048 (ms per trunk run).

``python bench.py [--steps K] [--warmup W] [--n 512] [--no-cpu-baseline] [--no-trunk]``;
one GPU only. ``--ladder`` instead prints one JSON line per length of the trunk's length
ladder (N = 768 ... 2048 full trunks, then single blocks upward until the device is out of
memory); ``--trunk-only`` prints the trunk line alone (with the engine ``pytorch``
backend's trunk time beside it, the fp32 CPU oracle's per-block time x 144, and the trunk
replayed as one captured graph at N = 128 and 512).
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
    ap.add_argument("--settle-ms", type=float, default=500.0,
                    help="after the warm-up steps, keep running untimed steps until this much wall "
                         "time has passed since the first one (the GPU clock ramps up under load)")
    ap.add_argument("--n", type=int, default=512)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--kernel-reps", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-runs", type=int, default=3)
    ap.add_argument("--copy-reference-mb", type=int, default=0,
                    help="also run a plain device copy of this many MiB (the HBM-counter calibration)")
    ap.add_argument("--no-trunk", action="store_true", help="skip the 48-block trunk measurement")
    ap.add_argument("--no-logit-regimes", action="store_true",
                    help="skip the flash core's large-logit timings (counter passes take the bench shape only)")
    ap.add_argument("--trunk-only", action="store_true")
    ap.add_argument("--no-reference-backend", action="store_true",
                    help="with --trunk-only: skip the engine pytorch backend's trunk run")
    ap.add_argument("--no-graph", action="store_true",
                    help="with --trunk-only: skip the captured-graph replays (N = 128 and 512)")
    ap.add_argument("--ladder", action="store_true")
    ap.add_argument("--msa", action="store_true",
                    help="time the MSA-stack ops at L = 256 / 384 tokens, 512 MSA rows")
    ap.add_argument("--shapes", action="store_true",
                    help="time only the template-stack and confidence-head shapes of the block")
    ap.add_argument("--no-shapes", action="store_true",
                    help="leave the template-stack and confidence-head blocks out of the default line")
    ap.add_argument("--ladder-max", type=int, default=16384)
    return ap.parse_args()


def real_length(n: int, seed: int) -> int:
    import torch

    g = torch.Generator().manual_seed(seed)
    lo = min(300, n)
    return int(torch.randint(lo, n + 1, (1,), generator=g).item())


def event_time_ms(fn, reps: int, warm: int = 1) -> float:
    """Average ms of ``fn`` over ``reps`` launches between two events on the current stream,
    after ``warm`` untimed launches."""
    import torch

    for _ in range(max(1, warm)):
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
    vt = torch.randn(1, heads, n, np_ // 32, d, 32, device="cuda", generator=g).bfloat16()  # key-blocked v^T
    bias = torch.randn(1, heads, np_, np_, device="cuda", generator=g)
    keep = torch.arange(np_, device="cuda") < length
    bias = torch.where(keep[None, None, None, :], bias, torch.tensor(float("-inf"), device="cuda"))
    bias = kernels.blocked_bias(bias)
    out = torch.empty(1, n, n, heads * d, device="cuda", dtype=torch.bfloat16)

    def launch():
        kernels.flash_attention_bias(q, k, vt, bias, out, rows_valid=n, n_valid=n)

    # steady clock: the kernel runs untimed for about 300 ms first (the GPU raises its clock
    # under sustained load; a burst of a few launches after other work measures the ramp)
    one = event_time_ms(launch, 1)
    settle = max(50, int(300.0 / max(one, 1e-3)))
    ms = event_time_ms(launch, reps, warm=settle)
    flops = 4.0 * n**3 * heads * d
    achieved = flops / (ms * 1e-3) / 1e12
    return {"bound": "mfma", "kernel": "flash_attn_bias", "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": recorded_traffic("flash_attn_bias_n512"), "us_per_launch": round(ms * 1e3, 2),
            "flop_per_launch": flops}


def flash_logit_regimes(n: int, reps: int, q_scales=(0.25, 2.0, 8.5)) -> list[dict]:
    """The flash core at the workload's full-size shape with q scaled so that the q . k logits
    grow from the bench's small ones to the trained-weight regime (a row's largest logit about
    100 nats, 144 log2 units, above the offset taken from its first bias tile). For each scale:
    the time per launch, and the share of (head, row, query) softmax rows whose largest logit
    exceeds that offset by more than 64 log2 units (each takes the lazy rescale at least once)
    or falls more than 100 below it (the exact two-pass path), counted on the same operands."""
    import torch

    from foldforge_amd import kernels

    heads, d = 4, 32
    np_ = (n + 127) // 128 * 128
    rows = []
    for qs in q_scales:
        g = torch.Generator(device="cuda").manual_seed(1)
        q = (torch.randn(1, heads, n, np_, d, device="cuda", generator=g) * qs).bfloat16()
        k = torch.randn(1, heads, n, np_, d, device="cuda", generator=g).bfloat16()
        vt = torch.randn(1, heads, n, np_ // 32, d, 32, device="cuda", generator=g).bfloat16()
        bias = torch.randn(1, heads, np_, np_, device="cuda", generator=g)
        offset = bias[0, :, :, :32].amax(dim=-1)  # [heads, query]: the first key tile's maximum
        over = under = 0
        top = torch.empty(0)
        for h in range(heads):
            for r0 in range(0, n, 64):
                logits = torch.matmul(q[0, h, r0:r0 + 64].float(), k[0, h, r0:r0 + 64].float().transpose(1, 2))
                top = (logits + bias[0, h][None]).amax(dim=-1) - offset[h][None]  # [rows, query]
                over += int((top > 64).sum())
                under += int((top < -100).sum())
        total = heads * n * np_
        blocked = kernels.blocked_bias(bias)
        out = torch.empty(1, n, n, heads * d, device="cuda", dtype=torch.bfloat16)

        def launch():
            kernels.flash_attention_bias(q, k, vt, blocked, out, rows_valid=n, n_valid=n)

        one = event_time_ms(launch, 1)
        ms = event_time_ms(launch, reps, warm=max(50, int(300.0 / max(one, 1e-3))))
        rows.append({"q_scale": qs, "logit_std_log2": round(qs * d ** 0.5, 2),
                     "us_per_launch": round(ms * 1e3, 2),
                     "rows_rescaled_frac": round(over / total, 5), "rows_exact_frac": round(under / total, 5),
                     "finite": bool(torch.isfinite(out.float()).all())})
        del q, k, vt, bias, blocked, out, top
        torch.cuda.empty_cache()
    return rows


def layernorm_roofline(n: int, reps: int) -> dict:
    import torch

    from foldforge_amd import kernels

    from foldforge_amd import _native

    x = torch.randn(n * n, 128, device="cuda").bfloat16()
    w = torch.ones(128, device="cuda")
    b = torch.zeros(128, device="cuda")
    kernels.layer_norm(x, w, b, 1e-5)  # argument checks of the public wrapper, once
    # The kernel takes ~20 us, about what one Python-level call costs on the host: the timed
    # launches go straight to the C-ABI with a preallocated output, and 10x as many of them
    # (a burst of a few ms), so that the events measure the kernel and not the host.
    y = torch.empty_like(x)
    lib = _native.lib()
    stream = torch.cuda.current_stream().cuda_stream
    args = (x.data_ptr(), w.data_ptr(), b.data_ptr(), y.data_ptr(), n * n, 128, 1e-5, 0, stream)

    def launch():
        _native.check(lib.ffk_layer_norm(*args), "layer_norm")

    reps = max(200, 10 * reps)
    ms = event_time_ms(launch, reps, warm=reps)
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


FLASH_SOURCES = ("foldforge_amd/csrc/triattn.hip", "foldforge_amd/csrc/ffk_device.h",
                 "foldforge_amd/csrc/ffk_kernels.h")


def source_digest(paths=FLASH_SOURCES) -> str:
    """sha256 over the named source files (in order): the code a counter summary was taken on."""
    import hashlib

    h = hashlib.sha256()
    for p in paths:
        h.update((ROOT / p).read_bytes())
    return h.hexdigest()


def recorded_traffic(kernel: str) -> float | None:
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3 counter summary
    (``profiles/<kernel>_traffic.md``, line ``traffic_bytes_per_launch: <n>``). The summary
    names the digest of the flash-core sources it was measured on (``source_sha256: <hex>``);
    a summary of other sources is stale and gives None, as does a missing one."""
    path = ROOT / "profiles" / f"{kernel}_traffic.md"
    if not path.exists():
        return None
    fields = {}
    for line in path.read_text().splitlines():
        key, sep, val = line.strip().partition(":")
        if sep and key in ("traffic_bytes_per_launch", "source_sha256"):
            fields[key] = val.strip()
    if fields.get("source_sha256") != source_digest() or "traffic_bytes_per_launch" not in fields:
        return None
    return float(fields["traffic_bytes_per_launch"])


TRUNK_BLOCKS, TRUNK_PASSES, D_SINGLE = 48, 3, 384


def block_gflop(n: int, d_single: int = 0) -> float:
    """Algorithmic GFLOP of one block: TriMul x2, TriAttn x2 (core + projections), pair
    transition, and with a single track the attention with pair bias + single transition."""
    c, h, hd = 128, 128, 128
    trimul = 2 * n**3 * h + n * n * (8 * c * h + 2 * c * c + 2 * h * c)
    triattn = 4 * n**3 * hd + n * n * (8 * c * hd + 2 * c * 4 + 2 * hd * c)
    trans = n * n * (4 * c * 4 * c + 2 * 4 * c * c)
    total = 2 * trimul + 2 * triattn + trans
    if d_single:
        cs = d_single
        total += n * (8 * cs * cs + 2 * cs * cs) + 4 * n * n * cs + 2 * n * n * c * 16
        total += n * (4 * cs * 4 * cs + 2 * 4 * cs * cs)
    return total / 1e9


def op_gflop(n: int, keys: int | None = None) -> dict[str, float]:
    """GFLOP of each pair op of one block at N = n. ``keys`` (the key stages the kernels run on a
    ragged input: the 32-key stages up to the last real key) shortens the contraction and the
    attention core; None counts all n (the algorithmic work)."""
    c, h, hd = 128, 128, 128
    k = n if keys is None else keys
    trimul = 2 * n * n * k * h + n * n * (8 * c * h + 2 * c * c + 2 * h * c)
    triattn = 4 * n * n * k * hd + n * n * (8 * c * hd + 2 * c * 4 + 2 * hd * c)
    trans = n * n * (4 * c * 4 * c + 2 * 4 * c * c)
    return {"trimul_outgoing": trimul / 1e9, "trimul_incoming": trimul / 1e9,
            "triattn_starting": triattn / 1e9, "triattn_ending": triattn / 1e9, "transition": trans / 1e9}


def key_extent(n: int, length: int) -> int:
    """Keys the contraction and the flash core run over: 32-key stages up to the last real key."""
    return min(n, (length + 31) // 32 * 32)


#: The reference's per-op times for this block (engine ``cuda`` backend, H100 80GB, bf16, AF3
#: widths, L = 384; docs/archive/BACKENDS-engine-2.3.md:257-262): not MI355X numbers, shown
#: beside ours for scale only.
REFERENCE_H100_MS_384 = {"trimul_outgoing": 0.52, "triattn_starting": 0.28, "transition": 0.11}

OP_ATTRS = (("trimul_outgoing", "tri_multi_outgoing"), ("trimul_incoming", "tri_multi_incoming"),
            ("triattn_starting", "tri_atten_starting"), ("triattn_ending", "tri_atten_ending"),
            ("transition", "transition_pair"))


def op_times(block, z, mask, length: int, reps: int) -> dict:
    """ms of each pair op of ``block`` (whole op: LayerNorm, projections, core, gate, output,
    residual) between HIP events, with its executed TFLOP/s, and the block's own ms."""
    import torch

    from foldforge_amd.modules import attention_then_transition

    n = z.shape[1]
    gf = op_gflop(n, key_extent(n, length))
    ops = {}
    with torch.no_grad():
        for name, attr in OP_ATTRS:
            op = getattr(block, attr)
            call = (lambda: op(z)) if name == "transition" else (lambda: op(z, mask))
            ms = event_time_ms(call, reps, warm=max(20, reps))
            ops[name] = {"ms": round(ms, 4), "tflops_executed": round(gf[name] / ms, 1)}
        # the block runs its last two ops as one call (the attention's output projection inside
        # the transition kernel)
        fused_ms = event_time_ms(lambda: attention_then_transition(
            block.tri_atten_ending, block.transition_pair, z, mask), reps, warm=max(20, reps))
        block_ms = event_time_ms(lambda: block(z, mask), reps, warm=max(10, reps))
    fused = {"ms": round(fused_ms, 4),
             "tflops_executed": round((gf["triattn_ending"] + gf["transition"]) / fused_ms, 1)}
    calls = sum(ops[k]["ms"] for k in ("trimul_outgoing", "trimul_incoming", "triattn_starting")) + fused_ms
    return {"ops": ops, "triattn_ending_transition_fused": fused, "ms_per_block": round(block_ms, 4),
            "sum_of_ops_ms": round(sum(o["ms"] for o in ops.values()), 4),
            "sum_of_block_calls_ms": round(calls, 4)}


def single_op_n128(reps: int) -> dict:
    """The reference's CPU-runnable case on the GPU: the triangle-attention op (starting node) on
    z [1, 128, 128, 128] ~N(0, 1) (seed 0), 4 heads x 32, all-ones mask, random init from seed 0;
    the hip op on the bf16 rounding of z, and the engine pytorch backend on the same GPU in fp32
    (the case's own precision)."""
    import torch

    from foldforge_amd import factories
    from foldforge_amd.trunk import randomise

    z = torch.randn(1, 128, 128, 128, generator=torch.Generator().manual_seed(0)).cuda()
    mask = torch.ones(1, 128, dtype=torch.bool, device="cuda")
    ta = randomise(factories.triangle_attention(128, 4, starting=True, model="af3"), seed=0).cuda()
    out = {"workload": "triangle attention, starting node, z [1, 128, 128, 128], 4 x 32 heads, all-ones mask, "
                       "seed 0"}
    with torch.no_grad():
        ta.set_backend("hip")
        zb = z.bfloat16()
        out["hip_ms_bf16"] = round(event_time_ms(lambda: ta(zb, mask), reps, warm=max(20, reps)), 4)
        ref = randomise(factories.triangle_attention(128, 4, starting=True, model="af3", precision="fp32"),
                        seed=0).cuda()
        ref.set_backend("pytorch")
        out["pytorch_gpu_ms_fp32"] = round(event_time_ms(lambda: ref(z, mask), reps, warm=5), 4)
    return out


def trunk_inputs(n: int, seed: int = 0):
    import torch

    g = torch.Generator().manual_seed(seed + 7)
    z = torch.randn(1, n, n, 128, generator=g).bfloat16()
    s = torch.randn(1, n, D_SINGLE, generator=g).bfloat16()
    mask = torch.ones(1, n, dtype=torch.bool)
    return z, s, mask


def time_trunk(model, z, s, mask, runs: int, warmup: int = 1) -> tuple[float, object]:
    """ms per trunk run (TRUNK_PASSES passes over the blocks) between HIP events."""
    import torch

    with torch.no_grad():
        for _ in range(warmup):
            out = model(z, mask, s, passes=TRUNK_PASSES)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(runs):
            out = model(z, mask, s, passes=TRUNK_PASSES)
        end.record()
        end.synchronize()
    return start.elapsed_time(end) / runs, out


def trunk_measure(n: int, runs: int, *, pytorch_too: bool = False, cpu_too: bool = False) -> dict:
    """The 48-block trunk with its single track, every op on hip (guard: error)."""
    import torch

    import foldforge_amd

    model = foldforge_amd.load(backend="miniworld", device="cuda", blocks=TRUNK_BLOCKS, seed=0,
                               d_single=D_SINGLE, unsupported="error")
    z_cpu, s_cpu, mask_cpu = trunk_inputs(n)
    z, s, mask = z_cpu.cuda(), s_cpu.cuda(), mask_cpu.cuda()
    ms, (pair, single) = time_trunk(model, z, s, mask, runs)
    evals = TRUNK_BLOCKS * TRUNK_PASSES
    blk = model.blocks[0]
    with torch.no_grad():
        zb = blk(z, mask)
        apb_ms = event_time_ms(lambda: blk.single_attention(s, zb, mask), 20)
        str_ms = event_time_ms(lambda: blk.single_transition(s), 20)
    rms = lambda t: float(t.float().pow(2).mean().sqrt())  # noqa: E731
    gf = block_gflop(n, D_SINGLE)
    out = {
        "workload": f"48-block Pairformer trunk with single track, N={n}, c_z=128, c_s={D_SINGLE}, "
                    f"APB 16x24, {TRUNK_PASSES} passes ({evals} block evaluations), all-ones mask, "
                    "z, s ~N(0,1), seeded random init (to_out/squeeze x0.25)",
        "n": n, "ms_per_trunk": round(ms, 2), "ms_per_block": round(ms / evals, 4),
        "trunk_tflops": round(gf * evals / ms, 1),
        "single_track_us_per_block": {"attention_pair_bias": round(apb_ms * 1e3, 1),
                                      "single_transition": round(str_ms * 1e3, 1)},
        "final_rms": {"pair": round(rms(pair), 4), "single": round(rms(single), 4)},
        "finite": bool(torch.isfinite(pair.float()).all() and torch.isfinite(single.float()).all()),
    }
    if pytorch_too:
        ref = foldforge_amd.load(backend="pytorch", device="cuda", blocks=TRUNK_BLOCKS, seed=0,
                                 d_single=D_SINGLE)
        ms_ref, (pr, sr) = time_trunk(ref, z, s, mask, 1)
        where = mask[:, :, None] & mask[:, None, :]
        from oracle import pairstack as ps

        out["pytorch_backend"] = {
            "ms_per_trunk": round(ms_ref, 1),
            "hip_speedup": round(ms_ref / ms, 2),
            "hip_vs_pytorch_rel_rms": {"pair": round(ps.rel_rms(pair.cpu().double(), pr.cpu().double(),
                                                                 where.cpu()), 5),
                                       "single": round(ps.rel_rms(single.cpu().double(),
                                                                  sr.cpu().double()), 5)},
        }
        del ref
    if cpu_too:
        from oracle import pairstack as ps

        threads = min(16, os.cpu_count() or 1)
        torch.set_num_threads(threads)
        state = {k[len("blocks.0."):]: v.cpu() for k, v in model.state_dict().items()
                 if k.startswith("blocks.0.")}
        ps.pairformer_block(z_cpu, mask_cpu, state, s=s_cpu)
        t0 = time.perf_counter()
        ps.pairformer_block(z_cpu, mask_cpu, state, s=s_cpu)
        per_block = time.perf_counter() - t0
        out["cpu_baseline"] = {"value": round(per_block * evals, 1), "unit": "s per trunk run",
                               "cores": threads, "kind": "port",
                               "sample": f"one block with single track at N={n} (fp32 oracle, 1 warm-up, "
                                         f"1 timed) x {evals}: an extrapolation"}
    return out


def cpu_baseline_trunk_parity(n: int, evals=(0, 71, 143)) -> dict:
    """The trunk's parity check beside its timing (the fp32 oracle as the checker only).

    The hip trunk of ``trunk_measure`` is run once more, untimed, recording the input and
    output of block evaluations ``evals`` (0-based); the fp32 CPU oracle is run from each
    recorded input and the update's rel-RMS (pair over valid pairs, single over valid tokens)
    is reported against the oracle with the residual stream rounded to bf16 after every op (the
    engine contract: an op returns ``x + f(x)`` in its input dtype; the per-block bar 3e-2), and
    against the oracle with an fp32 stream throughout, beside the engine ``pytorch`` backend's
    bf16 block on the same input (deep in the trunk the stream is large against a block's
    update, so the stream's own bf16 rounding dominates the second comparison for either
    backend). The final state is compared with the fp32 reference trunk (the engine
    ``pytorch`` backend with an fp32 residual stream, same GPU), beside the ``pytorch``
    backend's own bf16 trunk: the rounding floor of a bf16 stream."""
    import torch

    import foldforge_amd
    from oracle import pairstack as ps

    z_cpu, s_cpu, mask_cpu = trunk_inputs(n)
    model = foldforge_amd.load(backend="miniworld", device="cuda", blocks=TRUNK_BLOCKS, seed=0,
                               d_single=D_SINGLE, unsupported="error")
    prev, taken, stream = [z_cpu.cuda(), s_cpu.cuda()], {}, []
    rms = lambda t: round(float(t.float().pow(2).mean().sqrt()), 3)  # noqa: E731

    def observe(p, i, pair, single):
        e = TRUNK_BLOCKS * p + i
        if e in evals:
            taken[e] = (prev[0].cpu(), prev[1].cpu(), pair.cpu(), single.cpu())
        if (e + 1) % 16 == 0:
            stream.append([e + 1, rms(pair), rms(single)])
        prev[0], prev[1] = pair, single

    with torch.no_grad():
        hz, hs = model(z_cpu.cuda(), mask_cpu.cuda(), s_cpu.cuda(), passes=TRUNK_PASSES, on_block=observe)
    hz, hs = hz.cpu().double(), hs.cpu().double()
    state = model.state_dict()
    del model
    prev.clear()
    with torch.no_grad():
        bref = foldforge_amd.load(backend="pytorch", device="cuda", blocks=TRUNK_BLOCKS, seed=0,
                                  d_single=D_SINGLE)
        bblock = {}
        for e in evals:
            zi, si = taken[e][0].cuda(), taken[e][1].cuda()
            bz_e, bs_e = bref.blocks[e % TRUNK_BLOCKS](zi, mask_cpu.cuda(), si)
            bblock[e] = (bz_e.cpu(), bs_e.cpu())
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    where = mask_cpu[:, :, None] & mask_cpu[:, None, :]
    rows = []

    def upd(out, inp, want, on):
        return round(ps.rel_rms(out.double() - inp.double(), want.double() - inp.double(), on), 5)

    for e in evals:
        zi, si, zo, so = taken[e]
        i = e % TRUNK_BLOCKS
        sub = {k[len(f"blocks.{i}."):]: v.cpu() for k, v in state.items() if k.startswith(f"blocks.{i}.")}
        oz, os_ = ps.pairformer_block(zi, mask_cpu, sub, n_head_pair=4, s=si, n_head_single=16,
                                      io_dtype=torch.bfloat16)
        wz, ws = ps.pairformer_block(zi, mask_cpu, sub, n_head_pair=4, s=si, n_head_single=16)
        bz_e, bs_e = bblock[e]
        rows.append({"evaluation": e + 1,
                     "pair_update_rel_rms": upd(zo, zi, oz, where),
                     "single_update_rel_rms": upd(so, si, os_, mask_cpu),
                     "vs_fp32_stream": {"pair": upd(zo, zi, wz, where), "single": upd(so, si, ws, mask_cpu)},
                     "pytorch_backend_bf16": {"pair": upd(bz_e, zi, oz, where), "single": upd(bs_e, si, os_, mask_cpu),
                                              "vs_fp32_stream": {"pair": upd(bz_e, zi, wz, where),
                                                                 "single": upd(bs_e, si, ws, mask_cpu)}}})
    with torch.no_grad():
        ref = foldforge_amd.load(backend="pytorch", device="cuda", blocks=TRUNK_BLOCKS, seed=0,
                                 d_single=D_SINGLE, dtype=torch.float32)
        fz, fs = ref(z_cpu.float().cuda(), mask_cpu.cuda(), s_cpu.float().cuda(), passes=TRUNK_PASSES)
        fz, fs = fz.cpu().double(), fs.cpu().double()
        del ref
        bz, bs = bref(z_cpu.cuda(), mask_cpu.cuda(), s_cpu.cuda(), passes=TRUNK_PASSES)
        bz, bs = bz.cpu().double(), bs.cpu().double()
        del bref
    torch.cuda.empty_cache()
    return {
        "sampled_block_updates_vs_fp32_oracle": rows,
        "stream_rms": {"every_16_evaluations": stream, "columns": ["evaluation", "pair", "single"],
                       "input": [rms(z_cpu), rms(s_cpu)]},
        "final_state_vs_fp32_reference_trunk": {
            "hip": {"pair": round(ps.rel_rms(hz, fz, where), 5), "single": round(ps.rel_rms(hs, fs), 5)},
            "pytorch_backend_bf16": {"pair": round(ps.rel_rms(bz, fz, where), 5),
                                     "single": round(ps.rel_rms(bs, fs), 5)},
        },
        "note": "per-block bar 3e-2 on the update against the oracle with a bf16 residual stream; the "
                "fp32 reference trunk is the engine pytorch backend with an fp32 residual stream on the "
                "same GPU",
    }


def graph_measure(n: int, runs: int = 3) -> dict:
    """The 48 x 3 trunk run eagerly and as one captured graph (foldforge_amd.execution)."""
    import torch

    import foldforge_amd
    from foldforge_amd.execution import capture_trunk

    model = foldforge_amd.load(backend="miniworld", device="cuda", blocks=TRUNK_BLOCKS, seed=0,
                               d_single=D_SINGLE, unsupported="error")
    z_cpu, s_cpu, mask_cpu = trunk_inputs(n)
    z, s, mask = z_cpu.cuda(), s_cpu.cuda(), mask_cpu.cuda()
    eager_ms, (pe, se) = time_trunk(model, z, s, mask, runs)
    graph = capture_trunk(model, z, mask, s, passes=TRUNK_PASSES)
    graph_ms = event_time_ms(lambda: graph(z, mask, s), runs, warm=1)
    pg, sg = graph(z, mask, s)
    torch.cuda.synchronize()
    return {"n": n, "eager_ms_per_trunk": round(eager_ms, 2), "graph_ms_per_trunk": round(graph_ms, 2),
            "graph_speedup": round(eager_ms / graph_ms, 2),
            "graph_equals_eager": bool(torch.equal(pg, pe) and torch.equal(sg, se))}


def msa_measure(reps: int = 20) -> dict:
    """MSA pair-weighted averaging at the reference's op-table shapes: L = 256 / 384 tokens,
    512 MSA rows, AF3 widths (c_m 64, c_z 128, 8 heads x 8), bf16; hip and the engine pytorch
    backend on the same GPU."""
    import torch

    from foldforge_amd import factories
    from foldforge_amd.trunk import randomise

    out = {"workload": "MSA pair-weighted averaging, 512 MSA rows, c_m=64, c_z=128, 8 heads x "
                       "d_head (8: AF3; 32: the reference's op-table cell), all-ones mask, bf16, "
                       "seeded random init", "rows": []}
    depth, cm, heads = 512, 64, 8
    for dh in (8, 32):
        mod = randomise(factories.msa_pair_weighted_averaging(cm, 128, heads, dh), seed=0).cuda()
        hd = heads * dh
        for n in (256, 384):
            g = torch.Generator().manual_seed(n)
            m = torch.randn(1, depth, n, cm, generator=g).bfloat16().cuda()
            z = torch.randn(1, n, n, 128, generator=g).bfloat16().cuda()
            mask = torch.ones(1, n, dtype=torch.bool, device="cuda")
            row = {"n": n, "d_head": dh}
            with torch.no_grad():
                for backend in ("hip", "pytorch"):
                    mod.set_backend(backend)
                    row[f"{backend}_ms"] = round(
                        event_time_ms(lambda: mod(m, z, mask), reps, warm=max(50, reps)), 4)
            gflop = (2 * depth * n * cm * 2 * hd + 2 * n * n * hd * depth + 2 * depth * n * hd * cm
                     + 2 * n * n * 128 * heads) / 1e9
            row["gflop"] = round(gflop, 2)
            row["hip_tflops"] = round(gflop / row["hip_ms"], 1)
            out["rows"].append(row)
    return out


def msa_block_measure(reps: int = 10) -> dict:
    """One AF3 MSA-stack block (outer product mean, MSA pair-weighted averaging 8 x 8, MSA
    transition, the pair track with triangle attention) at L = 256 / 384 tokens, 512 MSA rows,
    every op on hip: ms per block with the MSA track on a second stream beside the pair track
    (the default) and strictly sequential, and the engine pytorch backend on the same GPU."""
    import torch

    from foldforge_amd import dispatch, factories
    from foldforge_amd.trunk import randomise

    out = {"workload": "AF3 MSA-stack block, 512 MSA rows, c_m=64, c_z=128, all-ones masks, bf16, "
                       "seeded random init", "rows": []}
    depth, cm = 512, 64
    block = randomise(factories.msa_block(cm, 128, 4), seed=0).cuda()
    for n in (256, 384):
        g = torch.Generator().manual_seed(n)
        msa = torch.randn(depth, n, cm, generator=g).bfloat16().cuda()
        z = torch.randn(n, n, 128, generator=g).bfloat16().cuda()
        msa_mask = torch.ones(depth, n, device="cuda")
        pair_mask = torch.ones(n, n, device="cuda")
        row = {"n": n}
        with torch.no_grad():
            block.set_backend("hip")
            dispatch.set_refusal(block, "error")
            for overlap, key in ((True, "hip_ms"), (False, "hip_sequential_ms")):
                block.overlap_tracks = overlap
                row[key] = round(event_time_ms(lambda: block(msa, z, msa_mask, pair_mask), reps, warm=reps), 4)
            block.overlap_tracks = True
            block.set_backend("pytorch")
            row["pytorch_ms"] = round(event_time_ms(lambda: block(msa, z, msa_mask, pair_mask), max(2, reps // 5)), 4)
        out["rows"].append(row)
    return out


def opm_measure(reps: int = 20) -> dict:
    """Outer product mean at the reference's op-table shapes: L = 256 / 384 tokens, 512 MSA
    rows, c_m 64, 32 x 32 outer products, c_z 128, AF3 form (n + 1e-3 divisor, bias before
    the divide), 90% of the MSA entries real; hip and the engine pytorch backend."""
    import torch

    from foldforge_amd import factories
    from foldforge_amd.trunk import randomise

    out = {"workload": "outer product mean, 512 MSA rows, c_m=64, hidden 32, c_z=128, AF3 divisor, "
                       "90% of MSA entries real, bf16, seeded random init", "rows": []}
    depth, cm = 512, 64
    mod = randomise(factories.outer_product_mean(cm, 128, 32, count_offset=1e-3,
                                                 normalize_before_proj=False), seed=0).cuda()
    for n in (256, 384):
        g = torch.Generator().manual_seed(n)
        m = torch.randn(1, depth, n, cm, generator=g).bfloat16().cuda()
        rows = (torch.rand(1, depth, n, generator=g) < 0.9).cuda()
        row = {"n": n}
        with torch.no_grad():
            for backend in ("hip", "pytorch"):
                mod.set_backend(backend)
                row[f"{backend}_ms"] = round(
                    event_time_ms(lambda: mod(m, rows), reps, warm=max(50, reps)), 4)
        gflop = (2 * depth * n * n * 32 * 32 + 2 * n * n * 1024 * 128 + 2 * depth * n * cm * 64) / 1e9
        row["gflop"] = round(gflop, 2)
        row["hip_tflops"] = round(gflop / row["hip_ms"], 1)
        out["rows"].append(row)
    # Chai-1's grouped form at its trunk width: 8 groups of 8 channels, product norm, c_z 256
    out["grouped"] = {"workload": "outer product mean (Chai-1), 512 MSA rows, c_m=64, 8 groups of 8, "
                                  "product norm, c_z=256, 90% of MSA entries real, bf16", "rows": []}
    gmod = randomise(factories.outer_product_mean(cm, 256, 64, groups=8), seed=1).cuda()
    for n in (256, 384):
        g = torch.Generator().manual_seed(n + 1)
        m = torch.randn(1, depth, n, cm, generator=g).bfloat16().cuda()
        rows = (torch.rand(1, depth, n, generator=g) < 0.9).cuda()
        row = {"n": n}
        with torch.no_grad():
            for backend in ("hip", "pytorch"):
                gmod.set_backend(backend)
                row[f"{backend}_ms"] = round(
                    event_time_ms(lambda: gmod(m, rows), reps, warm=max(50, reps)), 4)
        gflop = (2 * depth * n * n * 512 + 2 * n * n * 512 * 256 + 2 * depth * n * cm * 128) / 1e9
        row["gflop"] = round(gflop, 2)
        row["hip_tflops"] = round(gflop / row["hip_ms"], 1)
        out["grouped"]["rows"].append(row)
    return out


def shapes_measure(reps: int = 10) -> dict:
    """The same block at its other shapes: the template stacks of AF3 (pair 64, triangle
    attention 4 x 16, hidden 64, transition x 2), Protenix-1 (4 x 32 heads, hidden 128) and
    Boltz-2 (4 x 32 heads, transition x 4), 4 templates batched (``spec.py`` of the reference:
    template heads, head width and hidden width per family), and the confidence head's block
    (pair 128 with the single track, 5 samples batched), all at N = 384; ms per block on hip
    and on the engine pytorch backend (same GPU)."""
    import torch

    from foldforge_amd import dispatch, factories
    from foldforge_amd.trunk import randomise

    n = 384
    out = {"n": n, "rows": []}
    cases = (
        ("template stack block (AF3): pair 64, 4 x 16 heads, hidden 64, transition x2, 4 templates",
         dict(d_pair=64, triangle_model="af3", d_hidden_tri_attention=16, pair_transition_n=2), 4, 64, 0),
        ("template stack block (Protenix-1): pair 64, 4 x 32 heads, hidden 128, transition x2, 4 templates",
         dict(d_pair=64, triangle_model="protenix", d_hidden_tri_attention=32, d_hidden_tri_multi=128,
              pair_transition_n=2), 4, 64, 0),
        ("template stack block (Boltz-2): pair 64, 4 x 32 heads, hidden 64, transition x4, 4 templates",
         dict(d_pair=64, triangle_model="boltz2", d_hidden_tri_attention=32, pair_transition_n=4), 4, 64, 0),
        ("template stack block (RoseTTAFold3): pair 64, 4 x 64 heads, hidden 64, transition x4, 4 templates",
         dict(d_pair=64, triangle_model="rf3", d_hidden_tri_attention=64, pair_transition_n=4), 4, 64, 0),
        ("trunk block (Chai-1): pair 256, 4 x 64 heads, hidden 256, transition x2, batch 1",
         dict(d_pair=256, triangle_model="chai1", d_hidden_tri_attention=64, pair_transition_n=2), 1, 256, 0),
        ("confidence head block (AF3): pair 128 + single 384, 5 samples",
         dict(d_pair=128, triangle_model="af3", d_single=384), 5, 128, 384),
    )
    for name, kwargs, batch, c, cs in cases:
        block = randomise(factories.pairformer_block(**kwargs), seed=1, out_scale=0.25).cuda()
        g = torch.Generator(device="cuda").manual_seed(2)
        z = torch.randn(batch, n, n, c, device="cuda", generator=g).bfloat16()
        mask = torch.ones(batch, n, dtype=torch.bool, device="cuda")
        s = torch.randn(batch, n, cs, device="cuda", generator=g).bfloat16() if cs else None
        args = (z, mask) if s is None else (z, mask, s)
        row = {"workload": name, "batch": batch}
        with torch.no_grad():
            for backend in ("hip", "pytorch"):
                block.set_backend(backend)
                dispatch.set_refusal(block, "error" if backend == "hip" else None)
                row[f"{backend}_ms"] = round(event_time_ms(lambda: block(*args), reps, warm=max(20, reps)), 3)
        row["hip_speedup"] = round(row["pytorch_ms"] / row["hip_ms"], 2)
        out["rows"].append(row)
        del block, z, s
        torch.cuda.empty_cache()
    return out


def ladder(max_n: int) -> list[dict]:
    """Config 5: full trunks at N = 768 .. 2048, then single blocks (with single track) at
    larger N until the device runs out of memory."""
    import torch

    import foldforge_amd

    lines = []
    for n in (768, 1024, 1536, 2048):
        torch.cuda.empty_cache()
        lines.append(trunk_measure(n, 1))
        print(json.dumps({"ladder": lines[-1]}), flush=True)
    model = foldforge_amd.load(backend="miniworld", device="cuda", blocks=1, seed=0,
                               d_single=D_SINGLE, unsupported="error")
    blk = model.blocks[0]
    for n in (3072, 4096, 6144, 8192, 10240, 12288, 16384):
        if n > max_n:
            break
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats()
        try:
            # drawn on the device: the fp32 draw of z alone would need 4 N^2 128 bytes of host memory
            g = torch.Generator(device="cuda").manual_seed(7)
            z = torch.randn(1, n, n, 128, device="cuda", generator=g, dtype=torch.bfloat16)
            s = torch.randn(1, n, D_SINGLE, device="cuda", generator=g, dtype=torch.bfloat16)
            mask = torch.ones(1, n, dtype=torch.bool, device="cuda")
            with torch.no_grad():
                blk(z, mask, s)
                torch.cuda.synchronize()
                ms = event_time_ms(lambda: blk(z, mask, s), 1)
            peak = torch.cuda.max_memory_allocated() / 2**30
            row = {"n": n, "ms_per_block": round(ms, 2),
                   "block_tflops": round(block_gflop(n, D_SINGLE) / ms, 1),
                   "ms_per_trunk_extrapolated": round(ms * TRUNK_BLOCKS * TRUNK_PASSES, 1),
                   "peak_gib": round(peak, 1)}
        except torch.cuda.OutOfMemoryError as exc:
            row = {"n": n, "out_of_memory": str(exc).splitlines()[0][:160]}
        lines.append(row)
        print(json.dumps({"ladder": row}), flush=True)
        z = s = mask = None
        if "out_of_memory" in row:
            break
    return lines


def _cpu_ops(z, mask, state, runs: int) -> tuple[dict, float, object]:
    """The fp32 oracle's block on the CPU, op by op: median ms of each op over ``runs`` runs
    after one warm-up, the median block ms, and the block's output."""
    from oracle import pairstack as ps

    sub = lambda prefix: ps.sub_params(state, prefix)  # noqa: E731
    steps = (
        ("trimul_outgoing", lambda x: ps.triangle_multiplication(x, mask, sub("tri_multi_outgoing"), outgoing=True)),
        ("trimul_incoming", lambda x: ps.triangle_multiplication(x, mask, sub("tri_multi_incoming"), outgoing=False)),
        ("triattn_starting", lambda x: ps.triangle_attention(x, mask, sub("tri_atten_starting"), starting=True, n_head=4)),
        ("triattn_ending", lambda x: ps.triangle_attention(x, mask, sub("tri_atten_ending"), starting=False, n_head=4)),
        ("transition", lambda x: ps.transition(x, sub("transition_pair"))),
    )
    times: dict[str, list[float]] = {name: [] for name, _ in steps}
    blocks, out = [], None
    for r in range(runs + 1):
        x = z.float()
        t_block = time.perf_counter()
        for name, fn in steps:
            t0 = time.perf_counter()
            x = fn(x)
            if r:
                times[name].append(time.perf_counter() - t0)
        if r:
            blocks.append(time.perf_counter() - t_block)
        out = x
    ops = {name: round(statistics.median(t) * 1e3, 1) for name, t in times.items()}
    return ops, statistics.median(blocks) * 1e3, out


def cpu_model() -> str:
    import platform

    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(z, mask, state, gpu_out, runs: int, small: dict | None = None) -> dict:
    """The fp32 CPU oracle on the host's cores (at most 16 threads, the box's CPU share):
    the timed workload's block op by op, the N = 384 block (``small``: z, mask, state) op by op,
    and the single triangle-attention op at z [1, 128, 128, 128] (the reference's CPU case)."""
    import torch

    from oracle import pairstack as ps

    threads = min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    ops, block_ms, out = _cpu_ops(z, mask, state, runs)
    where = mask[:, :, None] & mask[:, None, :]
    rr = ps.rel_rms(gpu_out.double() - z.double(), out.double() - z.double(), where)
    result = {"value": round(block_ms, 1), "unit": "ms per block",
              "cores": threads, "kind": "port",
              "cores_note": f"capped at 16 threads: the host's CPU share for one GPU (os.cpu_count() = "
                            f"{os.cpu_count()} counts the whole host, shared with the other GPUs' jobs)",
              "sample": f"the full timed workload: one block at N={z.shape[1]}, fp32, oracle/pairstack.py, "
                        f"op by op, median of {runs} after 1 warm-up; {threads} threads of {cpu_model()}",
              "ops_ms": ops, "gpu_vs_cpu_update_rel_rms": round(rr, 5)}
    if small is not None:
        ops384, block384, _ = _cpu_ops(small["z"], small["mask"], small["state"], runs)
        result["n384"] = {"ms_per_block": round(block384, 1), "ops_ms": ops384}
    # the single triangle-attention op (starting node) on z [1, 128, 128, 128] fp32, 4 x 32 heads,
    # all-ones mask, seed 0 (the reference's CPU-runnable case)
    from foldforge_amd import factories
    from foldforge_amd.trunk import randomise

    ta = randomise(factories.triangle_attention(128, 4, starting=True, model="af3", precision="fp32"), seed=0)
    params = {k: v.float() for k, v in ta.state_dict().items()}
    z1 = torch.randn(1, 128, 128, 128, generator=torch.Generator().manual_seed(0))
    m1 = torch.ones(1, 128, dtype=torch.bool)
    ps.triangle_attention(z1, m1, params, starting=True, n_head=4)
    times = []
    for _ in range(max(3, runs)):
        t0 = time.perf_counter()
        ps.triangle_attention(z1, m1, params, starting=True, n_head=4)
        times.append(time.perf_counter() - t0)
    result["triattn_op_n128_fp32_ms"] = round(statistics.median(times) * 1e3, 2)
    return result


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the pair stack's "
              "multi-GPU sharding is a design note, not part of this build", file=sys.stderr)
        return 2
    import torch

    from foldforge_amd import dispatch, factories
    from foldforge_amd.trunk import randomise

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    if args.ladder:
        ladder(args.ladder_max)
        return 0
    if args.shapes:
        print(json.dumps({"shapes": shapes_measure(args.steps)}), flush=True)
        return 0
    if args.msa:
        print(json.dumps({"msa": msa_measure(args.steps), "opm": opm_measure(args.steps),
                          "msa_block": msa_block_measure(max(5, args.steps // 2))}), flush=True)
        return 0
    if args.trunk_only:
        trunk = trunk_measure(512, max(1, args.steps // 10), pytorch_too=not args.no_reference_backend,
                              cpu_too=not args.no_cpu_baseline)
        if not args.no_graph:
            trunk["graph"] = [graph_measure(n) for n in (128, 512)]
        print(json.dumps({"trunk": trunk}), flush=True)
        return 0
    dev = torch.device("cuda:0")
    n = args.n
    length = real_length(n, args.seed)
    g = torch.Generator().manual_seed(args.seed)
    z_cpu = torch.randn(1, n, n, 128, generator=g).bfloat16()
    mask_cpu = torch.ones(1, n, dtype=torch.bool)
    mask_cpu[0, length:] = False
    block = randomise(factories.pairformer_block(d_pair=128, triangle_model="af3"), seed=args.seed).to(dev)
    block.set_backend("hip")
    dispatch.set_refusal(block, "error")  # a refused call would raise instead of running torch ops
    z, mask = z_cpu.to(dev), mask_cpu.to(dev)

    with torch.no_grad():
        t_warm = time.perf_counter()
        for _ in range(args.warmup):
            out = block(z, mask)
        torch.cuda.synchronize()
        settle_steps = 0
        while (time.perf_counter() - t_warm) * 1e3 < args.settle_ms:
            for _ in range(10):
                out = block(z, mask)
            settle_steps += 10
            torch.cuda.synchronize()
        settle_ms = (time.perf_counter() - t_warm) * 1e3
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        start.record()
        for _ in range(args.steps):
            out = block(z, mask)
        end.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    ms_per_step = start.elapsed_time(end) / args.steps
    hip_calls = dispatch.served_count(block, "hip")
    print(f"timed {args.steps} steps: {ms_per_step:.3f} ms/step (wall {wall * 1e3 / args.steps:.3f}); "
          f"hip op calls {hip_calls}", file=sys.stderr, flush=True)

    per_op = op_times(block, z, mask, length, args.kernel_reps)
    g384 = torch.Generator().manual_seed(args.seed + 1)
    z384_cpu = torch.randn(1, 384, 384, 128, generator=g384).bfloat16()
    mask384_cpu = torch.ones(1, 384, dtype=torch.bool)
    block384 = randomise(factories.pairformer_block(d_pair=128, triangle_model="af3"), seed=args.seed + 1).to(dev)
    block384.set_backend("hip")
    dispatch.set_refusal(block384, "error")
    per_op_384 = op_times(block384, z384_cpu.to(dev), mask384_cpu.to(dev), 384, args.kernel_reps)
    per_op_384["reference_h100_engine_cuda_ms"] = REFERENCE_H100_MS_384
    per_op_128 = single_op_n128(args.kernel_reps)
    print(f"N=384 block {per_op_384['ms_per_block']} ms; ops " +
          ", ".join(f"{k} {v['ms']}" for k, v in per_op_384["ops"].items()), file=sys.stderr, flush=True)

    roof = flash_roofline(n, length, args.kernel_reps)
    if not args.no_logit_regimes:
        roof["logit_regimes"] = flash_logit_regimes(n, args.kernel_reps)
        print("flash logit regimes: " + "; ".join(
            f"q x{r['q_scale']} {r['us_per_launch']} us (rescaled {r['rows_rescaled_frac']})"
            for r in roof["logit_regimes"]), file=sys.stderr, flush=True)
    ln = layernorm_roofline(n, args.kernel_reps)
    print(f"flash core {roof['us_per_launch']} us {roof['achieved']} TFLOP/s; "
          f"layernorm {ln['us_per_launch']} us {ln['achieved']} GB/s", file=sys.stderr, flush=True)
    gpu_out = out.cpu()
    copy = copy_reference(args.copy_reference_mb) if args.copy_reference_mb > 0 else None

    base = None
    if not args.no_cpu_baseline:
        small = {"z": z384_cpu, "mask": mask384_cpu,
                 "state": {k: v.cpu() for k, v in block384.state_dict().items()}}
        base = cpu_baseline(z_cpu, mask_cpu, {k: v.cpu() for k, v in block.state_dict().items()},
                            gpu_out, args.cpu_runs, small)
        print(f"cpu baseline {base['value']} ms/block on {base['cores']} threads", file=sys.stderr, flush=True)

    gflop = block_gflop(n)
    gflop_run = sum(op_gflop(n, key_extent(n, length)).values())
    trunk = None
    ladder_rows = None
    if not args.no_trunk:
        trunk = trunk_measure(512, 2)
        print(f"trunk {trunk['ms_per_trunk']} ms ({trunk['ms_per_block']} ms/block)", file=sys.stderr,
              flush=True)
        if not args.no_cpu_baseline:
            trunk["parity"] = cpu_baseline_trunk_parity(512)
            print(f"trunk parity {json.dumps(trunk['parity'])}", file=sys.stderr, flush=True)
        ladder_rows = []
        for ln_ in (768, 1024, 1536, 2048):
            torch.cuda.empty_cache()
            row = trunk_measure(ln_, 1)
            ladder_rows.append({k: row[k] for k in ("n", "ms_per_trunk", "ms_per_block", "trunk_tflops", "finite")})
            print(f"ladder N={ln_}: trunk {row['ms_per_trunk']} ms", file=sys.stderr, flush=True)
    shapes = None
    if not args.no_shapes:
        torch.cuda.empty_cache()
        shapes = shapes_measure(10)
        print("shapes: " + "; ".join(f"{r['workload'].split(':')[0]} {r['hip_ms']} ms" for r in shapes["rows"]),
              file=sys.stderr, flush=True)
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
            "block_gflop_executed": round(gflop_run, 1),
            "block_tflops_executed": round(gflop_run / ms_per_step, 1),
            "key_extent_executed": key_extent(n, length),
            "clock_settle": {"untimed_steps_after_warmup": settle_steps, "ms": round(settle_ms, 1)},
        },
        "roofline": roof,
        "kernels": {"layer_norm": ln, **({"copy_reference": copy} if copy else {})},
        "cpu_baseline": base,
        "ops": {"n512_ragged": per_op, "n384": per_op_384, "n128_single_triattn_op": per_op_128},
        "trunk": trunk,
        "ladder": ladder_rows,
        "shapes": shapes,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
