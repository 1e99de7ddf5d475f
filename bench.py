#!/usr/bin/env python3
"""Benchmark: the fused per-layer ops of one ACE-Step DiT block on MI355X.

Workload (the metric's configuration): DiT block, bf16 activations, hidden
2048, T=6000 latent frames x batch 2 (CFG pair) = 12000 rows, 16 Q / 8 KV
heads x 128 (NEOX rope, theta 1e4, frame-index positions), SwiGLU at
intermediate 6144. One step = the block's fused-op launches in
dit_ggml_build_layer order (reference dit-graph.h:367-448), captured once
into a HIP graph and replayed:
  norm_sa        = rms_norm*w -> AdaLN modulate (hidden)
  q, k           = QK-norm -> rope on views of the fused QKV projection output
  h1, norm_ffn   = hidden + sa_out * gate_sa, and rms_norm*w -> AdaLN of it
                   (one pass: the gated residual fused into the FFN norm)
  ff             = swiglu(gate_up)
  h2             = h1 + ffn_out * gate_ffn
The same block with the residual and the norm as separate launches (six
launches, the op-per-node structure of the reference graph) is timed too and
reported under "unfused".
The GEMM / attention outputs between them (qkv, sa_out, gate_up, ffn_out)
are synthetic N(0,1) bf16 tensors resident in HBM before timing starts.

value = algorithmic bytes of the step's launches / measured step time (GB/s);
algorithmic bytes count every input read once and every output written
once at its storage type (bf16 activations, f32 vectors).

cpu_baseline: the CPU oracle (a restatement of the ggml-cpu arithmetic)
running the reference's unfused F32 node graph for the same block on a row
sample, OpenMP over rows, threads = logical CPUs / 2 (the reference's
backend policy) capped by the job's CPU share.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "hbd-acestep.cpp_amd"))

H, NH, NKV, D, I_FF = 2048, 16, 8, 128, 6144
T_FRAMES, BATCH = 6000, 2
ROWS = T_FRAMES * BATCH
THETA, EPS = 1e4, 1e-6
HBM_PEAK_GBS = 8000.0


def block_bytes(rows: int, es: int = 2, fused: bool = True) -> dict:
    """Algorithmic bytes per launch (inputs read once + outputs written once)."""
    act = rows * H * es
    vec = H * 4
    qk = rows * (NH + NKV) * D * es
    b = {
        "rms_norm_modulate_sa": 2 * act + 3 * vec,
        "qk_norm_rope": 2 * qk + rows * 4 + 2 * D * 4,
    }
    if fused:
        # h1 = h + sa_out * gate_sa and norm_ffn = AdaLN(rms_norm(h1) * w) in one pass
        b["add_rms_norm_modulate_ffn"] = 4 * act + 4 * vec
    else:
        b["gated_add_sa"] = 3 * act + vec
        b["rms_norm_modulate_ffn"] = 2 * act + 3 * vec
    b["swiglu"] = rows * 2 * I_FF * es + rows * I_FF * es
    b["gated_add_ffn"] = 3 * act + vec
    return b


def bf16_bits(a: np.ndarray) -> np.ndarray:
    u = a.astype(np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _setup():
    """Synthetic block inputs resident in HBM, and the fused / unfused launch lists."""
    from acestep_ops import device, ops
    from acestep_ops.device import DTensor, Stream

    rng = np.random.default_rng(42)

    def dev_bf16(shape):
        return DTensor.from_numpy(bf16_bits(rng.standard_normal(shape, dtype=np.float32)), "bf16")

    def dev_f32(shape, scale=1.0, mean=0.0):
        return DTensor.from_numpy((rng.standard_normal(shape, dtype=np.float32) * scale + mean).astype(np.float32))

    hidden = dev_bf16((BATCH, T_FRAMES, H))
    qkv = dev_bf16((ROWS, (NH + 2 * NKV) * D))
    sa_out = dev_bf16((BATCH, T_FRAMES, H))
    gate_up = dev_bf16((BATCH, T_FRAMES, 2 * I_FF))
    ffn_out = dev_bf16((BATCH, T_FRAMES, H))
    adaln = dev_f32((6 * H,), 0.1)
    sa_w, ff_w = dev_f32((H,), 0.1, 1.0), dev_f32((H,), 0.1, 1.0)
    q_w, k_w = dev_f32((D,), 0.1, 1.0), dev_f32((D,), 0.1, 1.0)
    pos = DTensor.from_numpy(np.tile(np.arange(T_FRAMES, dtype=np.int32), BATCH))
    shift_sa, scale_sa, gate_sa, shift_ff, scale_ff, gate_ff = (adaln[i * H:(i + 1) * H] for i in range(6))
    q = qkv[:, :NH * D].unflatten(1, (NH, D))
    k = qkv[:, NH * D:(NH + NKV) * D].unflatten(1, (NKV, D))
    norm_sa = DTensor.empty((BATCH, T_FRAMES, H), "bf16")
    norm_ff = DTensor.empty((BATCH, T_FRAMES, H), "bf16")
    h1 = DTensor.empty((BATCH, T_FRAMES, H), "bf16")
    h2 = DTensor.empty((BATCH, T_FRAMES, H), "bf16")
    q_out = DTensor.empty((ROWS, NH, D), "bf16")
    k_out = DTensor.empty((ROWS, NKV, D), "bf16")
    ff = DTensor.empty((BATCH, T_FRAMES, I_FF), "bf16")
    stream = Stream()
    sh = stream.handle
    device.synchronize()

    fused = [
        lambda: ops.rms_norm_modulate(hidden, sa_w, scale_sa, shift_sa, EPS, out=norm_sa, stream=sh),
        lambda: ops.qk_norm_rope(q, q_w, pos, EPS, D, THETA, k=k, k_w=k_w, q_out=q_out, k_out=k_out, stream=sh),
        lambda: ops.add_rms_norm(hidden, sa_out, EPS, gate=gate_sa, w=ff_w, scale=scale_ff, shift=shift_ff,
                                 out_sum=h1, out_norm=norm_ff, stream=sh),
        lambda: ops.swiglu(gate_up, out=ff, stream=sh),
        lambda: ops.gated_add(h1, ffn_out, gate_ff, out=h2, stream=sh),
    ]
    unfused = [
        fused[0], fused[1],
        lambda: ops.gated_add(hidden, sa_out, gate_sa, out=h1, stream=sh),
        lambda: ops.rms_norm_modulate(h1, ff_w, scale_ff, shift_ff, EPS, out=norm_ff, stream=sh),
        fused[3], fused[4],
    ]
    # plain bf16 copy of a known size (the SwiGLU output, 147.456 MB each way):
    # the reference point for scaling the FETCH_SIZE / WRITE_SIZE counters
    ff_copy = DTensor.empty((BATCH, T_FRAMES, I_FF), "bf16")
    calib = lambda: ops.cpy(ff, ff_copy, stream=sh)  # noqa: E731
    keep = (hidden, qkv, sa_out, gate_up, ffn_out, adaln, sa_w, ff_w, q_w, k_w, pos, norm_sa, norm_ff, h1, h2, q_out,
            k_out, ff, ff_copy)
    return fused, unfused, calib, stream, keep


def pmc_pass():
    """Each fused launch once, then the calibration copy, eagerly (for rocprofv3 --pmc)."""
    from acestep_ops import device

    fused, _, calib, stream, _keep = _setup()
    for f in fused:
        f()
    calib()
    stream.synchronize()
    device.synchronize()
    print("pmc pass: 5 block launches + 1 calibration copy (bf16, 147456000 B read, 147456000 B written)",
          flush=True)


def gpu_bench(steps: int, warmup: int):
    from acestep_ops import device
    from acestep_ops.device import Event, Graph

    fused, unfused, _calib, stream, _keep = _setup()
    sh = stream.handle

    def graph_of(launches):
        g = Graph()
        with g.capture(stream):
            for f in launches:
                f()
        return g

    def time_graph(g, n):
        a, b = Event(), Event()
        stream.synchronize()
        a.record(sh)
        for _ in range(n):
            g.launch()
        b.record(sh)
        b.synchronize()
        return a.elapsed_ms(b) / n

    def per_kernel(launches, n, g_ahead):
        """Per-launch device time inside the block sequence. Each sample first
        queues 8 replays of the block graph (about 1.6 ms of device work) so the
        host has enqueued every event and launch of the sample before the
        device reaches them: the event pairs then bracket only the kernel."""
        ev = [[Event() for _ in range(len(launches) + 1)] for _ in range(n)]
        stream.synchronize()
        for i in range(n):
            for _ in range(8):
                g_ahead.launch()
            ev[i][0].record(sh)
            for j, f in enumerate(launches):
                f()
                ev[i][j + 1].record(sh)
        stream.synchronize()
        return [1000.0 * float(np.mean([ev[i][j].elapsed_ms(ev[i][j + 1]) for i in range(n)]))
                for j in range(len(launches))]

    g_fused, g_unfused = graph_of(fused), graph_of(unfused)
    for _ in range(warmup):
        g_fused.launch()
        g_unfused.launch()
    stream.synchronize()

    # timed region: K graph replays of the fused block
    device.synchronize()
    t0 = time.perf_counter()
    ms_step = time_graph(g_fused, steps)
    device.synchronize()
    wall = time.perf_counter() - t0
    ms_unfused = time_graph(g_unfused, steps)

    names_f = list(block_bytes(ROWS, fused=True).keys())
    names_u = list(block_bytes(ROWS, fused=False).keys())
    pk_f = dict(zip(names_f, per_kernel(fused, steps, g_fused)))
    pk_u = dict(zip(names_u, per_kernel(unfused, steps, g_unfused)))
    return ms_step, ms_unfused, wall, pk_f, pk_u


def cpu_bench(rows: int, reps: int, threads: int):
    """The reference's unfused F32 node graph for one DiT block on `rows` rows."""
    from oracle import oracle as orc

    orc.set_threads(threads)
    rng = np.random.default_rng(7)
    x = rng.standard_normal((rows, H), dtype=np.float32)
    qkv = rng.standard_normal((rows, (NH + 2 * NKV) * D), dtype=np.float32)
    q = np.ascontiguousarray(qkv[:, :NH * D].reshape(rows, NH, D))   # ggml_cont of the views
    k = np.ascontiguousarray(qkv[:, NH * D:(NH + NKV) * D].reshape(rows, NKV, D))
    sa_out = rng.standard_normal((rows, H), dtype=np.float32)
    gu = rng.standard_normal((rows, 2 * I_FF), dtype=np.float32)
    ffn_out = rng.standard_normal((rows, H), dtype=np.float32)
    ad = (rng.standard_normal(6 * H, dtype=np.float32) * 0.1).astype(np.float32)
    w1 = (rng.standard_normal(H, dtype=np.float32) * 0.1 + 1).astype(np.float32)
    w2 = w1.copy()
    qw = (rng.standard_normal(D, dtype=np.float32) * 0.1 + 1).astype(np.float32)
    kw = qw.copy()
    pos = np.arange(rows, dtype=np.int32) % T_FRAMES

    def block():
        n = orc.rms_norm_modulate(x, w1, ad[H:2 * H], ad[:H], EPS)
        qo = orc.qk_norm_rope(q, qw, pos, EPS, D, THETA)
        ko = orc.qk_norm_rope(k, kw, pos, EPS, D, THETA)
        h1 = orc.gated_add(x, sa_out, ad[2 * H:3 * H])
        n2 = orc.rms_norm_modulate(h1, w2, ad[4 * H:5 * H], ad[3 * H:4 * H], EPS)
        f = orc.swiglu(gu)
        h2 = orc.gated_add(h1, ffn_out, ad[5 * H:6 * H])
        return n, qo, ko, n2, f, h2

    for _ in range(3):
        block()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        block()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts)), float(np.sum(ts))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-rows", type=int, default=1500, help="row sample for the CPU baseline")
    ap.add_argument("--cpu-reps", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="launch each block kernel once plus a copy of known size, for counter collection")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); every op of the path is "
              "row-parallel and shards by rows with no communication, so per-GPU throughput is the N=1 figure.",
              file=sys.stderr)
        sys.exit(2)
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: one process / one GPU only", file=sys.stderr)
        sys.exit(2)

    if args.pmc_pass:
        pmc_pass()
        return
    kb = block_bytes(ROWS, fused=True)
    kb_u = block_bytes(ROWS, fused=False)
    total_bytes = sum(kb.values())
    ms_step, ms_unfused, wall, per_k, per_k_u = gpu_bench(args.steps, args.warmup)
    value = total_bytes / (ms_step * 1e-3) / 1e9
    dom = "swiglu"
    dom_gbs = kb[dom] / (per_k[dom] * 1e-6) / 1e9

    # HBM bytes per launch of the dominant kernel from the committed counter
    # summary (FETCH_SIZE and WRITE_SIZE, each scaled by a copy of known size)
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "dit_block_T6000_traffic.md")
    if os.path.exists(tpath):
        for line in open(tpath):
            if line.startswith("traffic_bytes_per_launch k_swiglu:"):
                traffic = int(line.split(":", 1)[1].strip())

    cpu = None
    if not args.no_cpu:
        threads = max(1, min((os.cpu_count() or 2) // 2, int(os.environ.get("OMP_NUM_THREADS", "16"))))
        med, spent = cpu_bench(args.cpu_rows, args.cpu_reps, threads)
        scale = ROWS / args.cpu_rows
        cpu_block_s = med * scale
        cpu = {
            "value": round(total_bytes / cpu_block_s / 1e9, 3),
            "unit": "GB/s",
            "cores": threads,
            "kind": "port",
            "us_per_block": round(cpu_block_s * 1e6, 1),
            "sample": (f"reference's unfused F32 ggml node graph of one DiT block (rms_norm, mul, add, rope, swiglu "
                       f"nodes) on {args.cpu_rows} of {ROWS} rows, median of {args.cpu_reps} reps after 3 warm-ups "
                       f"({spent:.1f} s of CPU work), scaled x{scale:.1f} to the full block; GB/s uses the same "
                       f"bf16 byte accounting as value"),
        }

    line = {
        "metric": "fused-op HBM GB/s (% of ~8 TB/s peak) + µs per DiT block at T=6000, 1 GPU",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "us_per_block": round(ms_step * 1e3, 2),
        "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "ACE-Step DiT block fused ops, bf16, H=2048, T=6000 x N=2 (12000 rows), 16/8 heads "
                               "x 128, SwiGLU I=6144; 5 launches/step (gated residual fused into the FFN norm), "
                               "replayed as one HIP graph",
                   "rows": ROWS, "hidden": H, "intermediate": I_FF, "bytes_per_step": total_bytes},
        "per_kernel_us": {k: round(v, 2) for k, v in per_k.items()},
        "per_kernel_gbs": {k: round(kb[k] / (per_k[k] * 1e-6) / 1e9, 1) for k in kb},
        "unfused": {"us_per_block": round(ms_unfused * 1e3, 2), "bytes_per_step": sum(kb_u.values()),
                    "gbs": round(sum(kb_u.values()) / (ms_unfused * 1e-3) / 1e9, 1),
                    "per_kernel_us": {k: round(v, 2) for k, v in per_k_u.items()}},
        "roofline": {"bound": "hbm", "achieved": round(dom_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom_gbs / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": "k_swiglu (bf16)",
                     "bytes_per_launch": kb[dom]},
        "cpu_baseline": cpu,
        "wall_s": round(wall, 4),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
