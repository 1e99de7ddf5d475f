#!/usr/bin/env python3
"""Benchmark: the fused per-layer ops of one ACE-Step DiT block on MI355X.

Workload (the metric's configuration): DiT block, bf16 activations, hidden
2048, T=6000 latent frames x batch 2 (CFG pair) = 12000 rows, 16 Q / 8 KV
heads x 128 (NEOX rope, theta 1e4, frame-index positions), SwiGLU at
intermediate 6144. One step = one block's fused-op launches in
dit_ggml_build_layer order (reference dit-graph.h:367-448). K steps are timed
as one replay of a HIP graph holding K consecutive blocks, as a DiT step runs
its blocks back to back in one graph (dit-graph.h:498-590, the layer loop).
A block's first op, the self-attention norm, reads the previous block's last
output with no GEMM in between, so it runs fused into the previous block's
last launch; the graph starts with one standalone norm for the first block:
  [first block only] hidden_norm = rms_norm*w -> AdaLN modulate (hidden)
  q, k           = QK-norm -> rope on views of the fused QKV projection output
  h1, norm_ffn   = hidden + sa_out * gate_sa, and rms_norm*w -> AdaLN of it
                   (one pass: the gated residual fused into the FFN norm)
  ff             = swiglu(gate_up)
  hidden, norm_sa = h1 + ffn_out * gate_ffn, and the next block's
                   rms_norm*w -> AdaLN of it (one pass)
The timed graph holds the first-block norm and K blocks of 4 launches; value
counts its bytes. Two comparisons are timed too: the block as 5 launches with
its own norm ("five_launch_block", no fusion across blocks), and as 6 launches,
the op-per-node structure of the reference graph ("unfused").
The GEMM / attention outputs between them (qkv, sa_out, gate_up, ffn_out)
are synthetic N(0,1) bf16 tensors resident in HBM before timing starts.

value = algorithmic bytes of the step's launches / measured step time (GB/s);
algorithmic bytes count every input read once and every output written
once at its storage type (bf16 activations, f32 vectors).

cpu_baseline: the CPU oracle (a restatement of the ggml-cpu arithmetic)
running the reference's unfused F32 node graph for the same block on a row
sample, OpenMP over rows, threads = logical CPUs / 2 (the reference's
backend policy) capped by the job's CPU share, built for the host's x86-64
level (AVX-512 when present); a second run uses every CPU of the job's
share. The host's CPU model, sockets, physical cores and logical CPUs are
recorded from lscpu.
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


def block_bytes(rows: int, es: int = 2, fused: bool = True, cross: bool = False) -> dict:
    """Algorithmic bytes per launch (inputs read once + outputs written once).
    cross: the steady-state block of a block sequence, whose last launch also
    makes the next block's self-attention norm (the first block's norm is
    lead_bytes)."""
    act = rows * H * es
    vec = H * 4
    qk = rows * (NH + NKV) * D * es
    b = {} if cross else {"rms_norm_modulate_sa": 2 * act + 3 * vec}
    b["qk_norm_rope"] = 2 * qk + rows * 4 + 2 * D * 4
    if fused:
        # h1 = h + sa_out * gate_sa and norm_ffn = AdaLN(rms_norm(h1) * w) in one pass
        b["add_rms_norm_modulate_ffn"] = 4 * act + 4 * vec
    else:
        b["gated_add_sa"] = 3 * act + vec
        b["rms_norm_modulate_ffn"] = 2 * act + 3 * vec
    b["swiglu"] = rows * 2 * I_FF * es + rows * I_FF * es
    if cross:
        b["gated_add_ffn_rms_norm_modulate_sa"] = 4 * act + 4 * vec
    else:
        b["gated_add_ffn"] = 3 * act + vec
    return b


def block_bytes_ca(rows: int, es: int = 2) -> dict:
    """Algorithmic bytes per launch of the steady-state block with the
    reference's cross-attention extras (dit-graph.h:428-433): the self-attention
    gated residual fused with the cross-attention RMSNorm*w, the per-head
    cross-attention Q-norm (328-331), and the cross-attention residual add fused
    with the FFN norm -> AdaLN."""
    act = rows * H * es
    vec = H * 4
    qk = rows * (NH + NKV) * D * es
    return {
        "qk_norm_rope": 2 * qk + rows * 4 + 2 * D * 4,
        "gated_add_sa_rms_norm_ca": 4 * act + 2 * vec,
        "rms_norm_ca_q": 2 * rows * NH * D * es + D * 4,
        "add_ca_rms_norm_modulate_ffn": 4 * act + 3 * vec,
        "swiglu": rows * 2 * I_FF * es + rows * I_FF * es,
        "gated_add_ffn_rms_norm_modulate_sa": 4 * act + 4 * vec,
    }


# the block with the reference's cross-attention extras as separate nodes
# (norm, Q-norm and residual add on top of the 6-launch block): its bytes and
# the time they take at 70 % of the HBM peak
CA_REF_BYTES = 1425.53e6
CA_REF_US_AT_70 = 254.6


def lead_bytes(rows: int, es: int = 2) -> int:
    """The first block's standalone self-attention norm."""
    return 2 * rows * H * es + 3 * H * 4


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
    # cross attention: its query projection and output (synthetic, resident),
    # the norm weights, and the normalized outputs
    ca_q = dev_bf16((ROWS, NH, D))
    ca_out = dev_bf16((BATCH, T_FRAMES, H))
    ca_w, ca_q_w = dev_f32((H,), 0.1, 1.0), dev_f32((D,), 0.1, 1.0)
    norm_ca = DTensor.empty((BATCH, T_FRAMES, H), "bf16")
    ca_q_out = DTensor.empty((ROWS, NH, D), "bf16")
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
    # the steady-state block of a sequence: the FFN gated residual writes the
    # next block's input (hidden, in place) and that block's self-attention
    # norm (its weights and AdaLN vectors stand in for the next block's)
    cross = [
        fused[1], fused[2], fused[3],
        lambda: ops.add_rms_norm(h1, ffn_out, EPS, gate=gate_ff, w=sa_w, scale=scale_sa, shift=shift_sa,
                                 out_sum=hidden, out_norm=norm_sa, stream=sh),
    ]
    # the steady-state block with cross attention (chain.cpp's use_cross_attn
    # branch, in the same launch order)
    cross_ca = [
        fused[1],
        lambda: ops.add_rms_norm(hidden, sa_out, EPS, gate=gate_sa, w=ca_w, out_sum=h1, out_norm=norm_ca, stream=sh),
        lambda: ops.rms_norm(ca_q, EPS, w=ca_q_w, out=ca_q_out, stream=sh),
        lambda: ops.add_rms_norm(h1, ca_out, EPS, w=ff_w, scale=scale_ff, shift=shift_ff, out_sum=h2,
                                 out_norm=norm_ff, stream=sh),
        fused[3],
        lambda: ops.add_rms_norm(h2, ffn_out, EPS, gate=gate_ff, w=sa_w, scale=scale_sa, shift=shift_sa,
                                 out_sum=hidden, out_norm=norm_sa, stream=sh),
    ]
    lead = fused[0]
    # plain bf16 copy of a known size (the SwiGLU output, 147.456 MB each way):
    # the reference point for scaling the FETCH_SIZE / WRITE_SIZE counters
    ff_copy = DTensor.empty((BATCH, T_FRAMES, I_FF), "bf16")
    calib = lambda: ops.cpy(ff, ff_copy, stream=sh)  # noqa: E731
    keep = (hidden, qkv, sa_out, gate_up, ffn_out, adaln, sa_w, ff_w, q_w, k_w, pos, norm_sa, norm_ff, h1, h2, q_out,
            k_out, ff, ff_copy, ca_q, ca_out, ca_w, ca_q_w, norm_ca, ca_q_out)
    return fused, unfused, cross, cross_ca, lead, calib, stream, keep


def pmc_pass():
    """Each fused launch once (the 5-launch block, then the cross-block
    residual + norm), then the calibration copy, eagerly (for rocprofv3 --pmc)."""
    from acestep_ops import device

    fused, _, cross, _cross_ca, _lead, calib, stream, _keep = _setup()
    for f in fused:
        f()
    cross[-1]()
    calib()
    stream.synchronize()
    device.synchronize()
    print("pmc pass: 5 block launches + the cross-block residual and norm + 1 calibration copy (bf16, 147456000 B "
          "read, 147456000 B written)", flush=True)


def pmc_pass_configs():
    """The C4 and C5 layers' QK-norm/rope, Q8_0 get_rows, Q8_0 KV store and
    dequant-back launched once each, eagerly, then the same calibration copy as
    pmc_pass (for rocprofv3 --pmc)."""
    from acestep_ops import device, ops
    from acestep_ops.device import DTensor, Stream

    gens = list(_qwen3_configs())
    for idx in (2, 3):  # C4, C5
        c = gens[idx]()
        for label, f in c["launches"]:
            if label in ("get_rows_q8_0", "kv_store_q8_0", "get_rows_kv_back", "qk_norm_rope"):
                f()
        c["stream"].synchronize()
        del c
        device.synchronize()
    st = Stream()
    a, b = DTensor.empty((BATCH, T_FRAMES, I_FF), "bf16"), DTensor.empty((BATCH, T_FRAMES, I_FF), "bf16")
    ops.cpy(a, b, stream=st.handle)
    st.synchronize()
    print("pmc pass (configs): C4 and C5 QK-norm/rope, get_rows, KV store, dequant back + 1 calibration copy "
          "(bf16, 147456000 B read, 147456000 B written)", flush=True)


def gpu_bench(steps: int, warmup: int):
    from acestep_ops import device
    from acestep_ops.device import Event, Graph

    fused, unfused, cross, cross_ca, lead, _calib, stream, _keep = _setup()
    sh = stream.handle

    def graph_of(launches, copies=1, first=None):
        """One HIP graph holding `copies` consecutive blocks (a DiT step runs its
        blocks back to back in one graph, so the ~11 us cost of launching a
        graph is paid once per graph, not once per block), after `first`."""
        g = Graph()
        with g.capture(stream):
            if first is not None:
                first()
            for _ in range(copies):
                for f in launches:
                    f()
        return g

    def time_steps(launches, n, first=None):
        """Device time of exactly n blocks (and `first`): one replay of an
        n-block graph, divided by n."""
        g = graph_of(launches, n, first)
        g.launch()  # first replay pays one-time costs
        stream.synchronize()
        a, b = Event(), Event()
        a.record(sh)
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

    g_cross, g_fused, g_unfused, g_ca = graph_of(cross), graph_of(fused), graph_of(unfused), graph_of(cross_ca)
    if warmup:
        graph_of(cross, warmup, lead).launch()
        graph_of(fused, warmup).launch()
        graph_of(unfused, warmup).launch()
        graph_of(cross_ca, warmup).launch()
    stream.synchronize()

    # timed region: the first block's norm and K blocks, one replay of that graph
    device.synchronize()
    t0 = time.perf_counter()
    ms_step = time_steps(cross, steps, lead)
    device.synchronize()
    wall = time.perf_counter() - t0
    ms_five = time_steps(fused, steps)
    ms_unfused = time_steps(unfused, steps)
    ms_ca = time_steps(cross_ca, steps)

    names_c = list(block_bytes(ROWS, cross=True).keys())
    names_f = list(block_bytes(ROWS, fused=True).keys())
    names_u = list(block_bytes(ROWS, fused=False).keys())
    pk_c = dict(zip(names_c, per_kernel(cross, steps, g_cross)))
    pk_f = dict(zip(names_f, per_kernel(fused, steps, g_fused)))
    pk_u = dict(zip(names_u, per_kernel(unfused, steps, g_unfused)))
    pk_ca = dict(zip(list(block_bytes_ca(ROWS).keys()), per_kernel(cross_ca, steps, g_ca)))
    return ms_step, ms_five, ms_unfused, wall, pk_c, pk_f, pk_u, (ms_ca, pk_ca)


def host_cpu() -> dict:
    """The host's CPU as lscpu reports it, the CPUs this job may run on, and the
    x86-64 level of the oracle build the CPU baseline loads (v4 with AVX-512)."""
    info = {}
    try:
        import subprocess

        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            info[k.strip()] = v.strip()
    except Exception:  # noqa: BLE001 -- lscpu is optional; /proc/cpuinfo covers the flags
        pass
    flags = set()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("flags"):
                flags = set(line.split(":", 1)[1].split())
                break
    except OSError:
        pass
    as_int = lambda k: int(info[k]) if info.get(k, "").isdigit() else None  # noqa: E731
    sockets, cps, tpc = as_int("Socket(s)"), as_int("Core(s) per socket"), as_int("Thread(s) per core")
    logical = os.cpu_count() or 1
    share = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else logical
    omp = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    job = min(share, omp) if omp > 0 else share
    v4 = {"avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"} <= flags
    return {"cpu_model": info.get("Model name", "unknown"), "sockets": sockets,
            "physical_cores": sockets * cps if sockets and cps else None, "threads_per_core": tpc,
            "logical_cpus": logical, "job_cpus": job, "isa": "x86-64-v4" if v4 else "x86-64-v3"}


def cpu_bench(rows: int, reps: int, threads: int, isa: str = "x86-64-v3"):
    """The reference's unfused F32 node graph for one DiT block on `rows` rows."""
    from oracle import oracle as orc

    if orc._lib is None:
        orc.use_isa("v4" if isa == "x86-64-v4" else "v3")
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


# ---------------------------------------------------------------------------
# The Qwen3 configurations (reported with --configs; the JSON line above stays
# the DiT block metric). Each is one layer's fused-op chain in
# qw3lm_forward_batch order (reference qwen3-lm.h:626-741), synthetic N(0,1)
# inputs resident in HBM; `steps` consecutive layers are captured in one HIP
# graph and timed as one replay.
# ---------------------------------------------------------------------------
Q8_ROW = lambda n: n // 32 * 34  # noqa: E731


def _qwen3_configs():
    from acestep_ops import device, ops
    from acestep_ops.device import DTensor

    rng = np.random.default_rng(42)
    H2D = 3  # hipMemcpyDeviceToDevice

    def dev(shape, dt="f32", scale=1.0, mean=0.0):
        a = (rng.standard_normal(shape, dtype=np.float32) * scale + mean).astype(np.float32)
        return DTensor.from_numpy(bf16_bits(a), "bf16") if dt == "bf16" else DTensor.from_numpy(a)

    def q8_table(n_rows, n, stream):
        """Q8_0 table of N(0, 0.02) rows: a 4096-row block quantized on the device
        with the REF quantizer (as GGUF tables are made), repeated to n_rows."""
        seed_rows = min(4096, n_rows)
        src = dev((seed_rows, n), scale=0.02)
        tab = DTensor.empty((n_rows, Q8_ROW(n)), "u8")
        ops.cpy(src, ops.Q8(tab[:seed_rows]), rounding=1, stream=stream.handle)
        for r0 in range(seed_rows, n_rows, seed_rows):
            nb = min(seed_rows, n_rows - r0) * Q8_ROW(n)
            device.check(device.hip().hipMemcpyAsync(tab.ptr + r0 * Q8_ROW(n), tab.ptr, nb, H2D, stream.handle),
                         "hipMemcpyAsync")
        stream.synchronize()
        return tab

    def layer(name, dt, T, H, NH_, NKV_, I, *, clamp=False, emb_rows=0, kv=None, split_glu=False, theta=1e6,
              pos=None, fuse_kv=False):
        """Launch list + algorithmic bytes for one Qwen3 layer at one shape."""
        from acestep_ops.device import Stream

        st = Stream()
        sh = st.handle
        es = 2 if dt == "bf16" else 4
        W = (NH_ + 2 * NKV_) * D
        if clamp:
            # 0.1 % outliers ~ N(0, 1000) and 16 values at +-1e5, so the FP16 clamp fires
            a = rng.standard_normal((T, H), dtype=np.float32)
            o = rng.choice(a.size, a.size // 1000, replace=False)
            a.reshape(-1)[o] = rng.standard_normal(o.size, dtype=np.float32) * 1000
            a.reshape(-1)[rng.choice(a.size, 16, replace=False)] = 1e5
            h = DTensor.from_numpy(a)
        else:
            h = dev((T, H), dt)
        attn, mlp = dev((T, H), dt), dev((T, H), dt)
        w_in, w_post = dev((H,), scale=0.1, mean=1.0), dev((H,), scale=0.1, mean=1.0)
        qw, kw = dev((D,), scale=0.1, mean=1.0), dev((D,), scale=0.1, mean=1.0)
        qkv = dev((T, W), dt)
        q = qkv[:, :NH_ * D].unflatten(1, (NH_, D))
        k = qkv[:, NH_ * D:(NH_ + NKV_) * D].unflatten(1, (NKV_, D))
        p = DTensor.from_numpy(np.asarray(pos if pos is not None else np.arange(T), np.int32))
        norm, norm2, h1, h2 = (DTensor.empty((T, H), dt) for _ in range(4))
        q_out, k_out = DTensor.empty((T, NH_, D), dt), DTensor.empty((T, NKV_, D), dt)
        if split_glu:
            g_, u_ = dev((T, I), dt), dev((T, I), dt)
        else:
            gu = dev((T, 2 * I), dt)
        ff = DTensor.empty((T, I), dt)
        act = T * H * es
        L, B = [], {}

        def add(label, fn, nbytes):
            L.append((label, fn))
            B[label] = nbytes

        keep = [h, attn, mlp, w_in, w_post, qw, kw, qkv, p, norm, norm2, h1, h2, q_out, k_out, ff, st]
        if emb_rows:
            tab = q8_table(emb_rows, H, st)
            ids = DTensor.from_numpy(rng.integers(0, emb_rows, T).astype(np.int32))
            emb = DTensor.empty((T, H), "f32")
            keep += [tab, ids, emb]
            add("get_rows_q8_0", lambda: ops.get_rows(ops.Q8(tab), ids, out=emb, stream=sh),
                T * Q8_ROW(H) + T * 4 + T * H * 4)
        add("rms_norm", lambda: ops.rms_norm(h, EPS, w_in, out=norm, stream=sh), 2 * act + H * 4)
        if not fuse_kv:
            add("qk_norm_rope", lambda: ops.qk_norm_rope(q, qw, p, EPS, D, theta, k=k, k_w=kw, q_out=q_out,
                                                         k_out=k_out, stream=sh),
                2 * T * (NH_ + NKV_) * D * es + T * 4 + 2 * D * 4)
        if kv is not None:
            n_seq, T_seq, max_seq, s0 = kv
            kc = DTensor.zeros((n_seq, NKV_, max_seq, Q8_ROW(D)), "u8")
            vc = DTensor.zeros((n_seq, NKV_, max_seq, Q8_ROW(D)), "u8")
            kk = k_out.view(n_seq, T_seq, NKV_, D)
            vv = qkv.view(n_seq, T_seq, W)[:, :, (NH_ + NKV_) * D:].unflatten(2, (NKV_, D))
            p0 = DTensor.from_numpy(np.asarray(s0, np.int32))
            keep += [kc, vc, p0]
            n_kv = n_seq * T_seq * NKV_ * D
            if fuse_kv:
                # QK-norm -> rope, and K/V straight into the Q8_0 caches: one launch
                vf = qkv[:, (NH_ + NKV_) * D:].unflatten(1, (NKV_, D))
                add("qk_norm_rope_kv_store_q8_0",
                    lambda: ops.qk_norm_rope_kv_store(q, qw, k, kw, vf, p, EPS, D, theta, ops.Q8(kc), ops.Q8(vc), p0,
                                                      q_out=q_out, stream=sh),
                    2 * T * NH_ * D * es + 2 * (n_kv * es + n_kv // 32 * 34) + T * 4 + n_seq * 4 + 2 * D * 4)
            else:
                add("kv_store_q8_0", lambda: ops.kv_store(kk, ops.Q8(kc), p0, v=vv, v_cache=ops.Q8(vc), stream=sh),
                    2 * (n_kv * es + n_kv // 32 * 34) + n_seq * 4)
            if T_seq > 1:
                # dequantize the written K and V rows back (get_rows on the caches viewed as row tables)
                rows = (np.arange(n_seq)[:, None, None] * NKV_ + np.arange(NKV_)[None, None, :]) * max_seq + \
                    (np.asarray(s0)[:, None, None] + np.arange(T_seq)[None, :, None])
                rid = DTensor.from_numpy(rows.reshape(-1).astype(np.int32))
                kt, vt = kc.view(n_seq * NKV_ * max_seq, Q8_ROW(D)), vc.view(n_seq * NKV_ * max_seq, Q8_ROW(D))
                kb, vb = DTensor.empty((rows.size, D), "f32"), DTensor.empty((rows.size, D), "f32")
                keep += [rid, kb, vb]
                add("get_rows_kv_back", lambda: (ops.get_rows(ops.Q8(kt), rid, out=kb, stream=sh),
                                                 ops.get_rows(ops.Q8(vt), rid, out=vb, stream=sh)),
                    2 * (rows.size * Q8_ROW(D) + rows.size * 4 + rows.size * D * 4))
        clamp_lim = (-65504.0, 65504.0) if clamp else None
        add("add_rms_norm", lambda: ops.add_rms_norm(h, attn, EPS, w=w_post, clamp=clamp_lim, out_sum=h1,
                                                     out_norm=norm2, stream=sh), 4 * act + H * 4)
        if split_glu:
            keep += [g_, u_]
            add("swiglu", lambda: ops.swiglu_split(g_, u_, out=ff, stream=sh), 3 * T * I * es)
        else:
            keep += [gu]
            add("swiglu", lambda: ops.swiglu(gu, out=ff, stream=sh), 3 * T * I * es)
        if clamp:
            add("add_clamp", lambda: ops.add_clamp(h1, mlp, out=h2, stream=sh), 3 * act)
        else:
            add("add", lambda: ops.add(h1, mlp, out=h2, stream=sh), 3 * act)
        return dict(name=name, launches=L, bytes=B, stream=st, keep=keep)

    r = np.random.default_rng(7)
    yield lambda: layer("C1 Qwen3-0.6B layer, fp32, T=512 (split SwiGLU, Q8_0 embedding 151669x1024)", "f32", 512,
                        1024, 16, 8, 3072, emb_rows=151669, split_glu=True)
    dpos = r.integers(0, 8192, 8)
    yield lambda: layer("C2 Qwen3-4B decode layer, bf16, batch 8 (QK-norm/rope fused with the Q8_0 KV store, "
                        "8192 slots)", "bf16", 8, 2560, 32, 8, 9728, kv=(8, 1, 8192, dpos), pos=dpos, fuse_kv=True)
    yield lambda: layer("C4 Qwen3-1.7B prefill layer, fp32, 4x4096 (clamp, Q8_0 embedding 151669x2048)", "f32",
                        16384, 2048, 16, 8, 6144, clamp=True, emb_rows=151669)
    s0 = r.integers(0, 6144, 8)
    ppos = (s0[:, None] + np.arange(2048)[None, :]).reshape(-1)
    yield lambda: layer("C5 Qwen3-4B prefill layer, fp32, 8x2048 (Q8_0 KV store at slots U[0,6144), dequant back)",
                        "f32", 16384, 2560, 32, 8, 9728, kv=(8, 2048, 8192, s0), pos=ppos)


def configs_bench(steps: int, warmup: int, emit: bool = True) -> list:
    """Per Qwen3 configuration: µs per layer (one replay of a graph of `steps`
    consecutive layers), and per op two timings that bracket the kernel's own
    duration:
      us      HIP event pairs around its launch inside the layer sequence; they
              include ~2.5-3 us of event and dispatch time per launch (most of
              the figure for the decode-sized ops);
      us_b2b  one replay of a graph of `steps` back-to-back launches of the op
              alone, per launch; no event time, but a repeated launch can
              re-read inputs that fit the 256 MB last-level cache.
    GB/s and frac use `us` (the conservative one), GB/s_b2b and frac_b2b
    us_b2b. One JSON line each when `emit`."""
    from acestep_ops import device
    from acestep_ops.device import Event, Graph

    out = []
    for key, make in zip(("C1", "C2", "C4", "C5"), _qwen3_configs()):
        c = make()
        st, sh = c["stream"], c["stream"].handle
        fns = [f for _, f in c["launches"]]
        # `steps` consecutive layers in one graph (a model runs its layers back
        # to back), replayed once after a warm-up replay
        g = Graph()
        with g.capture(st):
            for _ in range(steps):
                for f in fns:
                    f()
        g.launch()
        st.synchronize()
        a, b = Event(), Event()
        a.record(sh)
        g.launch()
        b.record(sh)
        b.synchronize()
        us_layer = 1000.0 * a.elapsed_ms(b) / steps
        g1 = Graph()
        with g1.capture(st):
            for f in fns:
                f()
        ev = [[Event() for _ in range(len(fns) + 1)] for _ in range(steps)]
        for i in range(steps):
            for _ in range(4):
                g1.launch()
            ev[i][0].record(sh)
            for j, f in enumerate(fns):
                f()
                ev[i][j + 1].record(sh)
        st.synchronize()
        per = {}
        for j, (label, f) in enumerate(c["launches"]):
            us = 1000.0 * float(np.mean([ev[i][j].elapsed_ms(ev[i][j + 1]) for i in range(steps)]))
            gb = Graph()
            with gb.capture(st):
                for _ in range(steps):
                    f()
            gb.launch()
            st.synchronize()
            a.record(sh)
            gb.launch()
            b.record(sh)
            b.synchronize()
            us_b2b = 1000.0 * a.elapsed_ms(b) / steps
            gbs = c["bytes"][label] / (us * 1e-6) / 1e9
            gbs_b = c["bytes"][label] / (us_b2b * 1e-6) / 1e9
            per[label] = {"us": round(us, 2), "us_b2b": round(us_b2b, 2), "MB": round(c["bytes"][label] / 1e6, 3),
                          "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 3),
                          "GB/s_b2b": round(gbs_b, 1), "frac_b2b": round(gbs_b / HBM_PEAK_GBS, 3)}
            del gb
        tot = sum(c["bytes"].values())
        r = {"key": key, "config": c["name"], "us_per_layer": round(us_layer, 2), "launches": len(fns),
             "bytes_per_layer": tot, "GB/s": round(tot / (us_layer * 1e-6) / 1e9, 1),
             "frac": round(tot / (us_layer * 1e-6) / 1e9 / HBM_PEAK_GBS, 3), "per_op": per}
        out.append(r)
        if emit:
            print(json.dumps(r), flush=True)
        del c, g, g1
        device.synchronize()
    return out


# ---------------------------------------------------------------------------
# Attention (reported with --attention): ggml_flash_attn_ext over the KV cache
# at the Qwen3-4B batch-8 decode shape (reference qwen3-lm.h:706-723): one
# query row per sequence, 32/8 heads x 128, an 8192-slot cache per sequence,
# sequence lengths U[1, 8192], the read length rounded up to 256 and the
# tail masked (qwen3-lm.h:582-596).
# ---------------------------------------------------------------------------
def attention_bench(steps: int):
    from acestep_ops import device, ops
    from acestep_ops.device import DTensor, Event, Graph, Stream

    N, NH_, NKV_, Dh, SLOTS = 8, 32, 8, 128, 8192
    rng = np.random.default_rng(11)
    lens = rng.integers(1, SLOTS + 1, N)
    read = min(SLOTS, int((lens.max() + 255) // 256 * 256))
    st = Stream()
    sh = st.handle
    q = DTensor.from_numpy(bf16_bits(rng.standard_normal((N, NH_, 1, Dh), dtype=np.float32)), "bf16")
    m = np.zeros((N, 1, 1, read), np.float32)
    for b, L in enumerate(lens):
        m[b, 0, 0, L:] = -np.inf
    mask = DTensor.from_numpy(m.astype(np.float16).view(np.uint16), "f16")
    y = DTensor.empty((N, 1, NH_, Dh), "f32")
    for kt in ("q8_0", "f16"):
        caches = []
        for _ in range(2):  # K, V
            src = DTensor.from_numpy(rng.standard_normal((N, NKV_, SLOTS, Dh), dtype=np.float32))
            if kt == "q8_0":
                c = DTensor.empty((N, NKV_, SLOTS, Q8_ROW(Dh)), "u8")
                ops.cpy(src, ops.Q8(c), stream=sh)
                caches.append(ops.Q8(c[:, :, :read]))
            else:
                c = DTensor.empty((N, NKV_, SLOTS, Dh), "f16")
                ops.cpy(src, c, stream=sh)
                caches.append(c[:, :, :read])
            st.synchronize()
            del src
        kc, vc = caches
        need = ops.flash_attn_workspace(q, kc, vc)
        ws = DTensor.empty((max(need, 1),), "u8")
        call = lambda: ops.flash_attn_ext(q, kc, vc, mask, 1.0 / float(np.sqrt(Dh)), out=y, workspace=ws,  # noqa
                                          stream=sh)
        call()
        st.synchronize()
        g = Graph()
        with g.capture(st):
            for _ in range(steps):
                call()
        g.launch()
        st.synchronize()
        a, b_ = Event(), Event()
        a.record(sh)
        g.launch()
        b_.record(sh)
        b_.synchronize()
        us = 1000.0 * a.elapsed_ms(b_) / steps
        row = Q8_ROW(Dh) if kt == "q8_0" else 2 * Dh
        kv_bytes = int(lens.sum()) * NKV_ * 2 * row
        alg = kv_bytes + N * read * 2 + N * NH_ * Dh * 2 + N * NH_ * Dh * 4
        gbs = alg / (us * 1e-6) / 1e9
        print(json.dumps({"config": f"C2 decode attention, Qwen3-4B batch 8, 32/8 heads x 128, {kt} KV cache of "
                                    f"{SLOTS} slots, lengths U[1,{SLOTS}] (sum {int(lens.sum())}), read length "
                                    f"{read}",
                          "us_per_call": round(us, 2), "launches": 2 if need else 1, "bytes_per_call": alg,
                          "kv_bytes": kv_bytes, "workspace_bytes": need, "GB/s": round(gbs, 1),
                          "frac": round(gbs / HBM_PEAK_GBS, 3)}), flush=True)
        del g, caches, kc, vc, ws
        device.synchronize()

    # DiT self-attention (dit-graph.h:227-231): S = T / patch_size rows per CFG
    # element (dit-graph.h:475; S=3000 for T=6000 frames at patch size 2, and
    # S=6000), x 2, 16/8 heads x 128, bf16 operands read as the block produces
    # them (q, k from the QK-norm/rope outputs, v a view of the QKV projection
    # rows), the F16 padding mask (all zero: no padding, the full-attention
    # layers) or none
    NB, NHD, NKVD = 2, 16, 8
    for S in (3000, 6000):
        qd = DTensor.from_numpy(bf16_bits(rng.standard_normal((NB * S, NHD, Dh), dtype=np.float32)), "bf16")
        kd = DTensor.from_numpy(bf16_bits(rng.standard_normal((NB * S, NKVD, Dh), dtype=np.float32)), "bf16")
        qkv = DTensor.from_numpy(bf16_bits(rng.standard_normal((NB * S, (NHD + 2 * NKVD) * Dh), dtype=np.float32)),
                                 "bf16")
        qv = qd.view(NB, S, NHD, Dh).permute(0, 2, 1, 3)
        kv = kd.view(NB, S, NKVD, Dh).permute(0, 2, 1, 3)
        vv = qkv.view(NB, S, NHD + 2 * NKVD, Dh)[:, :, NHD + NKVD:].permute(0, 2, 1, 3)
        yd = DTensor.empty((NB, S, NHD, Dh), "f32")
        zmask = DTensor.zeros((NB, 1, S, S), "f16")
        # the sliding-window layers' mask (dit-sampler.h:253-274, every even
        # layer, dit.h:399): |qi - ki| <= 128, no padding
        win = 128
        ii = np.arange(S)[:, None]
        wm = np.where(np.abs(ii - np.arange(S)[None, :]) <= win, 0.0, -np.inf).astype(np.float16)
        wmask = DTensor.from_numpy(np.ascontiguousarray(np.broadcast_to(wm, (NB, 1, S, S))).view(np.uint16), "f16")
        live = float(np.isfinite(wm).sum())  # (query, key) pairs the window keeps
        del wm, ii
        flops = 4.0 * S * S * Dh * NHD * NB
        wsd = DTensor.empty((max(ops.flash_attn_workspace(qv, kv, vv), 1),), "u8")
        for label, mk in ((f"F16 sliding-window mask (window {win})", wmask), ("F16 padding mask (all zero)", zmask),
                          ("no mask", None)):
            call = lambda: ops.flash_attn_ext(qv, kv, vv, mk, 1.0 / float(np.sqrt(Dh)), out=yd,  # noqa
                                              workspace=wsd, stream=sh)
            # 30 untimed calls first: the first series after the uploads above runs
            # ~10 % slow (measured: 992 us, then 890 us for the same S=6000 call
            # after another 20 calls), whichever case comes first
            for _ in range(30):
                call()
            st.synchronize()
            ev = [Event() for _ in range(steps + 1)]
            ev[0].record(sh)
            for i in range(steps):
                call()
                ev[i + 1].record(sh)
            st.synchronize()
            us = 1000.0 * ev[0].elapsed_ms(ev[steps]) / steps
            tf = flops / (us * 1e-6) / 1e12
            rec = {"config": f"DiT self-attention, bf16 q/k/v views, S={S} x {NB}, {NHD}/{NKVD} heads x {Dh}, {label}",
                   "us_per_call": round(us, 2), "TFLOP/s": round(tf, 1), "flop_per_call": flops,
                   "frac_of_bf16_dense": round(tf / 2500.0, 3)}
            if mk is wmask:
                # the window keeps `live` of the S*S pairs: rate and fraction on the
                # live pairs' flops (the dense figures would exceed the peak)
                lf = 4.0 * live * Dh * NHD * NB
                rec = {"config": rec["config"], "us_per_call": rec["us_per_call"],
                       "live_pairs_frac": round(live / (S * S), 4), "live_flop_per_call": lf,
                       "TFLOP/s": round(lf / (us * 1e-6) / 1e12, 1),
                       "frac_of_bf16_dense": round(lf / (us * 1e-6) / 1e12 / 2500.0, 3)}
            print(json.dumps(rec), flush=True)
        del qd, kd, qkv, qv, kv, vv, yd, zmask, wmask, wsd
        device.synchronize()

    # DiT cross attention (dit-graph.h:296-351): q from the S=3000 latent rows of
    # each CFG element, K/V from the condition encoder's enc_S rows (F16 casts),
    # 16/8 heads x 128, the F16 mask [enc_S, S] blocking the encoder's padding
    # (the last 40 positions here); flops count the live (query, key) pairs
    S, ENC = 3000, 512
    qc = DTensor.from_numpy(rng.standard_normal((NB, S, NHD, Dh), dtype=np.float32))
    qcv = qc.permute(0, 2, 1, 3)
    kc_ = DTensor.from_numpy(rng.standard_normal((NB, NKVD, ENC, Dh), dtype=np.float32).astype(np.float16).view(
        np.uint16), "f16")
    vc_ = DTensor.from_numpy(rng.standard_normal((NB, NKVD, ENC, Dh), dtype=np.float32).astype(np.float16).view(
        np.uint16), "f16")
    pm = np.zeros((NB, 1, S, ENC), np.float16)
    pm[..., ENC - 40:] = -np.inf
    pmask = DTensor.from_numpy(pm.view(np.uint16), "f16")
    yc = DTensor.empty((NB, S, NHD, Dh), "f32")
    wsc = DTensor.empty((max(ops.flash_attn_workspace(qcv, kc_, vc_), 1),), "u8")
    call = lambda: ops.flash_attn_ext(qcv, kc_, vc_, pmask, 1.0 / float(np.sqrt(Dh)), out=yc,  # noqa
                                      workspace=wsc, stream=sh)
    for _ in range(10):
        call()
    st.synchronize()
    ev = [Event() for _ in range(steps + 1)]
    ev[0].record(sh)
    for i in range(steps):
        call()
        ev[i + 1].record(sh)
    st.synchronize()
    us = 1000.0 * ev[0].elapsed_ms(ev[steps]) / steps
    lf = 4.0 * NB * NHD * S * (ENC - 40) * Dh
    print(json.dumps({"config": f"DiT cross attention, F32 q view S={S} x {NB}, {NHD}/{NKVD} heads x {Dh}, F16 K/V of "
                                f"{ENC} encoder rows, F16 padding mask (last 40 masked)",
                      "us_per_call": round(us, 2), "live_flop_per_call": lf,
                      "TFLOP/s": round(lf / (us * 1e-6) / 1e12, 1),
                      "frac_of_bf16_dense": round(lf / (us * 1e-6) / 1e12 / 2500.0, 3)}), flush=True)
    del qc, qcv, kc_, vc_, pmask, yc, wsc
    device.synchronize()

    # LM prefill attention over the KV cache (qw3lm_forward, qwen3-lm.h:429-549;
    # the songgen LM reads an F16 or a Q8_0 cache, songgen-lelm-gen.h:50-61):
    # Qwen3-4B 32/8 heads x 128, 8 sequences x 2048 new tokens from slot 0 of
    # an 8192-slot cache (the batched prefill's shape), F32 q as the rope output,
    # the causal F16 mask [kv_len, S] shared by the heads; flops count the
    # causal (query, key) pairs
    NP, SP, NHP, NKP = 8, 2048, 32, 8
    qp = DTensor.from_numpy(rng.standard_normal((NP, SP, NHP, Dh), dtype=np.float32))
    qpv = qp.permute(0, 2, 1, 3)
    ii = np.arange(SP)[:, None]
    cm = np.where(np.arange(SP)[None, :] <= ii, 0.0, -np.inf).astype(np.float16)
    cmask = DTensor.from_numpy(np.ascontiguousarray(np.broadcast_to(cm, (NP, 1, SP, SP))).view(np.uint16), "f16")
    del cm, ii
    yp = DTensor.empty((NP, SP, NHP, Dh), "f32")
    live = NP * NHP * SP * (SP + 1) / 2
    for kt in ("q8_0", "f16"):
        caches = []
        for _ in range(2):  # K, V
            src = DTensor.from_numpy(rng.standard_normal((NP, NKP, SP, Dh), dtype=np.float32))
            if kt == "q8_0":
                c = DTensor.empty((NP, NKP, SLOTS, Q8_ROW(Dh)), "u8")
                ops.cpy(src, ops.Q8(c[:, :, :SP]), stream=sh)
                caches.append(ops.Q8(c[:, :, :SP]))
            else:
                c = DTensor.empty((NP, NKP, SLOTS, Dh), "f16")
                ops.cpy(src, c[:, :, :SP], stream=sh)
                caches.append(c[:, :, :SP])
            st.synchronize()
            del src
        kc, vc = caches
        wsp = DTensor.empty((max(ops.flash_attn_workspace(qpv, kc, vc), 1),), "u8")
        call = lambda: ops.flash_attn_ext(qpv, kc, vc, cmask, 1.0 / float(np.sqrt(Dh)), out=yp,  # noqa
                                          workspace=wsp, stream=sh)
        for _ in range(10):
            call()
        st.synchronize()
        ev = [Event() for _ in range(steps + 1)]
        ev[0].record(sh)
        for i in range(steps):
            call()
            ev[i + 1].record(sh)
        st.synchronize()
        us = 1000.0 * ev[0].elapsed_ms(ev[steps]) / steps
        lf = 4.0 * live * Dh
        print(json.dumps({"config": f"Qwen3-4B prefill attention, {NP} x {SP} tokens from slot 0, {NHP}/{NKP} heads x "
                                    f"{Dh}, F32 q, causal F16 mask, {kt} KV cache of {SLOTS} slots",
                          "us_per_call": round(us, 2), "live_flop_per_call": lf,
                          "TFLOP/s": round(lf / (us * 1e-6) / 1e12, 1),
                          "frac_of_bf16_dense": round(lf / (us * 1e-6) / 1e12 / 2500.0, 3)}), flush=True)
        del caches, kc, vc, wsp
        device.synchronize()
    del qp, qpv, cmask, yp
    device.synchronize()

# ---------------------------------------------------------------------------
# Each kernel of the steady-state C3 block alone (reported with --kernels): a
# graph of `steps` back-to-back launches cycling over 4 sets of its operands
# (every set a fresh allocation, 4 x 147-442 MB, so no launch finds its inputs
# in the 256 MB Infinity Cache), the same calls and shapes as the block.
# ---------------------------------------------------------------------------
def kernels_bench(steps: int):
    from acestep_ops import device, ops
    from acestep_ops.device import DTensor, Event, Graph, Stream

    rng = np.random.default_rng(5)
    NS = 4

    def dev_bf16(shape):
        return DTensor.from_numpy(bf16_bits(rng.standard_normal(shape, dtype=np.float32)), "bf16")

    def dev_f32(shape, scale=1.0, mean=0.0):
        return DTensor.from_numpy((rng.standard_normal(shape, dtype=np.float32) * scale + mean).astype(np.float32))

    st = Stream()
    sh = st.handle
    adaln = dev_f32((6 * H,), 0.1)
    shift_sa, scale_sa, gate_sa, shift_ff, scale_ff, gate_ff = (adaln[i * H:(i + 1) * H] for i in range(6))
    sa_w, ff_w = dev_f32((H,), 0.1, 1.0), dev_f32((H,), 0.1, 1.0)
    q_w, k_w = dev_f32((D,), 0.1, 1.0), dev_f32((D,), 0.1, 1.0)
    pos = DTensor.from_numpy(np.tile(np.arange(T_FRAMES, dtype=np.int32), BATCH))
    kb = block_bytes(ROWS, cross=True)

    def qk_set():
        qkv = dev_bf16((ROWS, (NH + 2 * NKV) * D))
        q = qkv[:, :NH * D].unflatten(1, (NH, D))
        k = qkv[:, NH * D:(NH + NKV) * D].unflatten(1, (NKV, D))
        qo, ko = DTensor.empty((ROWS, NH, D), "bf16"), DTensor.empty((ROWS, NKV, D), "bf16")
        return (qkv, qo, ko), lambda: ops.qk_norm_rope(q, q_w, pos, EPS, D, THETA, k=k, k_w=k_w, q_out=qo,
                                                        k_out=ko, stream=sh)

    def ffn_norm_set():
        h, sa = dev_bf16((BATCH, T_FRAMES, H)), dev_bf16((BATCH, T_FRAMES, H))
        h1, nf = DTensor.empty((BATCH, T_FRAMES, H), "bf16"), DTensor.empty((BATCH, T_FRAMES, H), "bf16")
        return (h, sa, h1, nf), lambda: ops.add_rms_norm(h, sa, EPS, gate=gate_sa, w=ff_w, scale=scale_ff,
                                                         shift=shift_ff, out_sum=h1, out_norm=nf, stream=sh)

    def swiglu_set():
        gu = dev_bf16((BATCH, T_FRAMES, 2 * I_FF))
        ff = DTensor.empty((BATCH, T_FRAMES, I_FF), "bf16")
        return (gu, ff), lambda: ops.swiglu(gu, out=ff, stream=sh)

    def sa_norm_set():
        h1, fo = dev_bf16((BATCH, T_FRAMES, H)), dev_bf16((BATCH, T_FRAMES, H))
        hn, ns = DTensor.empty((BATCH, T_FRAMES, H), "bf16"), DTensor.empty((BATCH, T_FRAMES, H), "bf16")
        return (h1, fo, hn, ns), lambda: ops.add_rms_norm(h1, fo, EPS, gate=gate_ff, w=sa_w, scale=scale_sa,
                                                          shift=shift_sa, out_sum=hn, out_norm=ns, stream=sh)

    for name, make in (("qk_norm_rope", qk_set), ("add_rms_norm_modulate_ffn", ffn_norm_set),
                       ("swiglu", swiglu_set), ("gated_add_ffn_rms_norm_modulate_sa", sa_norm_set)):
        sets = [make() for _ in range(NS)]
        calls = [c for _, c in sets]
        for c in calls:
            c()
        st.synchronize()
        g = Graph()
        with g.capture(st):
            for i in range(steps):
                calls[i % NS]()
        g.launch()
        st.synchronize()
        res = []
        for _ in range(3):
            a, b_ = Event(), Event()
            a.record(sh)
            g.launch()
            b_.record(sh)
            b_.synchronize()
            res.append(1000.0 * a.elapsed_ms(b_) / steps)
        us = min(res)
        gbs = kb[name] / (us * 1e-6) / 1e9
        print(json.dumps({"config": f"C3 DiT block kernel alone: {name}, {steps} back-to-back launches in a graph over "
                                    f"{NS} operand sets", "us_per_launch": round(us, 2),
                          "us_per_launch_3_replays": [round(x, 2) for x in res], "bytes_per_launch": kb[name],
                          "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 3)}), flush=True)
        del g, sets, calls
        device.synchronize()


# ---------------------------------------------------------------------------
# Q8_0 matrix-vector products (reported with --gemv): ggml_mul_mat with Q8_0
# weights at the Qwen3-4B batch-8 decode shape (qwen3-lm.h:639-651, 729, 737,
# 755): the fused QKV, O, fused gate/up and down projections of one layer, and
# the LM head over the 151669-row token table. Weights are repacked once (the
# load-time layout); each call quantizes the 8 rows of x and runs the product.
# ---------------------------------------------------------------------------
def gemv_bench(steps: int):
    from acestep_ops import device, ops
    from acestep_ops.device import DTensor, Event, Graph, Stream

    H, I, NH_, NKV_, Dh, V, M = 2560, 9728, 32, 8, 128, 151669, 8
    shapes = [("QKV", H, (NH_ + 2 * NKV_) * Dh), ("O", NH_ * Dh, H), ("gate_up", H, 2 * I), ("down", I, H),
              ("lm_head", H, V)]
    rng = np.random.default_rng(13)
    st = Stream()
    sh = st.handle
    layer_us, layer_bytes = 0.0, 0
    for name, k, n in shapes:
        nbk = k // 32
        blocks = np.empty((n, nbk, 34), np.uint8)
        blocks[:, :, 2:] = rng.integers(-127, 128, (n, nbk, 32), dtype=np.int8).view(np.uint8)
        d = (rng.uniform(0.5, 1.0, (n, nbk)) * 2e-3).astype(np.float16).view(np.uint8).reshape(n, nbk, 2)
        blocks[:, :, :2] = d
        wa = ops.Q8(DTensor.from_numpy(blocks.reshape(n, nbk * 34)))
        wr = ops.q8_0_repack(wa, stream=sh)
        st.synchronize()
        del wa, blocks
        x = DTensor.from_numpy(rng.standard_normal((M, k), dtype=np.float32))
        y = DTensor.empty((M, n), "f32")
        ws = DTensor.empty((max(ops.mul_mat_q8_0_workspace(wr, x), 1),), "u8")
        # `steps` calls back to back in one graph (as a decode step issues them),
        # replayed once after a warm-up replay: the GPU time, not the host's
        g = Graph()
        with g.capture(st):
            for _ in range(steps):
                ops.mul_mat_q8_0(wr, x, out=y, workspace=ws, stream=sh)
        g.launch()
        st.synchronize()
        e0, e1 = Event(), Event()
        e0.record(sh)
        g.launch()
        e1.record(sh)
        e1.synchronize()
        us = 1000.0 * e0.elapsed_ms(e1) / steps
        nbytes = n * nbk * 34 + M * k * 4 + M * n * 4
        gbs = nbytes / (us * 1e-6) / 1e9
        if name != "lm_head":
            layer_us += us
            layer_bytes += nbytes
        print(json.dumps({"config": f"Q8_0 mul_mat {name}, Qwen3-4B decode batch {M}: k={k}, n={n}",
                          "us_per_call": round(us, 2), "bytes_per_call": nbytes,
                          "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 3)}), flush=True)
        del g, wr, x, y, ws
        device.synchronize()
    gbs = layer_bytes / (layer_us * 1e-6) / 1e9
    print(json.dumps({"config": f"Q8_0 mul_mat, one Qwen3-4B layer's four projections at batch {M}",
                      "us_per_layer": round(layer_us, 2), "bytes_per_layer": layer_bytes, "GB/s": round(gbs, 1),
                      "frac": round(gbs / HBM_PEAK_GBS, 3)}), flush=True)
    # the matrix kernel: the DiT projections at T = 6000 x 2 rows (dit-graph.h:36-49), H = 2048
    for name, k, n, m in (("DiT QKV", 2048, 4096, 12000), ("DiT gate/up", 2048, 12288, 12000),
                          ("DiT down", 6144, 2048, 12000), ("Qwen3-4B prefill QKV", 2560, 6144, 2048)):
        nbk = k // 32
        blocks = np.empty((n, nbk, 34), np.uint8)
        blocks[:, :, 2:] = rng.integers(-127, 128, (n, nbk, 32), dtype=np.int8).view(np.uint8)
        blocks[:, :, :2] = (rng.uniform(0.5, 1.0, (n, nbk)) * 2e-3).astype(np.float16).view(np.uint8).reshape(
            n, nbk, 2)
        wr = ops.q8_0_repack(ops.Q8(DTensor.from_numpy(blocks.reshape(n, nbk * 34))), stream=sh)
        del blocks
        x = DTensor.from_numpy(rng.standard_normal((m, k), dtype=np.float32))
        y = DTensor.empty((m, n), "f32")
        ws = DTensor.empty((max(ops.mul_mat_q8_0_workspace(wr, x), 1),), "u8")
        g = Graph()
        with g.capture(st):
            for _ in range(steps):
                ops.mul_mat_q8_0(wr, x, out=y, workspace=ws, stream=sh)
        g.launch()
        st.synchronize()
        e0, e1 = Event(), Event()
        e0.record(sh)
        g.launch()
        e1.record(sh)
        e1.synchronize()
        us = 1000.0 * e0.elapsed_ms(e1) / steps
        ops_ = 2.0 * m * n * k
        print(json.dumps({"config": f"Q8_0 mul_mat {name}: k={k}, n={n}, m={m}", "us_per_call": round(us, 2),
                          "TOPS": round(ops_ / (us * 1e-6) / 1e12, 1),
                          "frac_of_int8_dense": round(ops_ / (us * 1e-6) / 1e12 / 5000.0, 3)}), flush=True)
        del g, wr, x, y, ws
        device.synchronize()


# ---------------------------------------------------------------------------
# One whole Qwen3-4B decoder layer on the device (reported with --decode-layer):
# batch 8, Q8_0 weights, an F16 KV cache (the LM's own, qwen3-lm.h:190-191) and a
# Q8_0 one, 8192 slots per sequence, lengths U[1, 8192] and the 256-bucketed read
# (qw3lm_forward_batch, qwen3-lm.h:626-741). One JSON line per cache type.
# ---------------------------------------------------------------------------
def decode_layer_bench(steps: int):
    for kv_type in ("f16", "q8_0"):
        decode_layer_bench_kv(steps, kv_type)


def decode_layer_bench_kv(steps: int, kv_type: str):
    from acestep_ops import device, ops
    from acestep_ops.device import DTensor, Event, Graph, Stream
    from acestep_ops.qwen3 import Qwen3DecodeLayer, decode_mask

    H, Nh, Nkv, D, I, N, SLOTS = 2560, 32, 8, 128, 9728, 8, 8192
    rng = np.random.default_rng(11)
    lens = rng.integers(1, SLOTS + 1, N)
    pos = (lens - 1).astype(np.int32)
    read = min(SLOTS, int((lens.max() + 255) // 256 * 256))
    st = Stream()
    sh = st.handle

    def q8w(n, k):
        nbk = k // 32
        b = np.empty((n, nbk, 34), np.uint8)
        b[:, :, 2:] = rng.integers(-127, 128, (n, nbk, 32), dtype=np.int8).view(np.uint8)
        b[:, :, :2] = (rng.uniform(0.5, 1.0, (n, nbk)) * 2e-3).astype(np.float16).view(np.uint8).reshape(n, nbk, 2)
        return ops.Q8(DTensor.from_numpy(b.reshape(n, nbk * 34)))

    ones = lambda n: DTensor.from_numpy(np.ones(n, np.float32))  # noqa: E731
    layer = Qwen3DecodeLayer(q8w((Nh + 2 * Nkv) * D, H), q8w(H, Nh * D), q8w(2 * I, H), q8w(H, I), ones(H), ones(H),
                             ones(D), ones(D), H, Nh, Nkv, D, I, SLOTS, N, kv_type, stream=sh)
    if kv_type == "q8_0":
        kb = np.zeros((N, Nkv, SLOTS, D // 32 * 34), np.uint8)
        kb[..., 2:] = rng.integers(-127, 128, kb[..., 2:].shape, dtype=np.int8).view(np.uint8)
        kb.reshape(-1, 34)[:, :2] = np.full((kb.size // 34, 1), 1e-2, np.float16).view(np.uint8)
        layer.k_cache = ops.Q8(DTensor.from_numpy(kb))
        layer.v_cache = ops.Q8(DTensor.from_numpy(kb))
        row_bytes = D // 32 * 34
    else:
        kh = rng.standard_normal((N, Nkv, SLOTS, D), dtype=np.float32).astype(np.float16)
        layer.k_cache = DTensor.from_numpy(kh.view(np.uint16), "f16")
        layer.v_cache = DTensor.from_numpy(kh.view(np.uint16), "f16")
        row_bytes = D * 2
        del kh
    hidden = DTensor.from_numpy(rng.standard_normal((N, H), dtype=np.float32))
    out = DTensor.empty((N, H), "f32")
    dpos, dsets = DTensor.from_numpy(pos), DTensor.from_numpy(np.arange(N, dtype=np.int32))
    mask = decode_mask(pos, read)
    layer.forward(hidden, dpos, dsets, 0, read, mask, out=out)
    st.synchronize()
    g = Graph()
    with g.capture(st):
        for _ in range(steps):
            layer.forward(hidden, dpos, dsets, 0, read, mask, out=out)
    g.launch()
    st.synchronize()
    e0, e1 = Event(), Event()
    e0.record(sh)
    g.launch()
    e1.record(sh)
    e1.synchronize()
    us = 1000.0 * e0.elapsed_ms(e1) / steps
    wbytes = sum(w.n * (w.k // 32) * 34 for w in layer.w.values())
    # K/V bytes the step must read: each sequence's live keys (the mask's -inf tail
    # of the 256-bucketed read is skipped before any byte of it is loaded).
    kvb = int(lens.sum()) * Nkv * row_bytes * 2
    print(json.dumps({"config": f"Qwen3-4B decode layer, batch {N}, Q8_0 weights, {kv_type.upper()} KV cache ({SLOTS} "
                                f"slots, lengths U[1,{SLOTS}], read {read}), every op on the device",
                      "us_per_layer": round(us, 2), "weight_bytes": wbytes, "kv_bytes_live": kvb,
                      "GB/s": round((wbytes + kvb) / (us * 1e-6) / 1e9, 1),
                      "frac": round((wbytes + kvb) / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 3),
                      "tokens_per_s_36_layers": round(N / (36 * us * 1e-6), 1)}), flush=True)
    del layer, g
    device.synchronize()


# ---------------------------------------------------------------------------
# One whole Qwen3-4B decoder layer in prefill on the device (reported with
# --prefill-layer): the two CFG sequences (conditional and unconditional KV
# sets, qwen3-lm.h:429-431) of a 512-token prompt from slot 0, Q8_0 weights,
# an F16 KV cache (the LM's own, qwen3-lm.h:190-191) and a Q8_0 one
# (qw3lm_forward, qwen3-lm.h:429-549). One JSON line per cache type.
# ---------------------------------------------------------------------------
def prefill_layer_bench(steps: int):
    # the CFG pair of a 512-token prompt, and the batched prefill of 8 sequences
    # x 2048 tokens (the Qwen3-4B batch-8 prefill into a KV cache)
    for n, s_, slots in ((2, 512, 4096), (8, 2048, 8192)):
        for kv_type in ("f16", "q8_0"):
            prefill_layer_bench_kv(steps, kv_type, n, s_, slots)


def prefill_layer_bench_kv(steps: int, kv_type: str, N: int = 2, S: int = 512, SLOTS: int = 4096):
    from acestep_ops import device, ops
    from acestep_ops.device import DTensor, Event, Graph, Stream
    from acestep_ops.qwen3 import Qwen3Layer

    H, Nh, Nkv, D, I = 2560, 32, 8, 128, 9728
    rng = np.random.default_rng(17)
    st = Stream()
    sh = st.handle

    def q8w(n, k):
        nbk = k // 32
        b = np.empty((n, nbk, 34), np.uint8)
        b[:, :, 2:] = rng.integers(-127, 128, (n, nbk, 32), dtype=np.int8).view(np.uint8)
        b[:, :, :2] = (rng.uniform(0.5, 1.0, (n, nbk)) * 2e-3).astype(np.float16).view(np.uint8).reshape(n, nbk, 2)
        return ops.Q8(DTensor.from_numpy(b.reshape(n, nbk * 34)))

    ones = lambda n: DTensor.from_numpy(np.ones(n, np.float32))  # noqa: E731
    layer = Qwen3Layer(q8w((Nh + 2 * Nkv) * D, H), q8w(H, Nh * D), q8w(2 * I, H), q8w(H, I), ones(H), ones(H),
                       ones(D), ones(D), H, Nh, Nkv, D, I, SLOTS, N, kv_type, stream=sh)
    hidden = DTensor.from_numpy(rng.standard_normal((N, S, H), dtype=np.float32))
    out = DTensor.empty((N, S, H), "f32")
    inp = layer.prefill_inputs([0] * N, S, 0)
    layer.prefill_run(hidden, inp, out=out)  # allocates the layer's buffers outside the graph
    st.synchronize()
    g = Graph()
    with g.capture(st):
        for _ in range(steps):
            layer.prefill_run(hidden, inp, out=out)
    g.launch()
    st.synchronize()
    e0, e1 = Event(), Event()
    e0.record(sh)
    g.launch()
    e1.record(sh)
    e1.synchronize()
    us = 1000.0 * e0.elapsed_ms(e1) / steps
    T = N * S
    gemm = 2 * T * sum(w.n * w.k for w in layer.w.values())
    attn = 4 * D * Nh * N * (S * (S + 1) // 2)  # the causal pairs (masked tiles are skipped)
    print(json.dumps({"config": f"Qwen3-4B prefill layer, {N} sequences x {S} tokens from slot 0 of {SLOTS}-slot "
                                f"caches, Q8_0 weights, {kv_type.upper()} KV cache, every op on the device",
                      "us_per_layer": round(us, 1), "gemm_flop": gemm, "attn_flop_causal": attn,
                      "TFLOP/s": round((gemm + attn) / (us * 1e-6) / 1e12, 1),
                      "tokens_per_s_36_layers": round(T / (36 * us * 1e-6), 1)}), flush=True)
    del layer, g
    device.synchronize()


# ---------------------------------------------------------------------------
# One whole DiT layer (dit_ggml_build_layer, dit-graph.h:367-448) on the device:
# the DiT's shape (H 2048, 16/8 heads x 128, I 6144, Q8_0 weights, F32
# activations) over the CFG pair of S = 3000 latent tokens, with the cross
# attention over 512 encoder rows (the last 40 padding), as the two layer
# types run: a sliding window of 128 on the even layers and the padding mask
# (all zero) on the odd ones (dit-sampler.h:253-274). A graph of `steps` layer
# calls, replayed once untimed and once timed.
# ---------------------------------------------------------------------------
def dit_layer_bench(steps: int, emit: bool = True):
    """One JSON line per (mask, encoder K/V) variant, or (emit False) their figures as a list."""
    from acestep_ops import device, ops
    from acestep_ops.device import DTensor, Event, Graph, Stream
    from acestep_ops.dit import DiTLayer

    H, Nh, Nkv, D, I, N, S, E, WIN = 2048, 16, 8, 128, 6144, 2, 3000, 512, 128
    rng = np.random.default_rng(23)
    st = Stream()
    sh = st.handle

    def q8w(n, k):
        nbk = k // 32
        b = np.empty((n, nbk, 34), np.uint8)
        b[:, :, 2:] = rng.integers(-127, 128, (n, nbk, 32), dtype=np.int8).view(np.uint8)
        b[:, :, :2] = (rng.uniform(0.5, 1.0, (n, nbk)) * 2e-3).astype(np.float16).view(np.uint8).reshape(n, nbk, 2)
        return ops.Q8(DTensor.from_numpy(b.reshape(n, nbk * 34)))

    ones = lambda n: DTensor.from_numpy(np.ones(n, np.float32))  # noqa: E731
    layer = DiTLayer(q8w((Nh + 2 * Nkv) * D, H), q8w(H, Nh * D), q8w(2 * I, H), q8w(H, I), ones(H), ones(H),
                     ones(D), ones(D), H, Nh, Nkv, D, I, w_ca_q=q8w(Nh * D, H), w_ca_kv=q8w(2 * Nkv * D, H),
                     w_ca_o=q8w(H, Nh * D), ca_norm_w=ones(H), ca_q_norm_w=ones(D), ca_k_norm_w=ones(D), stream=sh)
    hidden = DTensor.from_numpy(rng.standard_normal((N, S, H), dtype=np.float32))
    enc = DTensor.from_numpy(rng.standard_normal((N, E, H), dtype=np.float32))
    adaln = DTensor.from_numpy((0.1 * rng.standard_normal((6, H))).astype(np.float32))
    out = DTensor.empty((N, S, H), "f32")
    pos = DiTLayer.positions(N, S)
    ii = np.arange(S)
    win = np.where(np.abs(ii[None, :] - ii[:, None]) <= WIN // 2, 0.0, -np.inf).astype(np.float16)
    wmask = DTensor.from_numpy(np.ascontiguousarray(np.broadcast_to(win, (N, 1, S, S))).view(np.uint16), "f16")
    del win
    zmask = DTensor.zeros((N, 1, S, S), "f16")
    pm = np.zeros((N, 1, S, E), np.float16)
    pm[..., E - 40:] = -np.inf
    cmask = DTensor.from_numpy(pm.view(np.uint16), "f16")
    T = N * S
    gemm = 2 * T * sum(w.n * w.k for name, w in layer.w.items() if name != "ca_kv") + \
        2 * N * E * layer.w["ca_kv"].n * layer.w["ca_kv"].k
    ca_pairs = 4 * D * Nh * N * S * (E - 40)
    results = []
    kv = layer.encode(enc)  # the encoder K/V once, for the runs that reuse them
    st.synchronize()
    for (label, mk, live), once in ((m, o) for m in ((f"sliding window {WIN}", wmask, None),
                                                      ("padding mask (all zero)", zmask, S)) for o in (False, True)):
        if once:
            call = lambda: layer.forward(hidden, adaln, pos, sa_mask=mk, ca_mask=cmask, out=out, enc_kv=kv)  # noqa
        else:
            call = lambda: layer.forward(hidden, adaln, pos, sa_mask=mk, enc=enc, ca_mask=cmask, out=out)  # noqa
        call()  # allocates the layer's buffers outside the graph
        st.synchronize()
        g = Graph()
        with g.capture(st):
            for _ in range(steps):
                call()
        g.launch()
        st.synchronize()
        e0, e1 = Event(), Event()
        e0.record(sh)
        g.launch()
        e1.record(sh)
        e1.synchronize()
        us = 1000.0 * e0.elapsed_ms(e1) / steps
        pairs = S * S if live else sum(min(S, i + WIN // 2 + 1) - max(0, i - WIN // 2) for i in range(S))
        sa = 4 * D * Nh * N * pairs
        fl = gemm - (2 * N * E * layer.w["ca_kv"].n * layer.w["ca_kv"].k if once else 0) + sa + ca_pairs
        rec = {"config": f"DiT layer, S={S} x {N}, H={H}, {Nh}/{Nkv} heads x {D}, I={I}, Q8_0 weights, "
                         f"F32 activations, self attention under the {label}, cross attention over {E} "
                         "encoder rows (40 padding), the encoder K/V "
                         + ("computed once per generation" if once else "recomputed in the step")
                         + ", every op on the device",
               "us_per_layer": round(us, 1), "gemm_flop": gemm, "attn_flop_live": sa + ca_pairs,
               "TFLOP/s": round(fl / (us * 1e-6) / 1e12, 1)}
        if emit:
            print(json.dumps(rec), flush=True)
        results.append(rec)
        del g
    del layer
    device.synchronize()
    return results


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-rows", type=int, default=ROWS, help="rows of the block the CPU baseline runs")
    ap.add_argument("--cpu-reps", type=int, default=64, help="timed CPU repetitions (about 10 s on 8 threads)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="leave the Qwen3 layer chains and the DiT layer out of the default line")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="launch each block kernel once plus a copy of known size, for counter collection")
    ap.add_argument("--pmc-configs", action="store_true",
                    help="launch the C4/C5 Q8_0 and QK-norm/rope kernels once plus a copy of known size, for counters")
    ap.add_argument("--configs", action="store_true",
                    help="time the Qwen3 layer op chains at the C1/C2/C4/C5 shapes instead (one JSON line each)")
    ap.add_argument("--attention", action="store_true",
                    help="time flash attention over the KV cache at the C2 decode shape (one JSON line per cache type)")
    ap.add_argument("--kernels", action="store_true",
                    help="each C3 block kernel alone, back to back over rotated operand sets")
    ap.add_argument("--decode-layer", action="store_true",
                    help="time one whole Qwen3-4B decoder layer at batch 8 (Q8_0 weights; F16 and Q8_0 KV caches), all on the device")
    ap.add_argument("--prefill-layer", action="store_true",
                    help="time one whole Qwen3-4B decoder layer in prefill (2 CFG sequences x 512 tokens; F16 and "
                         "Q8_0 KV caches), all on the device")
    ap.add_argument("--dit-layer", action="store_true",
                    help="time one whole DiT layer (S=3000 x 2, cross attention, both self-attention masks), all on "
                         "the device")
    ap.add_argument("--gemv", action="store_true",
                    help="time the Q8_0 mul_mat of the Qwen3-4B decode projections and LM head at batch 8")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: measures one GPU only (asked for --gpus {args.gpus}); every op of the path is "
              "row-parallel and shards by rows with no communication, so per-GPU throughput is the N=1 figure.",
              file=sys.stderr)
        sys.exit(2)
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: one process / one GPU only", file=sys.stderr)
        sys.exit(2)

    if args.pmc_pass:
        pmc_pass()
        return
    if args.pmc_configs:
        pmc_pass_configs()
        return
    if args.configs:
        configs_bench(args.steps, args.warmup)
        return
    if args.attention:
        attention_bench(args.steps)
        return
    if args.gemv:
        gemv_bench(args.steps)
        return
    if args.kernels:
        kernels_bench(args.steps)
        return
    if args.decode_layer:
        decode_layer_bench(args.steps)
        return
    if args.prefill_layer:
        prefill_layer_bench(args.steps)
        return
    if args.dit_layer:
        dit_layer_bench(args.steps)
        return
    kb = block_bytes(ROWS, cross=True)
    kb_f = block_bytes(ROWS, fused=True)
    kb_u = block_bytes(ROWS, fused=False)
    total_bytes = sum(kb.values())
    graph_bytes = args.steps * total_bytes + lead_bytes(ROWS)  # what the timed graph moves
    ms_step, ms_five, ms_unfused, wall, per_k, per_k_f, per_k_u, (ms_ca, per_k_ca) = gpu_bench(args.steps,
                                                                                                args.warmup)
    kb_ca = block_bytes_ca(ROWS)
    value = graph_bytes / (args.steps * ms_step * 1e-3) / 1e9
    dom = "swiglu"
    dom_gbs = kb[dom] / (per_k[dom] * 1e-6) / 1e9
    # the Qwen3 layer chains (C1 0.6B T=512, C2 4B decode batch 8, C4 1.7B
    # prefill 4x4096, C5 4B prefill 8x2048 into a Q8_0 KV cache), timed in the
    # same run; they do not enter value
    cfg = None if args.no_configs else configs_bench(min(args.steps, 20), args.warmup, emit=False)
    # a whole DiT layer (products, attention and the fused ops) over the same run's
    # clock; it does not enter value
    ditl = None if args.no_configs else dit_layer_bench(min(args.steps, 10), emit=False)

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
        hc = host_cpu()
        # the reference's backend policy: hardware_concurrency() / 2 threads
        # (backend.h:28-35), within the CPUs this job may use
        threads = max(1, min(hc["logical_cpus"] // 2, hc["job_cpus"]))
        med, spent = cpu_bench(args.cpu_rows, args.cpu_reps, threads, hc["isa"])
        scale = ROWS / args.cpu_rows
        cpu_block_s = med * scale
        all_t = hc["job_cpus"]
        if all_t != threads:
            med_a, spent_a = cpu_bench(args.cpu_rows, max(8, args.cpu_reps // 2), all_t, hc["isa"])
            all_run = {"threads": all_t, "us_per_block": round(med_a * scale * 1e6, 1),
                       "value": round(total_bytes / (med_a * scale) / 1e9, 3), "cpu_s": round(spent_a, 1)}
        else:
            all_run = {"threads": all_t, "same_as_policy_run": True,
                       "note": "every logical CPU this job may use is already in the policy run"}
        cpu = {
            "value": round(total_bytes / cpu_block_s / 1e9, 3),
            "unit": "GB/s",
            "cores": threads,
            "cores_note": (f"{threads} OpenMP threads (unpinned), so at most {threads} of the host's "
                           f"{hc['physical_cores']} physical cores ({hc['threads_per_core']} hardware thread(s) "
                           f"per core) busy at once"),
            "threads": threads,
            "kind": "port",
            "us_per_block": round(cpu_block_s * 1e6, 1),
            "host": hc,
            "all_logical_threads": all_run,
            "sample": (f"reference's unfused F32 ggml node graph of one DiT block (rms_norm, mul, add, rope, swiglu "
                       f"nodes, ggml-cpu arithmetic restated in C, built -O3 -march={hc['isa']}, OpenMP over rows) "
                       f"on {args.cpu_rows} of {ROWS} rows, {threads} threads (logical CPUs / 2, the reference's "
                       f"backend policy, within the job's {hc['job_cpus']} CPUs), median of {args.cpu_reps} reps "
                       f"after 3 warm-ups ({spent:.1f} s of CPU work)"
                       + (f", scaled x{scale:.2f} to the full block" if args.cpu_rows != ROWS else "")
                       + "; GB/s uses the same bf16 byte accounting as value"),
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
                               "x 128, SwiGLU I=6144; 4 launches/step (each gated residual fused with the norm "
                               "after it: the FFN norm, and the next block's self-attention norm); K steps timed as "
                               "one replay of a HIP graph of the first block's norm + K consecutive blocks",
                   "rows": ROWS, "hidden": H, "intermediate": I_FF, "bytes_per_step": total_bytes,
                   "bytes_first_block_norm": lead_bytes(ROWS)},
        "per_kernel_us": {k: round(v, 2) for k, v in per_k.items()},
        "per_kernel_gbs": {k: round(kb[k] / (per_k[k] * 1e-6) / 1e9, 1) for k in kb},
        "five_launch_block": {"us_per_block": round(ms_five * 1e3, 2), "bytes_per_step": sum(kb_f.values()),
                              "gbs": round(sum(kb_f.values()) / (ms_five * 1e-3) / 1e9, 1),
                              "per_kernel_us": {k: round(v, 2) for k, v in per_k_f.items()}},
        "unfused": {"us_per_block": round(ms_unfused * 1e3, 2), "bytes_per_step": sum(kb_u.values()),
                    "gbs": round(sum(kb_u.values()) / (ms_unfused * 1e-3) / 1e9, 1),
                    "per_kernel_us": {k: round(v, 2) for k, v in per_k_u.items()}},
        "block_with_cross_attn": {
            "launches": len(kb_ca), "us_per_block": round(ms_ca * 1e3, 2), "bytes_per_step": sum(kb_ca.values()),
            "gbs": round(sum(kb_ca.values()) / (ms_ca * 1e-3) / 1e9, 1),
            "reference_structure_bytes": CA_REF_BYTES, "reference_structure_us_at_70pct": CA_REF_US_AT_70,
            "per_kernel_us": {k: round(v, 2) for k, v in per_k_ca.items()},
            "per_kernel_gbs": {k: round(kb_ca[k] / (per_k_ca[k] * 1e-6) / 1e9, 1) for k in kb_ca}},
        "roofline": {"bound": "hbm", "achieved": round(dom_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom_gbs / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": "k_swiglu (bf16)",
                     "bytes_per_launch": kb[dom], "us_per_launch": round(per_k[dom], 2),
                     "timing": "mean of HIP event pairs around the kernel's launch inside the steady-state block "
                               "sequence on the bench stream (includes ~2.5-3 us of event and dispatch time that "
                               "rocprof's kernel duration leaves out)"},
        "configs": cfg,
        "dit_layer": ditl,
        "cpu_baseline": cpu,
        "wall_s": round(wall, 4),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
