"""AFA forward benchmark on one MI355X (BASELINE.json metric, configuration C3).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--workload c3]

--workload selects another configuration of BASELINE.json for the same JSON line (the default,
c3, is the metric's own configuration): c2 (B=4 H=8 L=2048 D=64 bf16 causal), c4 / c4f32
(B=32 H=4 L=1024 D=64 bf16 / fp32 causal, default Cayley parameters), c5 (B=2 H=16 L=8192
D=128 bf16 causal forward) and c5bwd (its analytical backward, 10 B H D N_pairs FLOPs); ring16,
c5ring8 and c3ring8 time distributed_ring_afa with its shards' hops run in turn on this GPU;
c3hop8 and c5hop8 time one ring hop at one GPU's shard shape, c3share8 C3's per-GPU share under
8-way batch x heads sharding; flash_c3, flash_tpu2k and flash_tpu4k time this library's forward
beside torch's softmax FlashAttention at the same shapes (the reference's own comparison).

Workload (C3): B=8, H=12, L=4096, D=64, bf16, causal, q/k Cayley-rotated in-kernel with
Cayley parameters t_i = 10000^(-2i/D); q, k, v ~ N(0, 1) synthetic, resident in HBM.
A step is one fused forward launch (afa_fwd through the C ABI) over the whole batch.

Printed: one JSON line with the whole-job throughput (TFLOP/s, FLOPs = 4 B H D L(L+1)/2),
the roofline of the kernel (HIP-event average launch time on the launch stream against the
2516.6 TFLOP/s bf16 dense MFMA peak) and the CPU baseline: the C restatement of the reference
algorithm (oracle/afa_contract.c, OpenMP) timed on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_BF16_TFLOPS = 2516.6  # 256 CU x 2.4 GHz x 4096 dense bf16 FLOP/clk/CU
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "afa_fwd_c3_bf16_traffic.json")
METRIC = "AFA fwd TFLOP/s + % bf16 MFMA peak at L=4096 D=64 (1 GPU); x vs host CPU ref"
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
# VALU ceiling of the bf16/fp16 forward: each score costs 7.5 VALU lane-operations (the rho^8 chain,
# row sum and bf16 pack: 120 VALU instructions per wave per 1024-score unit, counted in the
# kernel's gfx950 ISA), issued at 16 lanes per cycle per SIMD for unpacked fp32 (the published
# 157.3 TFLOP/s vector peak counts packed FMAs: 16 lanes x 2 x 2 FLOP), 1024 SIMDs at 2.4 GHz.
VALU_OPS_PER_SCORE = 7.5
VALU_LANE_OPS_PER_S = 16 * 1024 * 2.4e9
# name -> (B, H, L, D, dtype, causal, rotary freqs: "c3" | "default" | None, backward, description)
WORKLOADS = {
    "c1": (1, 4, 256, 64, "fp32", False, None, False, "C1: AFA forward, fp32, non-causal (latency-bound)"),
    "c3": (8, 12, 4096, 64, "bf16", True, "c3", False,
           "C3: AFA forward, causal, Cayley rotary inside the afa_fwd call (k rotated once by a pre-pass "
           "kernel, q rotated at load by the attention kernel)"),
    "c2": (4, 8, 2048, 64, "bf16", True, None, False, "C2: AFA forward, causal"),
    "c4": (32, 4, 1024, 64, "bf16", True, "default", False,
           "C4: AFA forward, causal, default Cayley rotary"),
    "c4f32": (32, 4, 1024, 64, "fp32", True, "default", False,
              "C4 (fp32): AFA forward, causal, default Cayley rotary"),
    "c5": (2, 16, 8192, 128, "bf16", True, None, False, "C5: AFA forward, causal, head_dim 128"),
    "c5bwd": (2, 16, 8192, 128, "bf16", True, None, True,
              "C5: AFA analytical backward (dq, dk, dv), causal, head_dim 128"),
    "c3bwd": (8, 12, 4096, 64, "bf16", True, "c3", True,
              "C3: AFA analytical backward (dq, dk, dv), causal, Cayley rotary"),
    "c4f32bwd": (32, 4, 1024, 64, "fp32", True, "default", True,
                 "C4 (fp32): AFA analytical backward (dq, dk, dv), causal, default Cayley rotary"),
    "c3share8": (1, 12, 4096, 64, "bf16", True, "c3", False,
                 "C3's share of one GPU out of 8 under batch x heads sharding: 12 of its 96 (b, h) pairs"),
}
# A-Softmax over the last axis of (rows, cols) scores: name -> (rows, cols, dtype, backward, description)
SOFTMAX_WORKLOADS = {
    "asoftmax": (96 * 2048, 2048, "bf16", False, "algebraic_softmax forward, (196608, 2048) bf16 scores"),
    "asoftmax_bwd": (96 * 2048, 2048, "bf16", True, "algebraic_softmax VJP, (196608, 2048) bf16 scores"),
}

# Fused Linear + OACE loss head: name -> (rows N, d_model, vocab, backward, description).  The
# reference benchmarks the forward at N=512, d_model=768, vocab=50257, bf16, (d_model, vocab)
# output head (scripts/benchmark_kernels.py:118-183, reported as tokens/s).
OACE_WORKLOADS = {
    "oace": (512, 768, 50257, False, "fused_linear_oace forward, reference benchmark configuration"),
    "oace_bwd": (512, 768, 50257, True, "fused_linear_oace backward (dh, dW), reference configuration"),
    "oace_n8k": (8192, 768, 50257, False, "fused_linear_oace forward, 8192 rows"),
    "oace_n8k_bwd": (8192, 768, 50257, True, "fused_linear_oace backward, 8192 rows"),
    "oace_train": (512, 768, 50257, "step", "fused_linear_oace forward + backward, reference configuration"),
    "oace_n8k_train": (8192, 768, 50257, "step", "fused_linear_oace forward + backward, 8192 rows"),
}


def environment():
    """What the line was measured with, after the reference's evidence records (which carry
    package versions and the sha256 of every source file, scripts/phase6_records.py:23-50):
    the GPU and its ISA, the HIP and torch versions, the sha256 (first 16 hex digits) of the loaded
    libafa_hip.so and of the kernel sources it was built from, and the host's CPU count."""
    import glob
    import hashlib

    import torch

    from algebraic_intelligence_amd import _lib

    def sha(paths):
        h = hashlib.sha256()
        for p in paths:
            with open(p, "rb") as f:
                h.update(os.path.basename(p).encode() + b"\0" + f.read())
        return h.hexdigest()[:16]

    props = torch.cuda.get_device_properties(0)
    srcs = sorted(glob.glob(os.path.join(ROOT, "algebraic_intelligence_amd", "csrc", "*")))
    return {"gpu": props.name, "arch": getattr(props, "gcnArchName", None),
            "compute_units": props.multi_processor_count, "hip": torch.version.hip,
            "torch": torch.__version__, "lib_sha16": sha([_lib.LIB_PATH]), "csrc_sha16": sha(srcs),
            "host_cpus": len(os.sched_getaffinity(0))}


def warm_up(step, args):
    """args.warmup untimed steps, then more until args.warmup_seconds have passed, so the timed
    steps run at the clock the GPU holds under sustained load.  Returns (steps run, seconds)."""
    import torch

    t0 = time.perf_counter()
    n = 0
    for _ in range(args.warmup):
        step()
        n += 1
    torch.cuda.synchronize()
    while time.perf_counter() - t0 < args.warmup_seconds:
        for _ in range(10):
            step()
        n += 10
        torch.cuda.synchronize()
    return n, round(time.perf_counter() - t0, 3)


def power_sample(step, seconds=1.5):
    """Run `step` back to back for `seconds` while sampling the board with amd-smi: the socket
    power (W) and the current clock of each XCD's graphics domain (MHz), as medians over the
    samples.  The dense MFMA peak assumes the 2.4 GHz maximum clock; under MFMA-dense work the
    board holds less (the clock falls with the density of MFMA work, also below the 1400 W board
    power limit)."""
    import re
    import shutil
    import subprocess
    import threading

    import torch

    exe = shutil.which("amd-smi")
    if exe is None:
        return {"available": False, "reason": "amd-smi not found"}
    texts = []
    stop = threading.Event()

    def sampler():
        time.sleep(0.4)
        while not stop.is_set():
            try:
                r = subprocess.run([exe, "metric", "-g", "0", "--power", "--clock"], capture_output=True,
                                   text=True, timeout=10)
                texts.append(r.stdout)
            except (OSError, subprocess.SubprocessError):
                return

    th = threading.Thread(target=sampler, daemon=True)
    th.start()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds or (not texts and time.perf_counter() - t0 < 4 * seconds):
        for _ in range(20):
            step()
        torch.cuda.synchronize()
    stop.set()
    th.join(timeout=15)
    power, clocks = [], []
    for text in texts:
        section, per = None, []
        for raw in text.splitlines():
            line = raw.strip()
            m = re.match(r"SOCKET_POWER:\s*([0-9.]+)\s*W", line)
            if m:
                power.append(float(m.group(1)))
            m = re.match(r"(GFX_\d+|MEM_\d+|[A-Z_]+\d*):$", line)
            if m:
                section = m.group(1)
            m = re.match(r"CLK:\s*([0-9.]+)\s*MHz", line)
            if m and section is not None and section.startswith("GFX_"):
                per.append(float(m.group(1)))
        if per:
            clocks.append(per)
    if not power:
        return {"available": False, "reason": "no SOCKET_POWER in amd-smi output"}
    import numpy as np

    out = {"available": True, "samples": len(power), "socket_w": float(np.median(power)), "limit_w": 1400.0}
    if clocks:
        c = np.median(np.array(clocks), axis=0)
        out.update({"gfx_mhz_per_xcd": [round(float(x)) for x in c], "gfx_mhz_mean": round(float(c.mean())),
                    "gfx_mhz_max": 2400})
    return out


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--warmup-seconds", type=float, default=1.0,
                    help="keep running untimed warmup steps until this much time has passed (the GPU "
                         "raises its clock over the first tens of milliseconds of load)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-power", action="store_true", help="skip the board power / clock sample")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample budget")
    ap.add_argument("--workload", default="c3",
                    choices=sorted(WORKLOADS) + sorted(SOFTMAX_WORKLOADS) + sorted(OACE_WORKLOADS)
                    + sorted(RING_WORKLOADS) + sorted(HOP_WORKLOADS) + sorted(FLASH_WORKLOADS))
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="instead of the benchmark, run a plain device copy of MIB MiB --steps times "
                         "(reference point for the FETCH_SIZE / WRITE_SIZE counters)")
    return ap.parse_args()


def copy_calibration(mib, steps):
    import torch

    src = torch.ones(mib * (1 << 20) // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": src.numel() * 4, "steps": steps}), flush=True)


def cpu_baseline(q, k, v, rot, seconds):
    """Time the C contract restatement on whole (b, h) heads of the same inputs until the
    budget is spent (at least one head); report TFLOP/s over the heads done."""
    import numpy as np

    from oracle import contract as C
    from tests.helpers import to_bits

    B, H, L, D = q.shape
    cores = len(os.sched_getaffinity(0))
    rc = rot.c.detach().cpu().numpy().astype(np.float32)
    rs = rot.s.detach().cpu().numpy().astype(np.float32)
    qb, kb, vb = (to_bits(t) for t in (q, k, v))
    heads, elapsed = 0, 0.0
    per_head_flops = 4 * D * L * (L + 1) // 2
    while heads < B * H and (heads == 0 or elapsed < seconds):
        b, h = divmod(heads, H)
        sl = (slice(b, b + 1), slice(h, h + 1))
        t0 = time.perf_counter()
        C.afa_fwd(qb[sl], kb[sl], vb[sl], C.DT_BF16, 0.5, True, None, (rc, rs), block_q=128, block_k=128,
                  nthreads=cores)
        elapsed += time.perf_counter() - t0
        heads += 1
    # the same on one core, one head
    t0 = time.perf_counter()
    C.afa_fwd(qb[:1, :1], kb[:1, :1], vb[:1, :1], C.DT_BF16, 0.5, True, None, (rc, rs), block_q=128, block_k=128,
              nthreads=1)
    one = time.perf_counter() - t0
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "")
    except OSError:
        pass
    return {
        "value": round(per_head_flops * heads / elapsed / 1e12, 6),
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "cpu": model,
        "one_core": {"value": round(per_head_flops / one / 1e12, 6), "unit": "TFLOP/s",
                     "sample": f"1 (b,h) head, {one:.1f} s"},
        "sample": f"{heads} of {B * H} (b,h) heads of C3 (L={L}, D={D}, bf16, causal, AGO), "
                  f"{elapsed:.1f} s, C restatement oracle/afa_contract.c with OpenMP",
    }


def softmax_bench(args, dev):
    """HBM-bound A-Softmax row kernels: GB/s of compulsory traffic (read x [and g], write y / dx)."""
    import torch

    from algebraic_intelligence_amd import _lib

    rows, cols, dt_name, backward, workload = SOFTMAX_WORKLOADS[args.workload]
    tdt = torch.bfloat16
    g = torch.Generator(device=dev).manual_seed(0)
    x = (torch.randn((rows, cols), generator=g, device=dev, dtype=torch.float32) * 3).to(tdt)
    y = torch.empty_like(x)
    gy = torch.randn((rows, cols), generator=g, device=dev, dtype=torch.float32).to(tdt)
    stream = torch.cuda.current_stream(dev)
    lib = _lib.lib()

    def step():
        if backward:
            r = lib.asoftmax_bwd(_lib.AFA_BF16, rows, cols, x.data_ptr(), gy.data_ptr(), y.data_ptr(),
                                 0.5, 1e-5, stream.cuda_stream)
        else:
            r = lib.asoftmax_fwd(_lib.AFA_BF16, rows, cols, x.data_ptr(), y.data_ptr(), 0.5, 1e-5,
                                 stream.cuda_stream)
        if r != 0:
            _lib.check(r, "asoftmax")

    warm = warm_up(step, args)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(args.steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    nbytes = rows * cols * 2 * (3 if backward else 2)
    gbs = nbytes / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": f"A-Softmax {'VJP' if backward else 'forward'} HBM GB/s [{args.workload}]",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "warmup_run": {"steps": warm[0], "seconds": warm[1]},
        "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": dt_name,
        "data": "synthetic: x ~ 3 N(0,1), g ~ N(0,1) bf16, resident in HBM",
        "config": {"workload": workload, "rows": rows, "cols": cols, "bytes_per_step": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": 8000.0, "unit": "GB/s",
                     "frac": round(gbs / 8000.0, 4), "traffic": None},
    }), flush=True)


def oace_bench(args, dev):
    """Fused Linear + OACE through the C ABI (bf16, (d_model, vocab) output head, workspace
    allocated once).  Throughput in tokens/s (the reference's metric) and MFMA TFLOP/s on the
    algorithmic work: 2 N V d for the logits plus the cheaper of a second sweep (2 N V d) and the
    Gram route (2 d^2 V + 2 N d^2) for the second moment; the backward is 6 N V d (recomputed
    logits, dh, dW)."""
    import torch

    from algebraic_intelligence_amd import _lib

    N, d, V, backward, workload = OACE_WORKLOADS[args.workload]
    g = torch.Generator(device=dev).manual_seed(0)
    h = torch.randn((N, d), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    w = torch.randn((d, V), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    t = torch.randint(0, V, (N,), generator=g, device=dev, dtype=torch.int64)
    loss = torch.empty((), dtype=torch.float32, device=dev)
    rows = torch.empty((N, 8), dtype=torch.float32, device=dev)
    dh = torch.empty_like(h)
    dw = torch.empty_like(w)
    one = torch.ones((), dtype=torch.float32, device=dev)
    lib = _lib.lib()
    wsb = lib.oace_workspace_size(_lib.AFA_BF16, N, d, V, 0, 0)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)

    def fwd():
        r = lib.oace_linear_fwd(_lib.AFA_BF16, N, d, V, h.data_ptr(), d, w.data_ptr(), 0, V, t.data_ptr(), 100.0,
                                2.0, loss.data_ptr(), rows.data_ptr(), 0, ws.data_ptr(), wsb, stream.cuda_stream)
        if r != 0:
            _lib.check(r, "oace_linear_fwd")

    def bwd():
        # same workspace as the forward, h and w unchanged: its transposed weights and (when it kept
        # them) its logits are reused (OACE_FLAG_WT_READY | OACE_FLAG_Z_READY)
        r = lib.oace_linear_bwd(_lib.AFA_BF16, N, d, V, h.data_ptr(), d, w.data_ptr(), 0, V, t.data_ptr(), 2.0,
                                rows.data_ptr(), one.data_ptr(), dh.data_ptr(), dw.data_ptr(), 0x30, ws.data_ptr(),
                                wsb, stream.cuda_stream)
        if r != 0:
            _lib.check(r, "oace_linear_bwd")

    def train():
        fwd()
        bwd()

    fwd()
    step = train if backward == "step" else bwd if backward else fwd
    warm = warm_up(step, args)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(args.steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    nvd = 2 * N * V * d
    # the logits once; their second moment from a second sweep (or the Gram route) unless the forward
    # keeps them (fp32 rows x padded vocabulary within 256 MB), when the backward reuses them too
    z_kept = N * (-(-V // 64) * 64) * 4 <= 256 << 20
    fwd_flops = nvd if z_kept else nvd + min(nvd, 2 * d * d * V + 2 * N * d * d)
    bwd_flops = 2 * nvd if z_kept else 3 * nvd
    flops = {False: fwd_flops, True: bwd_flops, "step": fwd_flops + bwd_flops}[backward]
    tflops = flops / (ms * 1e-3) / 1e12
    if not torch.isfinite(loss):
        raise RuntimeError("non-finite loss")
    print(json.dumps({
        "metric": f"fused Linear+OACE {dict([(False, 'forward'), (True, 'backward'), ('step', 'forward+backward')])[backward]} "
                  f"tokens/s (1 GPU) [{args.workload}]",
        "value": round(N / (ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "warmup_run": {"steps": warm[0], "seconds": warm[1]},
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: h, W ~ N(0,1) bf16, uniform targets, resident in HBM",
        "config": {"workload": workload, "rows": N, "d_model": d, "vocab": V, "w_layout": "(d_model, vocab)",
                   "logits_kept": z_kept, "flops_per_step": flops},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 3), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / PEAK_BF16_TFLOPS, 4), "traffic": None},
    }), flush=True)


# Sequence ring (distributed_ring_afa) with its hops run in turn on one GPU: name -> (B, H, L, D,
# dtype, causal, shards, description).  ring16 is the reference's 16-chip ring check
# (scripts/run_phase6_tpu.py:358-435: B=1 H=8 L=4096 as 16 shards of 256, D=64, fp32, non-causal).
# One ring hop at one GPU's shard shape: name -> (B, H, shard_len, D, dtype, description); one
# afa_fwd call with AFA_FLAG_ACCUMULATE, non-causal (every hop but the diagonal one).
HOP_WORKLOADS = {
    "c3hop8": (8, 12, 512, 64, "bf16", "one non-causal ring hop of C3 on 8 GPUs: 512 queries x 512 keys per head"),
    "c5hop8": (2, 16, 1024, 128, "bf16", "one non-causal ring hop of C5 on 8 GPUs: 1024 queries x 1024 keys per head"),
}

RING_WORKLOADS = {
    "ring16": (1, 8, 4096, 64, "fp32", False, 16, "distributed_ring_afa, the reference's 16-shard ring check"),
    "c5ring8": (2, 16, 8192, 128, "bf16", True, 8, "distributed_ring_afa, C5 shape as 8 shards of 1024"),
    "c3ring8": (8, 12, 4096, 64, "bf16", True, 8, "distributed_ring_afa, C3 shape (no rotary) as 8 shards of 512"),
}


def hop_bench(args, dev):
    """One ring hop as one GPU of the ring runs it: afa_fwd with AFA_FLAG_ACCUMULATE on its query
    shard and one received key/value shard, adding into fp32 accumulators resident in HBM."""
    import torch

    from algebraic_intelligence_amd import _lib

    B, H, S, D, dt_name, workload = HOP_WORKLOADS[args.workload]
    g = torch.Generator(device=dev).manual_seed(0)
    q, k, v = (torch.randn((B, H, S, D), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
               for _ in range(3))
    acc = torch.zeros((B, H, S, D), dtype=torch.float32, device=dev)
    den = torch.zeros((B, H, S), dtype=torch.float32, device=dev)
    lib = _lib.lib()
    stream = torch.cuda.current_stream(dev)
    wsb = lib.afa_fwd_workspace_size(_lib.AFA_BF16, B, H, S, D, 0)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=dev)
    strides = (__import__("ctypes").c_int64 * 12)(*(list(q.stride()[:3]) * 3 + list(acc.stride()[:3])))

    def step():
        r = lib.afa_fwd(_lib.AFA_BF16, B, H, S, D, q.data_ptr(), k.data_ptr(), v.data_ptr(), strides,
                        acc.data_ptr(), den.data_ptr(), None, None, 0, 0.0, 0, 0, _lib.FLAG_ACCUMULATE,
                        ws.data_ptr(), wsb, stream.cuda_stream)
        if r != 0:
            _lib.check(r, "afa_fwd")

    warm = warm_up(step, args)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(args.steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    flops = 4 * B * H * S * S * D
    tflops = flops / (ms * 1e-3) / 1e12
    # algorithmic bytes: q, k, v read; the fp32 accumulators read and written; row sums likewise
    nbytes = 3 * B * H * S * D * 2 + 2 * B * H * S * D * 4 + 2 * B * H * S * 4
    print(json.dumps({
        "metric": f"AFA ring hop TFLOP/s (1 GPU's share) [{args.workload}]",
        "value": round(tflops, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "warmup_run": {"steps": warm[0], "seconds": warm[1]}, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": dt_name,
        "data": "synthetic: q,k,v ~ N(0,1) bf16, fp32 accumulators, resident in HBM",
        "config": {"workload": workload, "batch": B, "heads": H, "shard_len": S, "head_dim": D, "causal": False,
                   "flops_per_step": flops},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 3), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(tflops / PEAK_BF16_TFLOPS, 4), "traffic": None,
                     "duration_of": "one afa_fwd call: the row-norm pre-pass and the hop kernel"},
        "hbm": {"algorithmic_bytes": nbytes, "achieved_gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
                "flop_per_byte": round(flops / nbytes, 1)},
    }), flush=True)


def ring_bench(args, dev):
    """The whole ring (accumulator clears, every hop's accumulating afa_fwd calls, the final
    division) as one step, against one fused forward call on the same inputs.  FLOPs as the
    forward's: 4 B H D per kept (query, key) pair, which the ring's hops cover exactly once."""
    import torch

    import algebraic_intelligence_amd as A

    B, H, L, D, dt_name, causal, n, workload = RING_WORKLOADS[args.workload]
    tdt = torch.bfloat16 if dt_name == "bf16" else torch.float32
    g = torch.Generator(device=dev).manual_seed(0)
    q, k, v = (torch.randn((B, H, L, D), generator=g, device=dev, dtype=torch.float32).to(tdt)
               for _ in range(3))
    stream = torch.cuda.current_stream(dev)
    res = {}

    def ring():
        res["out"] = A.distributed_ring_afa(q, k, v, sink_omega=0.5, causal=causal, num_devices=n)

    def full():
        A.pallas_afa_forward(q, k, v, sink_omega=0.5, causal=causal)

    def timed(step):
        warm = warm_up(step, args)
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(args.steps):
            step()
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / args.steps, warm

    ms, warm = timed(ring)
    ms_full, _ = timed(full)
    if not torch.isfinite(res["out"].float()).all():
        raise RuntimeError("non-finite output")
    flops = A.afa_flops(B, H, L, D, causal=causal)
    tflops = flops / (ms * 1e-3) / 1e12
    peak = PEAK_BF16_TFLOPS if dt_name == "bf16" else PEAK_FP32_TFLOPS
    print(json.dumps({
        "metric": f"AFA ring TFLOP/s, {n} shards on 1 GPU [{args.workload}]",
        "value": round(tflops, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "warmup_run": {"steps": warm[0], "seconds": warm[1]},
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": dt_name, "data": f"synthetic: q,k,v ~ N(0,1) {dt_name}, resident in HBM",
        "config": {"workload": workload, "batch": B, "heads": H, "seq_len": L, "head_dim": D, "causal": causal,
                   "shards": n, "shard_len": L // n, "sink_omega": 0.5, "flops_per_step": flops},
        "full_forward": {"ms": round(ms_full, 5), "tflops": round(flops / (ms_full * 1e-3) / 1e12, 3),
                         "ring_over_full": round(ms / ms_full, 3)},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 3), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(tflops / peak, 4), "traffic": None,
                     "duration_of": "one ring: accumulator clears, every hop's afa_fwd calls, afa_ring_finish"},
    }), flush=True)


# AFA against softmax FlashAttention on the same GPU, the reference's own bar for this path
# (scripts/run_phase6_tpu.py:147-240: pallas_afa_forward against JAX's Pallas flash attention on
# the same q, k, v; PASS at a throughput ratio >= 0.85; results/phase6/tpu/metrics.json:294-300
# gives 0.9841 at L=2048 and 0.9967 at L=4096).  name -> (B, H, L, D, causal, description); bf16,
# no rotary tables on either side.
FLASH_WORKLOADS = {
    "flash_c3": (8, 12, 4096, 64, True, "C3's shape without rotary tables, causal"),
    "flash_tpu2k": (1, 8, 2048, 128, False, "the reference's TPU comparison shape, L=2048, non-causal"),
    "flash_tpu4k": (1, 8, 4096, 128, False, "the reference's TPU comparison shape, L=4096, non-causal"),
}


def flash_bench(args, dev):
    """pallas_afa_forward (this library) and torch's scaled_dot_product_attention restricted to its
    flash backend, timed alike in one process on the same bf16 q, k, v.  The FLOPs of both are
    4 B H D N_pairs, so the ratio is the time ratio.  As the reference does, a missing flash
    kernel is recorded as unavailable rather than replaced by a dense softmax; torch's
    memory-efficient fused kernel is timed beside it for context."""
    import torch
    import torch.nn.functional as F

    import algebraic_intelligence_amd as A

    B, H, L, D, causal, workload = FLASH_WORKLOADS[args.workload]
    g = torch.Generator(device=dev).manual_seed(0)
    q, k, v = (torch.randn((B, H, L, D), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
               for _ in range(3))
    stream = torch.cuda.current_stream(dev)
    flops = A.afa_flops(B, H, L, D, causal=causal)

    def timed(step):
        warm = warm_up(step, args)
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(args.steps):
            step()
        end.record(stream)
        torch.cuda.synchronize()
        ms = start.elapsed_time(end) / args.steps
        return {"ms": round(ms, 5), "tflops": round(flops / (ms * 1e-3) / 1e12, 3),
                "warmup_run": {"steps": warm[0], "seconds": warm[1]}}

    afa = timed(lambda: A.pallas_afa_forward(q, k, v, sink_omega=0.5, causal=causal))
    others = {}
    try:
        from torch.nn.attention import SDPBackend, sdpa_kernel
        backends = {"flash": SDPBackend.FLASH_ATTENTION, "efficient": SDPBackend.EFFICIENT_ATTENTION}
    except ImportError as e:  # pragma: no cover - torch without the selector
        backends = {}
        others["flash"] = {"available": False, "reason": f"torch.nn.attention: {e}"}
    for name, be in backends.items():
        def step(be=be):
            with sdpa_kernel([be]):
                return F.scaled_dot_product_attention(q, k, v, is_causal=causal)
        try:
            step()
            torch.cuda.synchronize()
        except Exception as e:  # the backend has no kernel for this GPU, dtype or shape
            others[name] = {"available": False, "reason": f"{type(e).__name__}: {str(e)[:200]}"}
            continue
        others[name] = {"available": True, **timed(step)}
    fl = others.get("flash", {})
    ratio = round(fl["ms"] / afa["ms"], 4) if fl.get("available") else None
    print(json.dumps({
        "metric": f"AFA / softmax FlashAttention throughput ratio, same GPU [{args.workload}]",
        "value": ratio, "unit": "ratio (AFA TFLOP/s / flash TFLOP/s)", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": afa["ms"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic: q,k,v ~ N(0,1) bf16, resident in HBM",
        "config": {"workload": workload, "batch": B, "heads": H, "seq_len": L, "head_dim": D, "causal": causal,
                   "flops_per_step": flops},
        "afa": afa, "sdpa": others,
        "efficient_ratio": (round(others["efficient"]["ms"] / afa["ms"], 4)
                            if others.get("efficient", {}).get("available") else None),
        "reference_bar": {"gate": 0.85, "tpu_v4_ratio": {"L2048": 0.9841, "L4096": 0.9967}},
    }), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: the AFA path's multi-GPU sharding "
                                   "is a design note in the repository's documentation, so --gpus "
                                   "must be 1"}))
        sys.exit(2)

    if args.copy_calibration:
        copy_calibration(args.copy_calibration, args.steps)
        return

    import numpy as np
    import torch

    import algebraic_intelligence_amd as A
    from algebraic_intelligence_amd import _lib

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.workload in SOFTMAX_WORKLOADS:
        softmax_bench(args, dev)
        return
    if args.workload in OACE_WORKLOADS:
        oace_bench(args, dev)
        return
    if args.workload in FLASH_WORKLOADS:
        flash_bench(args, dev)
        return
    if args.workload in RING_WORKLOADS:
        ring_bench(args, dev)
        return
    if args.workload in HOP_WORKLOADS:
        hop_bench(args, dev)
        return
    B, H, L, D, dt_name, causal, rot_kind, backward, workload = WORKLOADS[args.workload]
    tdt = torch.bfloat16 if dt_name == "bf16" else torch.float32
    code = _lib.AFA_BF16 if dt_name == "bf16" else _lib.AFA_F32
    g = torch.Generator(device=dev).manual_seed(0)
    q, k, v = (torch.randn((B, H, L, D), generator=g, device=dev, dtype=torch.float32).to(tdt)
               for _ in range(3))
    rot = None
    if rot_kind is not None:
        freqs = 10000.0 ** (-2.0 * np.arange(D // 2) / D) if rot_kind == "c3" else None
        rot = A.build_cayley_rotary_matrix(D, L, freqs=freqs, device=dev)
    rc = rot.c.contiguous() if rot is not None else None
    rs = rot.s.contiguous() if rot is not None else None
    out = torch.empty_like(q)
    den = torch.empty((B, H, L, 1), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev)
    lib = _lib.lib()
    ptr = _lib.ptr

    # the call's workspace (rotated k and the fast-rho key bounds), allocated once outside the
    # timed region as a caller would
    fws_bytes = lib.afa_fwd_workspace_size(code, B, H, L, D, int(rot is not None))
    fws = torch.empty(max(fws_bytes, 1), dtype=torch.uint8, device=dev)

    def fwd():
        r = lib.afa_fwd(code, B, H, L, D, q.data_ptr(), k.data_ptr(), v.data_ptr(), None,
                        out.data_ptr(), den.data_ptr() if backward else None, ptr(rc), ptr(rs),
                        L if rot is not None else 0, 0.5, int(causal), 0, 0, fws.data_ptr(), fws_bytes,
                        stream.cuda_stream)
        if r != 0:
            _lib.check(r, "afa_fwd")

    step = fwd
    if backward:
        fwd()
        gout = torch.randn((B, H, L, D), generator=g, device=dev, dtype=torch.float32).to(tdt)
        dq, dk, dv = (torch.empty_like(q) for _ in range(3))
        ws_bytes = lib.afa_bwd_workspace_size(code, B, H, L, D, int(rot is not None))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)

        def step():
            r = lib.afa_bwd(code, B, H, L, D, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                            den.data_ptr(), gout.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                            ptr(rc), ptr(rs), L if rot is not None else 0, 0.5, int(causal), 0, 0,
                            ws.data_ptr(), ws_bytes,
                            stream.cuda_stream)
            if r != 0:
                _lib.check(r, "afa_bwd")

    warm = warm_up(step, args)
    # the timed region: K calls between two events, nothing else on the stream
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(args.steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    # per-call spread from a second, untimed pass with an event after every call
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    ev[0].record(stream)
    for i in range(args.steps):
        step()
        ev[i + 1].record(stream)
    torch.cuda.synchronize()
    ms_median = float(np.median([ev[i].elapsed_time(ev[i + 1]) for i in range(args.steps)]))
    flops = A.afa_flops(B, H, L, D, causal=causal) // 4 * (10 if backward else 4)
    tflops = flops / (ms * 1e-3) / 1e12
    # algorithmic HBM bytes: q, k, v in and out (forward); q, k, v, out, g in and dq, dk, dv out,
    # plus d (backward); the fp32 Cayley tables when given
    esz = 2 if dt_name == "bf16" else 4
    tensors = 8 if backward else 4
    nbytes = tensors * B * H * L * D * esz + (4 * B * H * L if backward else 0) + (4 * L * D if rot is not None else 0)
    gbs = nbytes / (ms * 1e-3) / 1e9
    if not torch.isfinite(out.float()).all():
        raise RuntimeError("non-finite output")
    peak = PEAK_BF16_TFLOPS if dt_name == "bf16" else PEAK_FP32_TFLOPS
    hbm_bound = flops / nbytes < peak * 1e12 / (PEAK_HBM_GBS * 1e9)  # below the ridge point

    traffic = None
    if args.workload == "c3" and os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    line = {
        "metric": METRIC,
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup, "warmup_run": {"steps": warm[0], "seconds": warm[1]},
        "ms_per_step": round(ms, 5),
        "ms_per_step_median": round(ms_median, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dt_name,
        "data": f"synthetic: q,k,v ~ N(0,1) {dt_name}, resident in HBM",
        "config": {"workload": workload, "batch": B, "heads": H, "seq_len": L, "head_dim": D,
                   "causal": causal, "sink_omega": 0.5, "flops_per_step": flops},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 3), "peak": peak,
                     "unit": "TFLOP/s", "frac": round(tflops / peak, 4), "traffic": traffic,
                     "duration_of": ("one afa_bwd call: every launch it makes" if backward else
                                     "one afa_fwd call: every launch it makes (with rotary tables at "
                                     "head_dim 64, the K rotation pre-pass and the attention kernel)")},
        "hbm": {"algorithmic_bytes": nbytes, "achieved_gbs": round(gbs, 1), "peak_gbs": PEAK_HBM_GBS,
                "frac": round(gbs / PEAK_HBM_GBS, 4), "flop_per_byte": round(flops / nbytes, 1)},
    }
    if hbm_bound:
        # arithmetic intensity below the ridge point: the HBM roofline bounds this configuration
        line["roofline"].update({"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                 "frac": round(gbs / PEAK_HBM_GBS, 4)})
    if not backward and dt_name == "bf16":
        # the score's VALU work against the same score's 4 D MFMA FLOPs
        valu = VALU_LANE_OPS_PER_S / VALU_OPS_PER_SCORE * 4 * D / 1e12
        both = 1.0 / (1.0 / peak + 1.0 / valu)
        line["roofline"]["valu_ceiling"] = {
            "tflops": round(valu, 1), "frac": round(tflops / valu, 4), "ops_per_score": VALU_OPS_PER_SCORE,
            "mfma_plus_valu_no_overlap_tflops": round(both, 1), "frac_of_no_overlap": round(tflops / both, 4)}
    if args.workload != "c3":
        line["metric"] = METRIC.replace("at L=4096 D=64", f"at L={L} D={D}") + f" [{args.workload}]"
        if backward:
            line["metric"] = line["metric"].replace("AFA fwd", "AFA bwd")
        if dt_name != "bf16":
            line["metric"] = line["metric"].replace("bf16 MFMA peak", f"{dt_name} MFMA peak")
    if not args.no_power:
        # board power and clocks under the same calls, sustained; run after the timed region
        line["power"] = power_sample(step)
    if not args.no_cpu and args.workload == "c3":
        line["cpu_baseline"] = cpu_baseline(q, k, v, rot, args.cpu_seconds)
        line["cpu_baseline"]["gpu_speedup"] = round(tflops / line["cpu_baseline"]["value"], 1)
    line["environment"] = environment()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
