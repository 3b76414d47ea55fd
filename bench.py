"""Benchmark of the LTV combined-QKV filter path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--workload filter|look_back|gpt|scan_fwd|prefill|decode|peaks|lt_f32]

Workload (the d12 training shape): x bf16
[32, 1024, 768] ~ N(0, 1); c.weight [2322, 768] fp32 ~ N(0, 1/768) (value rows
and the 18 gate rows, r = 128); logit_bias = 0; init_param ~ N(0, 1/768);
upstream dq, dk, dv ~ N(0, 1).  Synthetic data, random-init weights.

One step = one pass of the hot path through the drop-in filter module:
forward (bf16 MFMA projection into the head-major layout, gated EWMA scan) and
backward (reverse scan, projection dX and dW) via autograd.  Inputs are resident
in HBM before the timed region.  ``value`` = tokens / s = B*T*K / elapsed.

Before the W warm-up steps, untimed steps of the same workload run for
``--settle-s`` seconds (0.1 by default; reported as ``settle``): after an idle
period the GPU's clock ramps up over the first 15-20 ms of load (measured on
MI355X at configs[2]: per-step times fall from 590-630 us to about 520 us over
the first ~30 steps of a process), and the metric is the steady-state rate of a
training loop.  The timed region is still exactly K full steps.

``--workload look_back`` runs the same shapes through the look-back filter
with the d12 layer spec (P, Q, K) = (16, 16, 9): chunks of 16 steps, each
restarted from the inits over an 8-step warm-up (the reference's production
look-back configuration).  ``--workload gpt`` is BASELINE.json configs[3].
``--workload scan_fwd`` is configs[1], the standalone scan forward: bf16 head-major
values [32, 3 x 6, 1024, 128] ~ N(0, 1) with a per-element decay (r = 1)
a = sigmoid(z), z ~ N(2, 1), i.e. logit + bias = -z; fp32 state, bf16 out; a
step is one scan launch and ``value`` is its algorithmic GB/s.  ``--workload
prefill`` is configs[4]'s prefill: one forward of the filter at B = 8,
T = 8192 with long-memory decays (tokens / s).  ``--workload decode`` is
configs[4]'s decode: 256 single-token steps at B = 64 through the KV-cache
protocol after a 16-token prefill (tokens / s through the module), and the same
256 steps replayed from a captured HIP graph.  ``--workload lt_f32`` is the
filter's fp32 path's projection (the reference-layout ``fused_linear_transpose``,
forward and both gradients) at configs[2]'s shapes, in TFLOP/s.

Printed as one JSON line, with
  roofline     -- the dominant kernel's algorithmic bytes (or FLOPs) per launch
                  over its average duration (HIP events on the launch stream,
                  created without the system-scope fence, recorded in a second
                  pass of the same number of steps: a record still idles the
                  GPU for several microseconds, so the timed steps run
                  without them), against MI355X's published peak;
  kernels      -- the same figure for every kernel of the path;
  cpu_baseline -- the CPU oracle (oracle/ltv_oracle.py, a restatement of the
                  reference's sequential PyTorch path) timed on a bounded
                  sample of the same workload on the host cores.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "nanochat-filter_amd"))

COPY_CAL_BYTES = 256 << 20

# published MI355X peaks
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
F32_MFMA_PEAK_TFLOPS = 157.3

B, T, C = 32, 1024, 768
NH = NKVH = 6
D, R = 128, 128
DA = D // R
H = NH + 2 * NKVH
F = H * (D + DA)
FP = (F + 127) // 128 * 128  # packed weight rows
S_IO = 2  # bf16


def algorithmic_work():
    """Per-launch algorithmic bytes / FLOPs: the scan forward reads the values
    and logits (F columns) and the inits and writes the H·D outputs; the
    backward reads values, logits and upstream gradients and writes the
    F-column gradient (states recomputed, not re-read), plus the inits and
    their gradient; each projection GEMM is 2·M·C·F FLOPs."""
    scan_fwd = B * T * (F + H * D) * S_IO + B * H * D * S_IO + 4 * H * DA
    scan_bwd = B * T * (2 * F + H * D) * S_IO + 2 * B * H * D * S_IO + 4 * H * DA
    gemm = 2 * B * T * C * F
    return {
        "scan_fwd": ("hbm", scan_fwd),
        "scan_bwd": ("hbm", scan_bwd),
        "qkv_project_fwd": ("mfma", gemm),
        "qkv_project_bwd_input": ("mfma", gemm),
        "qkv_project_bwd_weight": ("mfma", gemm),
        # grad_x and grad_weight through one library call (one fused launch at d12)
        "qkv_project_bwd": ("mfma", 2 * gemm),
        "pack_weight": ("hbm", F * C * 4 + FP * C * 2),
    }


LOOK_BACK_PQK = (16, 16, 9)


def profiled_traffic(span: str, summary: str = "d12_traffic.json"):
    """HBM bytes per launch of a kernel span, from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary of this workload (copy-calibrated); None if not profiled."""
    path = os.path.join(ROOT, "profiles", summary)
    try:
        with open(path) as fh:
            d = json.load(fh)
        return d["bytes_per_launch"].get(span), d["source"]
    except (OSError, ValueError, KeyError):
        return None, None


def measured_peak(name: str, bound: str):
    """The box-measured ceiling for a kernel (profiles/peaks.json, written from
    ``bench.py --workload peaks``): the bf16 MFMA loop with random operands
    for the GEMMs, the HBM stream of the kernel's read/write mix in the scan's
    access shape for the scans, the grid-stride copy otherwise; None when the
    file is absent."""
    try:
        with open(os.path.join(ROOT, "profiles", "peaks.json")) as fh:
            p = json.load(fh)
    except (OSError, ValueError):
        return None
    if bound == "mfma":
        return p.get("bf16_mfma_tflops")
    return p.get("stream_gbs", {}).get(name, p.get("hbm_copy_gbs"))


def emit(out: dict) -> None:
    """Print the result line, after checking that no chained scan of the run
    reported a failure (the library's error mailbox; raises if one did)."""
    from nanochat_amd import _native as N
    N.check_chain_errors()
    print(json.dumps(out), flush=True)


def cpu_model() -> str:
    """The host CPU's model name (from /proc/cpuinfo), or "unknown"."""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(seconds_target: float = 10.0, pqk=None):
    """Time the oracle's forward+backward on a sample of the workload (with
    ``pqk``, the look-back scan in place of the full recurrence)."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import ltv_oracle as O

    cores = len(os.sched_getaffinity(0))
    Bs = 1  # one sequence of the 32 at full T and C
    rng = np.random.default_rng(0)
    x = rng.standard_normal((Bs, T, C), dtype=np.float32)
    w = (rng.standard_normal((F, C)) / np.sqrt(C)).astype(np.float32)
    ini = (rng.standard_normal((Bs, H, D)) / np.sqrt(C)).astype(np.float32)
    bias = np.zeros((H, DA), np.float32)
    dq = rng.standard_normal((Bs, T, NH, D), dtype=np.float32)
    dk = rng.standard_normal((Bs, T, NKVH, D), dtype=np.float32)
    dv = rng.standard_normal((Bs, T, NKVH, D), dtype=np.float32)
    reps = 0
    t0 = time.perf_counter()
    t_ = lambda a: np.ascontiguousarray(a.transpose(0, 2, 1, 3))  # noqa: E731
    with threadpool_limits(limits=cores):
        while True:
            if pqk is None:
                q, k, v, comb, saved = O.filter_forward(x, w, ini, bias, NH, NKVH, DA, R, "f32")
                O.filter_backward(x, w, ini, bias, comb, saved, dq, dk, dv, NH, NKVH, DA, R,
                                  "f32")
            else:
                comb = np.ascontiguousarray(
                    O.linear_transpose_forward(x, w, "f32").transpose(0, 2, 1))
                O.look_back_forward(comb, ini, bias, NH, NKVH, DA, R, *pqk, True, "f32")
                gc, _, _ = O.look_back_backward(comb, ini, bias, t_(dq), t_(dk), t_(dv), NH,
                                                NKVH, DA, R, *pqk, True, "f32")
                O.linear_transpose_backward(x, w, gc.transpose(0, 2, 1), "f32")
            reps += 1
            el = time.perf_counter() - t0
            if el >= seconds_target:
                break
    return {
        "value": round(Bs * T * reps / el, 1),
        "unit": "tokens/s",
        "cores": cores,
        "cpu": cpu_model(),
        "kind": "port",
        "sample": f"{reps} x fwd+bwd of {Bs} sequence(s) of the workload "
                  f"(T={T}, C={C}, F={F}{'' if pqk is None else f', look-back {pqk}'}), "
                  f"fp32 numpy, {el:.1f} s",
    }


def settle(step, seconds: float) -> int:
    """Untimed steps for ``seconds`` of wall time (the GPU clock's ramp from
    idle), counted from the end of a first step that takes the one-time costs
    (library load, first allocations); the queue is drained every 8 steps so
    it stays short.  Returns the number of steps run."""
    import torch
    if seconds <= 0:
        return 0
    step()
    torch.cuda.synchronize()
    n = 1
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(8):
            step()
        n += 8
        torch.cuda.synchronize()
    return n


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--settle-s", type=float, default=0.1,
                    help="untimed steps for this many seconds before the warm-up steps (the "
                         "GPU clock's ramp from idle); 0: none")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--workload",
                    choices=("filter", "look_back", "gpt", "scan_fwd", "prefill", "decode",
                             "peaks", "lt_f32"),
                    default="filter",
                    help="filter: BASELINE.json configs[2] (the default, the metric's workload); "
                         "look_back: the same shapes through the look-back filter with the d12 "
                         "layer spec (16, 16, 9); "
                         "gpt: configs[3], one training step of the 12-layer d12 GPT with the "
                         "filter in every layer (tokens/s and the filter's share of the step); "
                         "scan_fwd: configs[1], the standalone per-element-decay scan forward "
                         "(GB/s); prefill: configs[4]'s prefill, the filter forward at B=8, "
                         "T=8192 with decay sigmoid(N(3, 1.5)) (tokens/s); "
                         "peaks: the measured roofline peaks (MFMA loop, HBM streams in the "
                         "scan's access shape, the library GEMM on the projection's shapes); "
                         "lt_f32: the filter's fp32 path's projection, fused_linear_transpose "
                         "forward + backward at configs[2]'s shapes (TFLOP/s)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="after the timed region, run a plain device copy of 256 MiB five times "
                         "(the known-size reference for rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the path shards over B with no exchange but the weight-gradient reduction; "
              "only the single-GPU figure is reported)", file=sys.stderr)
        sys.exit(2)

    if args.workload == "gpt":
        gpt_main(args)
        return
    if args.workload == "scan_fwd":
        scan_fwd_main(args)
        return
    if args.workload == "prefill":
        prefill_main(args)
        return
    if args.workload == "decode":
        decode_main(args)
        return
    if args.workload == "peaks":
        peaks_main(args)
        return
    if args.workload == "lt_f32":
        lt_f32_main(args)
        return

    import torch
    from nanochat_amd import _native as N

    look_back = args.workload == "look_back"
    if look_back:
        from nanochat_amd.gpt_config import ChunksAndHistory
        from nanochat_amd.ltv_look_back_fused_concat_head_major_register_cast_blelloch_scan_qkv_filter import (
            LtvLookBackFusedConcatHeadMajorRegisterCastBlellochScanQkvFilter as LookBackFilter,
        )
        from nanochat_amd.ops.ltv_cuda_ops import (
            fused_linear_transpose,
            ltv_cuda_look_back_fused_concat_head_major_register_cast_blelloch_scan as look_back_op,
        )
        f = LookBackFilter(NH, NKVH, D, R, ChunksAndHistory(*LOOK_BACK_PQK),
                           transpose_op=fused_linear_transpose, look_back_op=look_back_op)
    else:
        from nanochat_amd.ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan_qkv_filter import (
            LtvCudaFusedConcatHeadMajorRegisterCastBlellochScanQkvFilter as Filter,
        )
        from nanochat_amd.ltv.ltv_filter import LtvInitValues
        f = Filter(NH, NKVH, D, R)

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    with torch.no_grad():
        f.c.weight.normal_(0.0, C ** -0.5)
        f.logit_bias.zero_()
        f.init_param.normal_(0.0, C ** -0.5)
    f = f.to(dev)
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(B, T, C, generator=g, device=dev).to(torch.bfloat16).requires_grad_(True)
    dq = torch.randn(B, T, NH, D, generator=g, device=dev).to(torch.bfloat16)
    dk = torch.randn(B, T, NKVH, D, generator=g, device=dev).to(torch.bfloat16)
    dv = torch.randn(B, T, NKVH, D, generator=g, device=dev).to(torch.bfloat16)
    if look_back:
        def forward():
            # the (H, D) parameter, as LtvLookBackQkvComputerModule hands it over
            # without a KV cache (its gradient summed over the batch in the library)
            return f(x, f.init_param, full_recurrence=False)
    else:
        none = LtvInitValues()

        def forward():
            return f(x, none)

    def step():
        f.zero_grad(set_to_none=True)
        x.grad = None
        q, k, v = forward()
        torch.autograd.backward([q, k, v], [dq, dk, dv])

    settled = settle(step, args.settle_s)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0

    # per-kernel durations from a second pass of the same steps: recording an
    # event leaves the GPU idle for several microseconds, so the timed steps
    # above run without them
    with N.KernelRecorder() as rec:
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()

    if args.calibrate_copy:
        src = torch.empty(COPY_CAL_BYTES, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()

    durs = rec.durations_ms()
    work = algorithmic_work()
    kernels = {}
    for name, ms in durs.items():
        bound, amount = work[name]
        avg = sum(ms) / len(ms)
        if bound == "hbm":
            ach, peak, unit = amount / (avg * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s"
        else:
            ach, peak, unit = amount / (avg * 1e-3) / 1e12, BF16_PEAK_TFLOPS, "TFLOP/s"
        mp = measured_peak(name, bound)
        kernels[name] = {"bound": bound, "avg_us": round(avg * 1e3, 2), "launches": len(ms),
                         "achieved": round(ach, 1), "peak": peak, "unit": unit,
                         "frac": round(ach / peak, 4), "work_per_launch": amount,
                         "peak_measured": mp,
                         "frac_measured": round(ach / mp, 4) if mp else None}
    dominant = max(kernels, key=lambda k: kernels[k]["avg_us"] * kernels[k]["launches"])
    dk_ = kernels[dominant]
    traffic, traffic_src = profiled_traffic(
        dominant, "d12_look_back_traffic.json" if look_back else "d12_traffic.json")
    roofline = {"kernel": dominant, "bound": dk_["bound"], "achieved": dk_["achieved"],
                "peak": dk_["peak"], "unit": dk_["unit"], "frac": dk_["frac"], "traffic": traffic,
                "traffic_source": traffic_src, "peak_measured": dk_["peak_measured"],
                "frac_measured": dk_["frac_measured"],
                "peak_measured_source": "profiles/peaks.json"}
    scan_time = kernels.get("scan_fwd", {}).get("avg_us", 0) + kernels.get("scan_bwd", {}).get("avg_us", 0)
    scan_bytes = work["scan_fwd"][1] + work["scan_bwd"][1]
    scan_gbs = scan_bytes / (scan_time * 1e-6) / 1e9 if scan_time else None

    ms_per_step = elapsed * 1e3 / args.steps
    metric = "QKV+EWMA scan fwd+bwd tokens/s and scan HBM GB/s (%peak) at B32 T1024 C768"
    workload = "configs[2]: d12 fused QKV projection + EWMA scan, fwd+bwd"
    if look_back:
        metric = ("look-back (P, Q, K) = (16, 16, 9) QKV+EWMA scan fwd+bwd tokens/s and scan "
                  "HBM GB/s (%peak) at B32 T1024 C768")
        workload = ("configs[2] shapes through the look-back filter, layer spec "
                    "(P, Q, K) = (16, 16, 9), fwd+bwd")
    out = {
        "metric": metric,
        "value": round(B * T * args.steps / elapsed, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": {"seconds": args.settle_s, "steps": settled},
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": workload,
                   "B": B, "T": T, "C": C, "n_head": NH, "n_kv_head": NKVH, "head_dim": D,
                   "r": R, "F": F, "parallelism": "single GPU"},
        "scan_gbs": round(scan_gbs, 1) if scan_gbs else None,
        "scan_frac_hbm": round(scan_gbs / HBM_PEAK_GBS, 4) if scan_gbs else None,
        "roofline": roofline,
        "kernels": kernels,
    }
    if look_back:
        out["config"]["look_back_pqk"] = list(LOOK_BACK_PQK)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds, LOOK_BACK_PQK if look_back else None)
    emit(out)


# the standalone scan forward, per-element decay
SF_B, SF_H, SF_T, SF_D = 32, 18, 1024, 128


# configs[1]'s and the d12 scan's arrays: 1,152 (b, head, 64-channel slab)
# sequences of T = 1024 steps x 128 bytes, 151 MB per array
PEAK_SLICES = 1152
PEAK_SLICE_BYTES = 1024 * 128


def peaks_main(args):
    """Measured peaks on this box, printed as one JSON line (no CPU baseline):
      * bf16 MFMA: v_mfma_f32_32x32x16_bf16 loop, two wavefronts per SIMD,
        random operand bits (and all-zero operands: higher clock);
      * HBM: 16-byte streams over 151 MB arrays -- grid-stride copy, read and
        write, and the scan's access shape (one contiguous 128 KB slice per
        workgroup, 1,152 workgroups) with 1, 2 and 3 arrays read and one
        written;
      * the library GEMM (torch.matmul, hipBLASLt) on the projection's three
        shapes, for comparison with this library's kernels;
      * the projection GEMM's k-step without its epilogue on every CU (64 KB
        of direct-to-LDS loads, 256 bf16 MFMAs on random bits, fragment
        reads, one barrier per step): each part alone and together, in us
        per step.
    Each figure is the median of ``--steps`` timed launches (HIP events)."""
    import ctypes
    import torch
    from nanochat_amd import _native as N

    lib = ctypes.CDLL(os.path.join(ROOT, "nanochat-filter_amd", "nanochat_amd", "libltv_peaks.so"))
    lib.ltv_peak_mfma.restype = ctypes.c_int
    lib.ltv_peak_mfma.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                  ctypes.c_void_p]
    lib.ltv_peak_stream.restype = ctypes.c_int
    lib.ltv_peak_stream.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int,
                                    ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                                    ctypes.c_uint32, ctypes.c_void_p]
    lib.ltv_peak_overlap.restype = ctypes.c_int
    lib.ltv_peak_overlap.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p,
                                     ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    dev = torch.device("cuda:0")
    st = N.stream_of(torch.empty(1, device=dev))
    n_cu = torch.cuda.get_device_properties(dev).multi_processor_count
    steps = max(3, args.steps)

    def timed(fn):
        for _ in range(2):
            fn()
        ts = []
        for _ in range(steps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            b.synchronize()
            ts.append(a.elapsed_time(b) * 1e-3)
        ts.sort()
        return ts[len(ts) // 2]

    out = {"metric": "measured roofline peaks (bf16 MFMA, HBM streams) on one MI355X",
           "n_gpus": 1, "steps": steps, "cus": n_cu, "published": {"bf16_mfma_tflops": 2500.0,
                                                                    "hbm_gbs": 8000.0}}
    # MFMA
    blocks, iters = 2 * n_cu, 4096
    res = torch.empty(blocks * 256, dtype=torch.float32, device=dev)
    flop = blocks * 4 * iters * 8 * 32768
    for name, zero in (("bf16_mfma_random", 0), ("bf16_mfma_zero", 1)):
        t = timed(lambda: N.check(lib.ltv_peak_mfma(res.data_ptr(), blocks, iters, zero, st),
                                  "ltv_peak_mfma"))
        out[name] = {"tflops": round(flop / t / 1e12, 1), "us": round(t * 1e6, 1)}
    # HBM streams
    nbytes = PEAK_SLICES * PEAK_SLICE_BYTES
    n16 = nbytes // 16
    arrs = [torch.empty(nbytes, dtype=torch.uint8, device=dev) for _ in range(4)]
    for a_ in arrs:
        a_.random_(0, 256)
    srcs = (ctypes.c_void_p * 3)(*[a_.data_ptr() for a_ in arrs[:3]])
    dst = arrs[3].data_ptr()

    def stream(nr, write, nt, slice16, nblocks):
        t = timed(lambda: N.check(lib.ltv_peak_stream(srcs, nr, dst, write, nt, n16, slice16,
                                                      nblocks, 0x9e3779b9, st),
                                  "ltv_peak_stream"))
        moved = (nr + (1 if write else 0)) * nbytes
        return {"gbs": round(moved / t / 1e9, 1), "us": round(t * 1e6, 1), "bytes": moved}

    gs = 64 * n_cu  # grid-stride workgroups
    out["copy_grid_nt"] = stream(1, 1, 1, 0, gs)
    out["copy_grid"] = stream(1, 1, 0, 0, gs)
    out["read_grid"] = stream(1, 0, 0, 0, gs)
    out["write_grid_nt"] = stream(0, 1, 1, 0, gs)
    sl = PEAK_SLICE_BYTES // 16
    for nr in (1, 2, 3):
        out[f"slices_{nr}r1w"] = stream(nr, 1, 0, sl, PEAK_SLICES)
        out[f"slices_{nr}r1w_nt"] = stream(nr, 1, 1, sl, PEAK_SLICES)
    del arrs
    torch.cuda.synchronize()
    # the GEMM k-step's parts beside each other (one workgroup of 8 wavefronts per CU)
    src_bytes = 64 << 20
    src = torch.empty(src_bytes, dtype=torch.uint8, device=dev)
    src.random_(0, 256)
    ov_out = torch.empty(n_cu * 512, dtype=torch.float32, device=dev)
    ov_steps = 600
    ov = {}
    for name, mode in (("loads", 5), ("mfma", 6), ("loads_mfma", 7), ("mfma_reads", 30),
                       ("loads_mfma_reads", 31), ("mfma_reads_sink", 58),
                       ("loads_mfma_reads_sink", 59), ("mfma_reads_2ahead", 94),
                       ("loads_mfma_reads_2ahead", 95)):
        t = timed(lambda: N.check(lib.ltv_peak_overlap(src.data_ptr(), src_bytes, ov_out.data_ptr(),
                                                       n_cu, ov_steps, mode, st),
                                  "ltv_peak_overlap"))
        ov[name] = round(t * 1e6 / ov_steps, 3)
    out["gemm_step_parts_us"] = ov
    del src, ov_out
    torch.cuda.synchronize()
    # library GEMM on the projection's shapes (bf16 in, bf16 out)
    M, Kc, Fp = B * T, C, 2432
    g = torch.Generator(device=dev).manual_seed(0)
    shapes = {"gemm_lib_forward": ((M, Kc), (Kc, Fp)),   # x (M, C) . Wp^T (C, Fp)
              "gemm_lib_grad_x": ((M, Fp), (Fp, Kc)),    # dC (M, Fp) . Wp (Fp, C)
              "gemm_lib_grad_weight": ((Fp, M), (M, Kc))}  # dC^T (Fp, M) . x (M, C)
    for name, (sa, sb) in shapes.items():
        a_ = torch.randn(sa, generator=g, device=dev).to(torch.bfloat16).contiguous()
        b_ = torch.randn(sb, generator=g, device=dev).to(torch.bfloat16).contiguous()
        t = timed(lambda: torch.matmul(a_, b_))
        out[name] = {"tflops": round(2 * M * Kc * F / t / 1e12, 1), "us": round(t * 1e6, 1),
                     "shape": [list(sa), list(sb)]}
        del a_, b_
    emit(out)


def lt_f32_main(args):
    """The filter's fp32 path projects through the reference-layout op
    ``fused_linear_transpose`` (x (B, T, C) . W (F, C)^T -> (B, F, T)).  One
    step at configs[2]'s shapes is its forward and both gradients from a
    (B, F, T) grad_out, through the ops the fp32 filter's autograd calls (the
    backward with its split workspace); value is the step's TFLOP/s (3 GEMMs
    of 2 B T C F FLOP), the roofline the forward GEMM against the fp32 MFMA
    peak, with the library GEMM (torch.matmul, hipBLASLt) on the forward's
    shape beside it."""
    import torch
    from nanochat_amd import _native as N
    import nanochat_amd.ops  # noqa: F401

    ops = torch.ops.nanochat_cuda
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn((B, T, C), generator=g, device=dev)
    w = torch.randn((F, C), generator=g, device=dev) / C ** 0.5
    go = torch.randn((B, F, T), generator=g, device=dev)
    gx, gw = torch.empty_like(x), torch.empty_like(w)

    def step():
        ops.fused_linear_transpose_cuda_op(x, w)
        ops.fused_linear_transpose_backward_kernel(x, w, go, gx, gw)

    settled = settle(step, args.settle_s)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    with N.KernelRecorder() as rec:
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
    if args.calibrate_copy:
        src = torch.empty(COPY_CAL_BYTES, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
    flop = 2.0 * B * T * C * F
    durs = rec.durations_ms()
    spans = {}
    for name, n_gemm in (("linear_transpose_fwd", 1), ("linear_transpose_bwd", 2)):
        ms = durs[name]
        avg = sum(ms) / len(ms)
        ach = n_gemm * flop / (avg * 1e-3) / 1e12
        spans[name] = {"avg_us": round(avg * 1e3, 2), "launches": len(ms),
                       "achieved": round(ach, 1), "peak": F32_MFMA_PEAK_TFLOPS,
                       "unit": "TFLOP/s", "frac": round(ach / F32_MFMA_PEAK_TFLOPS, 4),
                       "work_per_launch": n_gemm * flop}
    # the library GEMM on the forward's shape (same operands, fp32)
    lib_ms = []
    for _ in range(args.steps + 2):
        a_, b_ = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a_.record()
        torch.matmul(w, x.transpose(1, 2))
        b_.record()
        b_.synchronize()
        lib_ms.append(a_.elapsed_time(b_))
    lib_ms = sorted(lib_ms[2:])
    lib_t = lib_ms[len(lib_ms) // 2] * 1e-3
    fw = spans["linear_transpose_fwd"]
    traffic, traffic_src = profiled_traffic("linear_transpose_fwd", "lt_f32_traffic.json")
    out = {
        "metric": "fp32 reference-layout projection (fused_linear_transpose fwd + bwd) TFLOP/s, "
                  "configs[2] shapes x (32, 1024, 768) . W (2322, 768)^T",
        "value": round(3 * flop * args.steps / elapsed / 1e12, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": {"seconds": args.settle_s, "steps": settled},
        "ms_per_step": round(elapsed * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "fp32 path projection at configs[2] shapes (B=32, T=1024, "
                               "C=768, F=2322)",
                   "B": B, "T": T, "K": C, "F": F, "parallelism": "single GPU"},
        "roofline": {"kernel": "linear_transpose_fwd (gemm_f32m_kernel)", "bound": "mfma",
                     "achieved": fw["achieved"], "peak": F32_MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": fw["frac"], "traffic": traffic,
                     "traffic_source": traffic_src, "avg_us": fw["avg_us"],
                     "work_per_launch": flop},
        "spans": spans,
        "library_gemm_fwd": {"tflops": round(flop / lib_t / 1e12, 1), "us": round(lib_t * 1e6, 1),
                             "what": "torch.matmul(W, x^T), fp32 (hipBLASLt)"},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = lt_f32_cpu_baseline(args.cpu_seconds)
    emit(out)


def lt_f32_cpu_baseline(seconds_target: float):
    """The oracle's projection forward + backward (numpy, float64 accumulation)
    on one of the 32 sequences, repeated for about ``seconds_target``."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import ltv_oracle as O

    cores = len(os.sched_getaffinity(0))
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, T, C), dtype=np.float32)
    w = (rng.standard_normal((F, C)) / np.sqrt(C)).astype(np.float32)
    go = rng.standard_normal((1, F, T), dtype=np.float32)
    reps = 0
    t0 = time.perf_counter()
    with threadpool_limits(limits=cores):
        while True:
            O.linear_transpose_forward(x, w, "f32")
            O.linear_transpose_backward(x, w, go, "f32")
            reps += 1
            el = time.perf_counter() - t0
            if el >= seconds_target:
                break
    return {
        "value": round(3 * 2.0 * T * C * F * reps / el / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": cores,
        "cpu": cpu_model(),
        "kind": "port",
        "sample": f"{reps} x fwd+bwd of 1 sequence (T={T}, C={C}, F={F}), numpy float64 "
                  f"accumulation, {el:.1f} s",
    }


def scan_fwd_bytes():
    """Algorithmic bytes of one configs[1] launch: read the values and the
    per-element logits, write the outputs (bf16), read the inits (bf16) and the
    fp32 bias (formula of the scan forward with Da = D, r = 1)."""
    n = SF_B * SF_H * SF_T * SF_D
    return 3 * n * S_IO + SF_B * SF_H * SF_D * S_IO + 4 * SF_H * SF_D


def scan_fwd_cpu_baseline(seconds_target: float):
    """The oracle's scan forward on one batch row of configs[1] (fp32 numpy)."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import ltv_oracle as O

    cores = len(os.sched_getaffinity(0))
    rng = np.random.default_rng(0)
    u = rng.standard_normal((1, SF_T, SF_H, SF_D), dtype=np.float32)
    z = (2.0 + rng.standard_normal((1, SF_T, SF_H, SF_D))).astype(np.float32)
    comb = np.concatenate([u, -z], axis=-1).reshape(1, SF_T, -1)
    ini = np.zeros((1, SF_H, SF_D), np.float32)
    bias = np.zeros((SF_H, SF_D), np.float32)
    reps = 0
    t0 = time.perf_counter()
    with threadpool_limits(limits=cores):
        while True:
            O.scan_forward(comb, ini, bias, 6, 6, SF_D, 1, True, "f32")
            reps += 1
            el = time.perf_counter() - t0
            if el >= seconds_target:
                break
    per_row = scan_fwd_bytes() / SF_B
    return {"value": round(per_row * reps / el / 1e9, 3), "unit": "GB/s", "cores": cores,
            "cpu": cpu_model(), "kind": "port",
            "sample": f"{reps} x the scan forward of 1 of the {SF_B} batch rows "
                      f"(18 heads, T={SF_T}, D={SF_D}, r=1), fp32 numpy, {el:.1f} s"}


def scan_fwd_main(args):
    """one launch of the scan forward over bf16 head-major values
    (B, 18, T, D) with head-major per-element logits (B, 18, T, D) = -z."""
    import torch
    from nanochat_amd import _native as N
    from nanochat_amd.ops import ltv_hm_fast as hm

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(0)
    shape = (SF_B, SF_H, SF_T, SF_D)
    u = torch.randn(shape, generator=g, device=dev).to(torch.bfloat16)
    logits = (-(2.0 + torch.randn(shape, generator=g, device=dev))).to(torch.bfloat16)
    inits = torch.zeros((SF_B, SF_H, SF_D), dtype=torch.bfloat16, device=dev)
    bias = torch.zeros((SF_H, SF_D), dtype=torch.float32, device=dev)

    def step():
        return hm.scan_forward(u, logits, inits, bias, 6, 6, SF_D, 1, True)

    settled = settle(step, args.settle_s)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    with N.KernelRecorder() as rec:
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
    if args.calibrate_copy:
        src = torch.empty(COPY_CAL_BYTES, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
    ms = rec.durations_ms()["scan_fwd"]
    avg_us = sum(ms) / len(ms) * 1e3
    nbytes = scan_fwd_bytes()
    ach = nbytes / (avg_us * 1e-6) / 1e9
    traffic, traffic_src = profiled_traffic("scan_fwd", "scan_fwd_r1_traffic.json")
    ms_per_step = elapsed * 1e3 / args.steps
    out = {
        "metric": "standalone EWMA scan forward HBM GB/s (%peak), bf16 [32,3,6,1024,128], "
                  "per-element decay",
        "value": round(nbytes * args.steps / elapsed / 1e9, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": {"seconds": args.settle_s, "steps": settled},
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "configs[1]: standalone scan forward, per-element decay (r = 1)",
                   "B": SF_B, "heads": SF_H, "T": SF_T, "D": SF_D, "r": 1,
                   "parallelism": "single GPU"},
        "roofline": {"kernel": "scan_fwd", "bound": "hbm", "achieved": round(ach, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "traffic_source": traffic_src,
                     "avg_us": round(avg_us, 2), "work_per_launch": nbytes,
                     "peak_measured": measured_peak("scan_fwd_r1", "hbm"),
                     "frac_measured": (round(ach / measured_peak("scan_fwd_r1", "hbm"), 4)
                                       if measured_peak("scan_fwd_r1", "hbm") else None),
                     "peak_measured_source": "profiles/peaks.json"},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = scan_fwd_cpu_baseline(args.cpu_seconds)
    emit(out)


# long-sequence prefill
PF_B, PF_T = 8, 8192


def prefill_main(args):
    """configs[4]'s prefill: one forward of the drop-in filter (pack, bf16 MFMA
    projection, scan) on x bf16 [8, 8192, 768] ~ N(0, 1), c.weight ~
    N(0, 1/768) with the 18 gate rows scaled by 1.5 and logit_bias = -3, so
    logit + bias ~ N(-3, 1.5) and the decay a = sigmoid(z), z ~ N(3, 1.5), sits
    around 0.95 (long memory).  value = tokens / s of the forward."""
    import torch
    from nanochat_amd import _native as N
    from nanochat_amd.ltv.ltv_filter import LtvInitValues
    from nanochat_amd.ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan_qkv_filter import (
        LtvCudaFusedConcatHeadMajorRegisterCastBlellochScanQkvFilter as Filter,
    )

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    f = Filter(NH, NKVH, D, R)
    with torch.no_grad():
        f.c.weight.normal_(0.0, C ** -0.5)
        f.c.weight.view(H, D + DA, C)[:, D:] *= 1.5
        f.logit_bias.fill_(-3.0)
        f.init_param.normal_(0.0, C ** -0.5)
    f = f.to(dev)
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randn(PF_B, PF_T, C, generator=g, device=dev).to(torch.bfloat16)
    none = LtvInitValues()

    def step():
        with torch.no_grad():
            return f(x, none)

    settled = settle(step, args.settle_s)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    with N.KernelRecorder() as rec:
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
    if args.calibrate_copy:
        src = torch.empty(COPY_CAL_BYTES, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
    M = PF_B * PF_T
    work = {"pack_weight": ("hbm", F * C * 4 + FP * C * S_IO),
            "qkv_project_fwd": ("mfma", 2 * M * C * F),
            "scan_fwd": ("hbm", M * (F + H * D) * S_IO + PF_B * H * D * S_IO + 4 * H * DA)}
    kernels = {}
    for name, ms in rec.durations_ms().items():
        bound, amount = work[name]
        avg = sum(ms) / len(ms)
        if bound == "hbm":
            ach, peak, unit = amount / (avg * 1e-3) / 1e9, HBM_PEAK_GBS, "GB/s"
        else:
            ach, peak, unit = amount / (avg * 1e-3) / 1e12, BF16_PEAK_TFLOPS, "TFLOP/s"
        mp = measured_peak(name, bound)
        kernels[name] = {"bound": bound, "avg_us": round(avg * 1e3, 2), "launches": len(ms),
                         "achieved": round(ach, 1), "peak": peak, "unit": unit,
                         "frac": round(ach / peak, 4), "work_per_launch": amount,
                         "peak_measured": mp,
                         "frac_measured": round(ach / mp, 4) if mp else None}
    dominant = max(kernels, key=lambda k: kernels[k]["avg_us"] * kernels[k]["launches"])
    dk_ = kernels[dominant]
    traffic, traffic_src = profiled_traffic(dominant, "prefill_traffic.json")
    out = {
        "metric": "long-sequence prefill: LTV QKV filter forward tokens/s at B8 T8192 C768",
        "value": round(M * args.steps / elapsed, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": {"seconds": args.settle_s, "steps": settled},
        "ms_per_step": round(elapsed * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "configs[4] prefill: filter forward, decay sigmoid(N(3, 1.5))",
                   "B": PF_B, "T": PF_T, "C": C, "n_head": NH, "n_kv_head": NKVH,
                   "head_dim": D, "r": R, "parallelism": "single GPU"},
        "roofline": {"kernel": dominant, "bound": dk_["bound"], "achieved": dk_["achieved"],
                     "peak": dk_["peak"], "unit": dk_["unit"], "frac": dk_["frac"],
                     "traffic": traffic, "traffic_source": traffic_src,
                     "peak_measured": dk_["peak_measured"], "frac_measured": dk_["frac_measured"],
                     "peak_measured_source": "profiles/peaks.json"},
        "kernels": kernels,
    }
    emit(out)


# decode
DC_B, DC_T0, DC_N = 64, 16, 256


def decode_main(args):
    """configs[4]'s decode: B = 64 sequences, a 16-token prefill, then 256
    single-token steps through LtvCombinedQkvComputerModule and a KVCache (the
    filter state carried in the cache's last q/k/v rows).  A step is one token
    for the whole batch; ``--steps`` counts passes over the 256 tokens.
    value = decoded tokens / s through the module (what a serving loop calling
    the module sees, host dispatch included).  The same 256 steps captured in
    one HIP graph of fused decode kernels (each step's rows feeding the next)
    and replayed give the GPU-side rate without the Python dispatch."""
    import torch
    from nanochat_amd import _native as N
    from nanochat_amd.gpt_config import ChunksAndHistory
    from nanochat_amd.kv_cache import KVCache
    from nanochat_amd.ltv_combined_qkv_computer_module import LtvCombinedQkvComputerModule
    from nanochat_amd.ltv_cuda_fused_concat_head_major_register_cast_blelloch_scan_qkv_filter import (
        LtvCudaFusedConcatHeadMajorRegisterCastBlellochScanQkvFilter as Filter,
    )
    from nanochat_amd.ops import ltv_hm_fast as hm

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    f = Filter(NH, NKVH, D, R)
    with torch.no_grad():
        f.c.weight.normal_(0.0, C ** -0.5)
        f.c.weight.view(H, D + DA, C)[:, D:] *= 1.5
        f.logit_bias.fill_(-3.0)
        f.init_param.normal_(0.0, C ** -0.5)
    f = f.to(dev)
    m = LtvCombinedQkvComputerModule(0, f)
    g = torch.Generator(device=dev).manual_seed(0)
    xs = torch.randn(DC_B, DC_T0 + DC_N, C, generator=g, device=dev).to(torch.bfloat16)

    def new_cache():
        cache = KVCache(DC_B, NH, NKVH, DC_T0 + DC_N, D, 1,
                        [ChunksAndHistory(2147483647, 1, 1)])
        with torch.no_grad():
            m(xs[:, :DC_T0], cache)
        return cache

    def decode_pass(cache):
        with torch.no_grad():
            for t in range(DC_T0, DC_T0 + DC_N):
                m(xs[:, t:t + 1], cache)

    settled = settle(lambda: decode_pass(new_cache()), args.settle_s)
    for _ in range(max(args.warmup, 1)):
        decode_pass(new_cache())
    caches = [new_cache() for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for c in caches:
        decode_pass(c)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    tokens = DC_B * DC_N * args.steps

    # the fused kernel alone (HIP events), and the 256 steps as one HIP graph
    wpack = f._packed_weight()
    bias = f.logit_bias.detach().float().contiguous()
    with N.KernelRecorder() as rec:
        decode_pass(new_cache())
        torch.cuda.synchronize()
    cache = new_cache()
    last = cache.last_qkv
    prev0 = tuple(t.special[0].clone() for t in (last.q, last.k, last.v))

    def chain():
        prev = prev0
        for t in range(DC_T0, DC_T0 + DC_N):
            out = hm.decode_step(xs[:, t], wpack, prev, bias, NH, NKVH, DA, R, True)
            prev = (out[:, :NH], out[:, NH:NH + NKVH], out[:, NH + NKVH:])
        return out

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        chain()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        chain()
    graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        graph.replay()
    torch.cuda.synchronize()
    graph_s = time.perf_counter() - t0

    ms = rec.durations_ms()["qkv_decode"]
    avg_us = sum(ms) / len(ms) * 1e3
    fp = hm.packed_width(H, D, DA)
    nbytes = fp * C * S_IO + DC_B * (C + 2 * H * D) * S_IO  # weight, x, previous and new rows
    ach = nbytes / (avg_us * 1e-6) / 1e9
    out = {
        "metric": "decode: LTV QKV filter tokens/s at B64 (256 single-token steps, KV cache)",
        "value": round(tokens / elapsed, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": {"seconds": args.settle_s, "steps": settled},
        "ms_per_step": round(elapsed * 1e3 / (args.steps * DC_N), 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "configs[4] decode: 256 steps at B = 64 after a 16-token prefill, "
                               "through LtvCombinedQkvComputerModule + KVCache",
                   "B": DC_B, "prefill": DC_T0, "decode_steps": DC_N, "C": C, "n_head": NH,
                   "n_kv_head": NKVH, "head_dim": D, "r": R, "parallelism": "single GPU"},
        "graph": {"tokens_per_s": round(tokens / graph_s, 1),
                  "us_per_step": round(graph_s * 1e6 / (args.steps * DC_N), 2)},
        "roofline": {"kernel": "qkv_decode", "bound": "hbm", "achieved": round(ach, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                     "traffic": None, "avg_us": round(avg_us, 2), "work_per_launch": nbytes,
                     "peak_measured": measured_peak("qkv_decode", "hbm"),
                     "frac_measured": (round(ach / measured_peak("qkv_decode", "hbm"), 4)
                                       if measured_peak("qkv_decode", "hbm") else None),
                     "peak_measured_source": "profiles/peaks.json"},
    }
    emit(out)


def gpt_main(args):
    """one training step (forward + backward, no optimizer) of the
    12-layer d12 GPT on B=16, T=1024 token ids ~ U[0, 65536), random-init weights,
    bf16 autocast.  The filter's share is the summed duration of its library
    calls (HIP events on the launch stream) over the step time."""
    import torch
    from nanochat_amd import _native as N
    from nanochat_amd.gpt import GPT, GPTConfig

    Bg, Tg = 16, 1024
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    cfg = GPTConfig()
    model = GPT(cfg).to(dev)
    model.init_weights(randomise_output_projections=True)
    model.wte.to(dtype=torch.bfloat16)
    g = torch.Generator(device=dev).manual_seed(0)
    idx = torch.randint(0, cfg.vocab_size, (Bg, Tg), generator=g, device=dev)
    tgt = torch.randint(0, cfg.vocab_size, (Bg, Tg), generator=g, device=dev)

    def step():
        model.zero_grad(set_to_none=True)
        with torch.autocast(device_type="cuda", dtype=torch.bfloat16):
            loss = model(idx, tgt)
        loss.backward()

    settled = settle(step, args.settle_s)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    # the filter's calls timed with HIP events in a second pass (an event record
    # idles the GPU for several microseconds, so the timed steps run without)
    with N.KernelRecorder() as rec:
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
    durs = rec.durations_ms()
    filter_ms = sum(sum(v) for v in durs.values()) / args.steps
    ms_per_step = elapsed * 1e3 / args.steps
    out = {
        "metric": "GPT d12 training step tokens/s (fwd+bwd) and LTV filter share of the step",
        "value": round(Bg * Tg * args.steps / elapsed, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle": {"seconds": args.settle_s, "steps": settled},
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "configs[3]: 12-layer d12 GPT, filter in every layer, fwd+bwd "
                               "(no optimizer step)",
                   "B": Bg, "T": Tg, "n_layer": cfg.n_layer, "n_embd": cfg.n_embd,
                   "vocab": cfg.vocab_size, "parallelism": "single GPU"},
        "filter_ms_per_step": round(filter_ms, 4),
        "filter_share": round(filter_ms / ms_per_step, 4),
        "filter_kernels_us": {k: round(sum(v) / len(v) * 1e3, 2) for k, v in durs.items()},
    }
    emit(out)


if __name__ == "__main__":
    main()
