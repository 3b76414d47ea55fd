"""Build the gfx950 HIP library ``libnanochat_filter_amd.so`` in-tree.

    python nanochat-filter_amd/build_lib.py [--jobs N]

Compiles each source under ``csrc/`` with hipcc for gfx950 (in parallel) and
links them into ``nanochat_amd/libnanochat_filter_amd.so``; the roofline
microbenchmarks of ``csrc/bench/`` go into ``nanochat_amd/libltv_peaks.so``.
Always rebuilds.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "nanochat_amd", "libnanochat_filter_amd.so")
SOURCES = ["ltv_scan_fwd_bf16.hip", "ltv_scan_fwd_f32.hip", "ltv_scan_bwd_bf16.hip",
           "ltv_scan_bwd_f32.hip", "ltv_scan_abi.hip", "ltv_scan_lb.hip", "ltv_gemm.hip", "ltv_decode.hip",
           "ltv_abi.cpp"]
ARCH = "gfx950"
# roofline microbenchmarks for bench.py --workload peaks: a library of their own
PEAKS_SOURCES = ["bench/ltv_peaks.hip"]
PEAKS_OUT = os.path.join(HERE, "nanochat_amd", "libltv_peaks.so")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm under /opt/rocm)")


def common_flags():
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-Wall",
        "-Wno-unused-function",
        # never let the compiler form packed fp32 ops (v_pk_*_f32)
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    ]


def _compile(src: str, obj: str) -> tuple[str, int, str]:
    cmd = [hipcc(), *common_flags(), "-c", os.path.join(CSRC, src), "-o", obj]
    p = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in (p.stdout + p.stderr).splitlines()
                    if "packed-fp32-ops" not in l)
    return src, p.returncode, err


def build(jobs: int | None = None, verbose: bool = True) -> str:
    """Compile and link both libraries; returns the filter library's path."""
    tmp = tempfile.mkdtemp(prefix="ltv_build_")
    try:
        targets = [(SOURCES, OUT), (PEAKS_SOURCES, PEAKS_OUT)]
        objs = {out: [] for _, out in targets}
        jobs = jobs or min(len(SOURCES) + len(PEAKS_SOURCES), os.cpu_count() or 1)
        with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
            futs = []
            for srcs, out in targets:
                for src in srcs:
                    obj = os.path.join(tmp, os.path.splitext(os.path.basename(src))[0] + ".o")
                    objs[out].append(obj)
                    futs.append(ex.submit(_compile, src, obj))
            failed = []
            for f in futs:
                src, rc, err = f.result()
                if err.strip() and verbose:
                    print(f"[build] {src}:\n{err}", file=sys.stderr)
                if rc != 0:
                    failed.append(src)
            if failed:
                raise RuntimeError(f"hipcc failed for {failed}")
        for _, out in targets:
            tmp_out = out + ".tmp"
            cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs[out], "-o",
                   tmp_out]
            p = subprocess.run(cmd, capture_output=True, text=True)
            if p.returncode != 0:
                raise RuntimeError(f"link failed:\n{p.stdout}\n{p.stderr}")
            os.replace(tmp_out, out)
            if verbose:
                print(f"[build] wrote {out} ({os.path.getsize(out)} bytes)")
        return OUT
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    build(ap.parse_args().jobs)
