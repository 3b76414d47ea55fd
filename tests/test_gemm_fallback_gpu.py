"""The register-staged GEMM kernels (csrc/ltv_gemm_mfma.hpp).

They serve the projection when the direct-to-LDS kernels cannot address an
operand (more than 2^30 - 2^20 elements, or an output past 2^31 bytes), and
``LTV_GEMM_CFG=fwd,dx,dw,rows,0`` routes every projection GEMM through them.
The tuning is read once per process, so the projection parity cases of
test_gemm_gpu.py (forward values and logits, grad_x, grad_weight against a
float64 product of the same bf16 operands; ragged token counts and partial
dW splits) run in one child process with that setting.
"""

from __future__ import annotations

import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)

_CHILD = """
import sys
sys.path[:0] = [{tests!r}, {pkg!r}, {oracle!r}]
import test_gemm_gpu as t
for args in [(2, 256, 768, 6, 6, 128, 1), (1, 100, 64, 1, 1, 16, 2), (3, 33, 128, 2, 1, 64, 64),
             (1, 300, 256, 3, 0, 12, 4)]:
    t.test_qkv_project_fast_path(*args)
    print("qkv_project", args, "ok", flush=True)
for M in (1, 257, 8192 + 64):
    t.test_projection_ragged_token_counts(M)
    print("ragged", M, "ok", flush=True)
"""


def test_register_staged_gemm_parity():
    code = _CHILD.format(tests=HERE, pkg=os.path.join(ROOT, "nanochat-filter_amd"),
                         oracle=os.path.join(ROOT, "oracle"))
    env = dict(os.environ, LTV_GEMM_CFG="1,1,0,4096,0")
    r = subprocess.run([sys.executable, "-c", code], env=env, cwd=ROOT, capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    assert r.stdout.count(" ok") == 7, r.stdout
