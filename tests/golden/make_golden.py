"""Write golden vectors for the LTV scan from the reference's own Python oracle.

Run in the build container (where the read-only reference tree is mounted):

    python tests/golden/make_golden.py /root/reference

It loads ``nanochat/ops/ltv_reference_ops.py`` by file path (that file imports
only torch), runs ``ltv_fused_concat_head_major_register_cast_blelloch_scan_minimal``
(``ltv_reference_ops.py:162-192``) and, for the look-back cases with several
chunk windows, ``ltv_look_back_fused_concat_head_major_register_cast_sequential_scan_minimal``
(``:37-124``), forward and, through autograd, backward
(``QuantizedStateUpdate``, ``:7-34``) on small seeded inputs with the sigmoid
gate on, in fp32 and in bf16, and stores inputs and outputs as ``.npz`` data
(bf16 as uint16 bit patterns).  These cases are what the closed-form and
finite-difference checks cannot pin: torch's sigmoid rounding and the bf16
re-quantised state used by the alpha gradient.

The fixtures are data only; nothing under tests/ imports the reference at test
time, and the GPU box never sees the reference tree.
"""

from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

# (name, dtype, B, T, NH, NKVH, Da, r, seed)
CASES = [
    ("f32_r8", torch.float32, 2, 37, 2, 1, 1, 8, 0),
    ("f32_r2", torch.float32, 2, 19, 1, 1, 4, 2, 1),
    ("f32_r1", torch.float32, 1, 33, 1, 1, 8, 1, 2),
    ("bf16_r8", torch.bfloat16, 2, 37, 2, 1, 1, 8, 3),
    ("bf16_r2", torch.bfloat16, 2, 19, 1, 1, 4, 2, 4),
    ("bf16_r1", torch.bfloat16, 1, 33, 1, 1, 8, 1, 5),
    ("bf16_r16_t64", torch.bfloat16, 1, 64, 1, 1, 1, 16, 6),
]

# Look-back cases, several chunk windows each:
# (name, dtype, B, T, NH, NKVH, Da, r, P, Q, K, seed)
LOOK_BACK_CASES = [
    ("f32_p8q6k4", torch.float32, 2, 37, 1, 1, 2, 2, 8, 6, 4, 10),
    ("f32_p5q2k6", torch.float32, 1, 23, 1, 1, 1, 8, 5, 2, 6, 11),  # warm-up longer than Q
    ("f32_r1_p4q3k3", torch.float32, 1, 13, 1, 1, 4, 1, 4, 3, 3, 12),
    ("bf16_p16q16k9", torch.bfloat16, 2, 50, 2, 1, 1, 16, 16, 16, 9, 13),
    ("bf16_p0q3k2", torch.bfloat16, 1, 11, 1, 1, 2, 4, 0, 3, 2, 14),  # empty first chunk
]


def _load_reference(ref_root: str):
    path = os.path.join(ref_root, "nanochat", "ops", "ltv_reference_ops.py")
    spec = importlib.util.spec_from_file_location("ltv_reference_ops_golden", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    return t.numpy().copy()


def make_case(ref, name, dtype, B, T, NH, NKVH, Da, r, seed, pqk=None):
    g = torch.Generator().manual_seed(seed)
    H = NH + 2 * NKVH
    D = Da * r
    F = H * (D + Da)
    combined = torch.randn(B, T, F, generator=g).to(dtype)
    # gate logits centred so that alpha spans (0, 1) with tails near both ends
    gate = torch.randn(B, T, H, Da, generator=g) * 2.0
    c4 = combined.view(B, T, H, D + Da)
    c4[..., D:] = gate.to(dtype)
    inits = torch.randn(B, H, D, generator=g).to(dtype)
    logit_bias = (torch.randn(H, Da, generator=g) * 0.5).float()
    gq = torch.randn(B, NH, T, D, generator=g).to(dtype)
    gk = torch.randn(B, NKVH, T, D, generator=g).to(dtype)
    gv = torch.randn(B, NKVH, T, D, generator=g).to(dtype)

    c_ref = combined.clone().requires_grad_(True)
    i_ref = inits.clone().requires_grad_(True)
    b_ref = logit_bias.clone().requires_grad_(True)
    if pqk is None:
        oq, ok, ov = ref.ltv_fused_concat_head_major_register_cast_blelloch_scan_minimal(
            c_ref, i_ref, b_ref, NH, NKVH, Da, r, 2147483647, 1, 1, True
        )
        meta = [B, T, NH, NKVH, Da, r, 1 if dtype == torch.bfloat16 else 0]
    else:
        # ltv_reference_ops.py:37-124 with chunk restarts
        oq, ok, ov = ref.ltv_look_back_fused_concat_head_major_register_cast_sequential_scan_minimal(
            c_ref, i_ref, b_ref, NH, NKVH, Da, r, *pqk, True
        )
        meta = [B, T, NH, NKVH, Da, r, 1 if dtype == torch.bfloat16 else 0, *pqk]
    torch.autograd.backward([oq, ok, ov], [gq, gk, gv])
    return {
        "meta": np.array(meta, dtype=np.int64),
        "combined": _np(combined),
        "inits": _np(inits),
        "logit_bias": _np(logit_bias),
        "grad_q": _np(gq),
        "grad_k": _np(gk),
        "grad_v": _np(gv),
        "out_q": _np(oq),
        "out_k": _np(ok),
        "out_v": _np(ov),
        "grad_combined": _np(c_ref.grad),
        "grad_inits": _np(i_ref.grad),
        "grad_logit_bias": _np(b_ref.grad),
    }


def main():
    ref_root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    ref = _load_reference(ref_root)
    torch.set_num_threads(1)
    for case in CASES:
        data = make_case(ref, *case)
        out = os.path.join(HERE, f"scan_{case[0]}.npz")
        np.savez_compressed(out, **data)
        print("wrote", out, os.path.getsize(out), "bytes")
    for name, dtype, B, T, NH, NKVH, Da, r, P, Q, K, seed in LOOK_BACK_CASES:
        data = make_case(ref, name, dtype, B, T, NH, NKVH, Da, r, seed, pqk=(P, Q, K))
        out = os.path.join(HERE, f"look_back_{name}.npz")
        np.savez_compressed(out, **data)
        print("wrote", out, os.path.getsize(out), "bytes")


if __name__ == "__main__":
    main()
