"""CPU checks of the C-ABI library: it loads, exports every function declared in
include/nanochat_filter_amd.h, and the ctypes binding covers exactly those.
No compute calls (there is no GPU here)."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nanochat_filter_amd.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*(ltv_[a-z0-9_]+)\s*\(",
                       src, flags=re.M)
    return sorted(set(names))


def declared_arg_counts():
    """{name: number of parameters} of every declaration in the header."""
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    out = {}
    for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*(ltv_[a-z0-9_]+)\s*"
                         r"\(([^;]*?)\)\s*;", src, flags=re.M | re.S):
        args = " ".join(m.group(2).split())
        out[m.group(1)] = 0 if args in ("", "void") else len(re.split(r",(?![^\[]*\])", args))
    return out


def test_ctypes_argument_counts_match_header():
    """A ctypes prototype with one argument too few or too many shifts every
    later argument; each binding has exactly the header's parameter count."""
    from nanochat_amd import _native as N
    counts = declared_arg_counts()
    bad = {n: (len(args), counts.get(n)) for n, (_, args) in N.SIGNATURES.items()
           if len(args) != counts.get(n)}
    assert not bad, bad


def test_header_declares_entry_points():
    names = declared_functions()
    for must in ("ltv_hm_scan_forward", "ltv_hm_scan_backward", "ltv_qkv_project_forward",
                 "ltv_qkv_project_backward", "ltv_linear_transpose_forward",
                 "ltv_linear_transpose_backward"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from nanochat_amd import _native as N
    if not os.path.exists(N.LIB_PATH):
        pytest.skip("library not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(N.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_binding_matches_header():
    from nanochat_amd import _native as N
    assert sorted(N.SIGNATURES) == declared_functions()


def test_abi_version_and_host_only_queries():
    from nanochat_amd import _native as N
    if not os.path.exists(N.LIB_PATH):
        pytest.skip("library not built")
    lib = N.load()
    assert lib.ltv_abi_version() == 11
    # d12: 18 heads x (128 + 1) = 2322 -> padded to a multiple of 128; 18 logits -> 24
    assert lib.ltv_qkv_packed_width(18, 128, 1) == 2432
    assert lib.ltv_qkv_logit_width(18, 1) == 24
    assert lib.ltv_hm_scan_backward_workspace_size(1, 32, 1024, 6, 6, 1, 128) >= 32 * 18 * 4
    assert lib.ltv_qkv_project_backward_workspace_size(32768, 768, 18, 128, 1) > 0
    # reference-layout backward, fp32 at d12: grad_weight's 19 x 6 tiles of
    # 128 x 128 split over B T into S fp32 partials of F x K; a single tile
    # row and column with B T = 256 (one split): none
    ws = lib.ltv_linear_transpose_backward_workspace_size(N.DTYPE_F32, 32, 1024, 768, 2322, 0)
    assert ws > 0 and ws % (2322 * 768 * 4) == 0 and ws // (2322 * 768 * 4) >= 2
    assert lib.ltv_linear_transpose_backward_workspace_size(N.DTYPE_F32, 1, 256, 64, 100, 0) == 0
    # chained scan forward: 256-byte header + one 8-byte word per channel of
    # every chunk but a sequence's last.  configs[4] prefill (8 x 18 heads x 2
    # slabs of 64 channels): 16 chunks of 512 steps; fp32: slabs of 32
    # channels; d12 (1,152 tile workgroups), fewer than 8 chunks (T = 3584),
    # gate groups that are neither whole lanes nor r = 1, or T = 0: no chained
    # kernel
    assert lib.ltv_hm_scan_forward_chain_workspace_size(1, 8, 8192, 6, 6, 1, 128) == \
        256 + 8 * 18 * 2 * 15 * 64 * 8
    assert lib.ltv_hm_scan_forward_chain_workspace_size(0, 2, 4096, 6, 6, 1, 128) == \
        256 + 2 * 18 * 4 * 7 * 32 * 8
    assert lib.ltv_hm_scan_forward_chain_workspace_size(1, 2, 3584, 6, 6, 1, 128) == 0
    assert lib.ltv_hm_scan_forward_chain_workspace_size(1, 2, 3585, 6, 6, 1, 128) > 0
    assert lib.ltv_hm_scan_forward_chain_workspace_size(1, 32, 1024, 6, 6, 1, 128) == 0
    assert lib.ltv_hm_scan_forward_chain_workspace_size(1, 2, 64, 1, 1, 32, 4) == 0
    assert lib.ltv_hm_scan_forward_chain_workspace_size(1, 2, 0, 1, 1, 1, 128) == 0
    # chained scan backward: the same layout, one word per channel of a whole
    # head (CL V = 128) per chunk but a sequence's first.  B = 8 at d12 heads
    # (144 sequences): 16 chunks of 64 steps (16 channel lanes x 4 time groups
    # x 4 steps x 4 wavefronts); fp32: 32 channel lanes, chunks of 32 steps;
    # 256 sequences and more (B = 16: 288; d12: 576), one chunk (T = 64), gate
    # groups of 4 channels, or T = 0: no chained kernel
    assert lib.ltv_hm_scan_backward_chain_workspace_size(1, 8, 1024, 6, 6, 1, 128) == \
        256 + 8 * 18 * 15 * 128 * 8
    assert lib.ltv_hm_scan_backward_chain_workspace_size(0, 2, 1024, 6, 6, 1, 128) == \
        256 + 2 * 18 * 31 * 128 * 8
    assert lib.ltv_hm_scan_backward_chain_workspace_size(1, 16, 1024, 6, 6, 1, 128) == 0
    assert lib.ltv_hm_scan_backward_chain_workspace_size(1, 32, 1024, 6, 6, 1, 128) == 0
    assert lib.ltv_hm_scan_backward_chain_workspace_size(1, 2, 64, 6, 6, 1, 128) == 0
    assert lib.ltv_hm_scan_backward_chain_workspace_size(1, 2, 1024, 1, 1, 32, 4) == 0
    assert lib.ltv_hm_scan_backward_chain_workspace_size(1, 2, 0, 1, 1, 1, 128) == 0
    # the scan backward's own workspace holds the chained kernel's dbias
    # partials (one per (b, h, chunk)) as well as the tile kernel's
    assert lib.ltv_hm_scan_backward_workspace_size(1, 8, 1024, 6, 6, 1, 128) >= 8 * 18 * 16 * 4
    # argument errors are reported without touching a device
    rc = lib.ltv_qkv_project_forward(None, None, None, None, 2, 8, 12, 3, 64, 1, None)
    assert rc == 2 and "multiple of 8" in N.last_error()
    rc = lib.ltv_hm_scan_forward(7, None, None, None, None, None, None, None, None, None, None,
                                 None, 1, 1, 1, 1, 1, 1, 1, None)
    assert rc == 1
    # look-back: P >= T is the full recurrence (same workspace); chunk windows
    # need the warm-up buffers on top; bad chunking is an argument error
    full = lib.ltv_hm_scan_backward_workspace_size(1, 4, 64, 2, 1, 1, 16)
    assert lib.ltv_hm_look_back_scan_backward_workspace_size(1, 4, 64, 2, 1, 1, 16,
                                                             2147483647, 1, 1) == full
    assert lib.ltv_hm_look_back_scan_backward_workspace_size(1, 4, 64, 2, 1, 1, 16,
                                                             64, 5, 3) == full
    # 4 x 4 heads x 13 windows x 8 warm-up rows x 16 channels of bf16 states alone
    assert lib.ltv_hm_look_back_scan_backward_workspace_size(1, 4, 64, 2, 1, 1, 16,
                                                             16, 4, 9) > 4 * 4 * 13 * 8 * 16 * 2
    s3, s4 = (ctypes.c_int64 * 3)(1, 1, 1), (ctypes.c_int64 * 4)(1, 1, 1, 1)
    rc = lib.ltv_hm_look_back_scan_forward(1, None, s3, None, s3, None, None, s4, None, s4,
                                           None, s4, 1, 1, 1, 1, 1, 1, 4, 0, 1, 1, None)
    assert rc == 1 and "Q >= 1" in N.last_error()
    # a view whose in-tile byte offsets would pass 2 GiB is refused before any
    # launch (the scan tiles address memory through 32-bit offsets); the dummy
    # pointer is never dereferenced
    dummy = ctypes.create_string_buffer(64)
    p = ctypes.cast(dummy, ctypes.c_void_p)
    B, T, NH, NKVH, Da, r = 1, 8, 1, 0, 1, 128
    wide = 1 << 21  # elements per time step: 1,026 steps x 4 MiB > 2 GiB
    cs = (ctypes.c_int64 * 3)(T * wide, wide, 1)
    ins = (ctypes.c_int64 * 3)(128, 128, 1)
    outs = (ctypes.c_int64 * 4)(T * 128, T * 128, 128, 1)
    bias = (ctypes.c_float * 1)(0.0)
    rc = lib.ltv_hm_look_back_scan_forward(1, p, cs, p, ins, bias, p, outs, p, outs, p, outs,
                                           B, T, NH, NKVH, Da, r, 2147483647, 1, 1, 1, None)
    assert rc == 2 and "32-bit tile offsets" in N.last_error(), N.last_error()
    # so is a negative time stride (the offsets are unsigned)
    back = (ctypes.c_int64 * 3)(T * 130, -130, 1)
    rc = lib.ltv_hm_look_back_scan_forward(1, p, back, p, ins, bias, p, outs, p, outs, p, outs,
                                           B, T, NH, NKVH, Da, r, 2147483647, 1, 1, 1, None)
    assert rc == 2 and "negative" in N.last_error(), N.last_error()


def test_ops_import_without_gpu():
    import torch
    import nanochat_amd.ops  # noqa: F401
    assert hasattr(torch.ops.nanochat_cuda,
                   "ltv_fused_concat_head_major_register_cast_blelloch_scan_cuda_op")
    for variant in ("blelloch", "sequential"):
        assert hasattr(torch.ops.nanochat_cuda,
                       f"ltv_look_back_fused_concat_head_major_register_cast_{variant}_scan_cuda_op")
    assert hasattr(torch.ops.nanochat_amd, "qkv_filter")
    assert hasattr(torch.ops.nanochat_amd, "qkv_filter_backward")


def test_product_path_refuses_cpu_tensors():
    import torch
    import nanochat_amd.ops  # noqa: F401
    x = torch.zeros(1, 2, 8, dtype=torch.bfloat16)
    w = torch.zeros(2 * (8 + 1) * 3, 8)
    inits = torch.zeros(1, 6, 8, dtype=torch.bfloat16)
    bias = torch.zeros(6, 1)
    with pytest.raises(RuntimeError, match="GPU tensors"):
        torch.ops.nanochat_amd.qkv_filter(x, w, inits, bias, 2, 2, 1, 8)


def test_chain_error_mailbox_and_controls_host_side():
    """The chain error mailbox reads 0 before any chained launch (and never
    allocates or touches the device for that), and the test controls refuse
    a negative spin bound and accept the defaults back."""
    from nanochat_amd import _native as N
    if not os.path.exists(N.LIB_PATH):
        pytest.skip("library not built")
    lib = N.lib()
    assert lib.ltv_chain_take_error() == 0
    assert lib.ltv_chain_set_test_controls(-1, 0) == 1  # LTV_ERR_INVALID_ARG
    assert "spin_max" in N.last_error()
    assert lib.ltv_chain_set_test_controls(0, 0) == 0
    assert lib.ltv_chain_take_error() == 0


def test_look_back_windows_per_lane_control_host_side():
    """The short-window backward's windows-per-lane control refuses a negative
    value and accepts any positive one and 0 (automatic) back."""
    from nanochat_amd import _native as N
    if not os.path.exists(N.LIB_PATH):
        pytest.skip("library not built")
    lib = N.lib()
    assert lib.ltv_lb_set_windows_per_lane(-1) == 1  # LTV_ERR_INVALID_ARG
    assert "wpl" in N.last_error()
    assert lib.ltv_lb_set_windows_per_lane(3) == 0
    assert lib.ltv_lb_set_windows_per_lane(0) == 0


def test_peaks_library_exports_its_header():
    """libltv_peaks.so (bench.py --workload peaks) exports every function
    include/ltv_peaks.h declares."""
    from nanochat_amd import _native as N
    path = os.path.join(os.path.dirname(N.LIB_PATH), "libltv_peaks.so")
    if not os.path.exists(path):
        pytest.skip("peaks library not built")
    src = re.sub(r"/\*.*?\*/", "", open(os.path.join(ROOT, "include", "ltv_peaks.h")).read(),
                 flags=re.S)
    names = re.findall(r"^\s*int\s+(ltv_[a-z0-9_]+)\s*\(", src, flags=re.M)
    assert sorted(names) == ["ltv_peak_mfma", "ltv_peak_overlap", "ltv_peak_stream"]
    lib = ctypes.CDLL(path)
    assert all(hasattr(lib, n) for n in names)
