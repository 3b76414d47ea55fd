"""ctypes binding of ``libnanochat_filter_amd.so`` (the C ABI in
``include/nanochat_filter_amd.h``).

There is exactly one compute path: the HIP library.  If it is missing or fails
to load, every op raises -- nothing falls back to a CPU or PyTorch
implementation.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import NamedTuple

import torch

LIB_NAME = "libnanochat_filter_amd.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

DTYPE_F32 = 0
DTYPE_BF16 = 1

ERR_NAMES = {1: "LTV_ERR_INVALID_ARG", 2: "LTV_ERR_UNSUPPORTED", 3: "LTV_ERR_HIP",
             4: "LTV_ERR_WORKSPACE"}

_c_int = ctypes.c_int
_c_vp = ctypes.c_void_p
_c_sz = ctypes.c_size_t
_c_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes); kept in the order of include/nanochat_filter_amd.h
SIGNATURES = {
    "ltv_abi_version": (_c_int, []),
    "ltv_last_error": (ctypes.c_char_p, []),
    "ltv_hm_scan_forward": (
        _c_int,
        [_c_int, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp,
         _c_i64p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp],
    ),
    "ltv_hm_scan_forward_chain_workspace_size": (
        _c_sz, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "ltv_hm_scan_forward_ws": (
        _c_int,
        [_c_int, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp,
         _c_i64p, _c_vp, _c_sz, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp],
    ),
    "ltv_hm_scan_backward_workspace_size": (
        _c_sz, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "ltv_hm_scan_backward": (
        _c_int,
        [_c_int, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp,
         _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p,
         _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p,
         _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp,
         _c_vp, _c_sz, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp],
    ),
    "ltv_hm_scan_forward_split": (
        _c_int,
        [_c_int, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_vp, _c_i64p, _c_vp,
         _c_i64p, _c_vp, _c_i64p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp],
    ),
    "ltv_hm_scan_backward_split": (
        _c_int,
        [_c_int, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp,
         _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p,
         _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p,
         _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp,
         _c_vp, _c_sz, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp],
    ),
    # the look-back forms: the same arguments plus P, Q, K before use_sigmoid
    "ltv_hm_look_back_scan_forward": (
        _c_int,
        [_c_int, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp,
         _c_i64p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
         _c_int, _c_vp],
    ),
    "ltv_hm_look_back_scan_backward_workspace_size": (
        _c_sz, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "ltv_hm_look_back_scan_backward": (
        _c_int,
        [_c_int, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp,
         _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p,
         _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p,
         _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp,
         _c_vp, _c_sz, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
         _c_int, _c_vp],
    ),
    "ltv_hm_look_back_scan_forward_split": (
        _c_int,
        [_c_int, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_vp, _c_i64p, _c_vp,
         _c_i64p, _c_vp, _c_i64p, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
         _c_int, _c_int, _c_int, _c_vp],
    ),
    "ltv_hm_look_back_scan_forward_split_ws": (
        _c_int,
        [_c_int, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_int, _c_vp, _c_vp, _c_i64p,
         _c_vp,
         _c_i64p, _c_vp, _c_i64p, _c_vp, _c_sz, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
         _c_int, _c_int, _c_int, _c_int, _c_vp],
    ),
    "ltv_hm_look_back_scan_backward_split": (
        _c_int,
        [_c_int, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp,
         _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p,
         _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p,
         _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp,
         _c_vp, _c_sz, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
         _c_int, _c_vp],
    ),
    "ltv_hm_scan_backward_chain_workspace_size": (
        _c_sz, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    # the backward with a chain workspace: (chain workspace, bytes) after the workspace
    "ltv_hm_scan_backward_ws": (
        _c_int,
        [_c_int, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp,
         _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p,
         _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p,
         _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp,
         _c_vp, _c_sz, _c_vp, _c_sz, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
         _c_vp],
    ),
    "ltv_hm_look_back_scan_backward_split_ws": (
        _c_int,
        [_c_int, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_int, _c_vp,
         _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p,
         _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p,
         _c_vp, _c_i64p, _c_vp, _c_i64p, _c_int, _c_vp, _c_i64p, _c_vp,
         _c_vp, _c_sz, _c_vp, _c_sz, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
         _c_int, _c_int, _c_int, _c_vp],
    ),
    "ltv_linear_transpose_forward": (
        _c_int, [_c_int, _c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int, _c_vp]),
    "ltv_linear_transpose_backward": (
        _c_int,
        [_c_int, _c_vp, _c_vp, _c_vp, _c_int, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int,
         _c_vp],
    ),
    "ltv_linear_transpose_backward_workspace_size": (
        _c_sz, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "ltv_linear_transpose_backward_ws": (
        _c_int,
        [_c_int, _c_vp, _c_vp, _c_vp, _c_int, _c_vp, _c_vp, _c_vp, _c_sz, _c_int, _c_int, _c_int,
         _c_int, _c_vp],
    ),
    "ltv_qkv_packed_width": (_c_int, [_c_int, _c_int, _c_int]),
    "ltv_qkv_logit_width": (_c_int, [_c_int, _c_int]),
    "ltv_qkv_pack_weight": (
        _c_int, [_c_int, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int, _c_vp]),
    "ltv_qkv_project_forward": (
        _c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                 _c_vp]),
    "ltv_qkv_project_backward_workspace_size": (
        _c_sz, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "ltv_qkv_project_backward": (
        _c_int,
        [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_sz, _c_int, _c_int, _c_int, _c_int,
         _c_int, _c_vp],
    ),
    "ltv_qkv_project_backward_zero_padded": (
        _c_int,
        [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_sz, _c_int, _c_int, _c_int, _c_int,
         _c_int, _c_vp],
    ),
    "ltv_qkv_project_backward_input": (
        _c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp]),
    "ltv_qkv_project_backward_input_zero_padded": (
        _c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp]),
    "ltv_qkv_project_backward_weight": (
        _c_int,
        [_c_vp, _c_vp, _c_vp, _c_vp, _c_sz, _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp],
    ),
    "ltv_qkv_decode_step": (
        _c_int,
        [_c_vp, ctypes.c_int64, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64p, _c_vp, _c_vp,
         _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp],
    ),
    "ltv_qkv_decode_step_rows": (
        _c_int,
        [_c_vp, ctypes.c_int64, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64p, _c_vp, _c_vp,
         _c_vp, _c_vp, _c_vp, _c_i64p,
         _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp],
    ),
    "ltv_chain_take_error": (_c_int, []),
    "ltv_chain_set_test_controls": (_c_int, [_c_int, _c_int]),
    "ltv_lb_set_windows_per_lane": (_c_int, [_c_int]),
    "ltv_hm_scan_backward_noalloc_max_workspace": (_c_sz, []),
    "ltv_hm_scan_backward_noalloc": (
        _c_int,
        [_c_int, _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp,
         _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p,
         _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp, _c_i64p,
         _c_vp, _c_i64p, _c_vp, _c_i64p, _c_vp,
         _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp],
    ),
}

_lib = None
_lib_error: Exception | None = None
_lock = threading.Lock()


def load(path: str | None = None) -> ctypes.CDLL:
    """Load the library once; raise a RuntimeError naming the cause if it cannot be."""
    global _lib, _lib_error
    with _lock:
        if _lib is not None:
            return _lib
        p = path or LIB_PATH
        if not os.path.exists(p):
            _lib_error = RuntimeError(
                f"{LIB_NAME} not found at {p}: build it with "
                "`python nanochat-filter_amd/build_lib.py` (or __graft_entry__.build())"
            )
            raise _lib_error
        lib = ctypes.CDLL(p)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def lib() -> ctypes.CDLL:
    return _lib if _lib is not None else load()


def last_error() -> str:
    return lib().ltv_last_error().decode("utf-8", "replace")


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed ({ERR_NAMES.get(rc, rc)}): {last_error()}")


# ---------------------------------------------------------------------------
# argument helpers
# ---------------------------------------------------------------------------
def strides(t: torch.Tensor, n: int | None = None):
    s = list(t.stride())
    if n is not None:
        assert len(s) == n, (t.shape, n)
    return (ctypes.c_int64 * len(s))(*s)


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return DTYPE_F32
    if dt == torch.bfloat16:
        return DTYPE_BF16
    raise TypeError(f"LTV kernels support float32 and bfloat16 tensors, got {dt}")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    """The current HIP stream of t's device, as the raw handle the library
    takes (read without building a torch Stream object where torch offers it:
    host time matters on the single-token decode path)."""
    if _raw_stream is not None:
        return _raw_stream(t.device.index if t.device.index is not None
                           else torch.cuda.current_device())
    return torch.cuda.current_stream(t.device).cuda_stream


# Chain workspaces of the chained scan forward and backward (the library's
# *_ws entry points): zeroed once, left zeroed by every call, so one buffer per
# (device, stream) serves every later call on that stream, in either
# direction (calls on one stream run one after another).  Under graph capture
# each call gets a fresh zeroed buffer from the graph's pool (its zero fill is
# captured with it).
_CHAIN_WS: dict = {}

CHAIN_ERRORS = {1: "a chunk's wait for its carry ran past its bound",
                2: "the chain workspace was not zero at the launch"}


class ChainWorkspace(NamedTuple):
    """A chained call's workspace: hold ``buf`` until the library call has
    been made (the pointer is only valid while the tensor lives)."""
    buf: torch.Tensor | None
    ptr: int | None
    nbytes: int


_NO_CHAIN = ChainWorkspace(None, None, 0)


def chain_sync_check() -> bool:
    """Whether every chained call synchronises its stream and checks the
    library's error mailbox at once (LTV_CHAIN_SYNC_CHECK=1; the tests set
    it).  Otherwise a failure is reported by the next chained call."""
    return os.environ.get("LTV_CHAIN_SYNC_CHECK", "0") not in ("", "0")


def check_chain_errors() -> None:
    """Raise if a chained scan launched since the last check reported a
    failure (read from the library's host mailbox, no device
    synchronisation).  The chain workspaces are then dropped, so the next
    call starts from a fresh zeroed one."""
    code = lib().ltv_chain_take_error()
    if code == 0:
        return
    torch.cuda.synchronize()
    _CHAIN_WS.clear()
    raise RuntimeError(
        f"chained LTV scan failed (code {code}: {CHAIN_ERRORS.get(code, 'unknown')}); the "
        "outputs of chained scan calls since the previous check are invalid, and the chain "
        "workspaces have been reset")


def chain_workspace(device: torch.device, nbytes: int):
    """A 256-byte aligned, all-zero device buffer of at least ``nbytes`` bytes
    reserved for the chained scans on the current stream, or None when
    nbytes == 0."""
    if nbytes <= 0:
        return None
    n = (nbytes + 255) // 256 * 256
    if torch.cuda.is_current_stream_capturing():
        return torch.zeros(n, dtype=torch.uint8, device=device)
    key = (device.index if device.index is not None else torch.cuda.current_device(),
           torch.cuda.current_stream(device).cuda_stream)
    buf = _CHAIN_WS.get(key)
    if buf is None or buf.numel() < n:
        buf = torch.zeros(n, dtype=torch.uint8, device=device)
        _CHAIN_WS[key] = buf
    return buf


def chain_workspace_for(dtype: torch.dtype, device: torch.device, B: int, T: int, NH: int,
                        NKVH: int, Da: int, r: int, backward: bool = False) -> ChainWorkspace:
    """The chain workspace for this scan shape (pointer None and 0 bytes where
    the chained forward -- or, with ``backward``, the chained backward -- does
    not apply).  Raises first if an earlier chained call reported a failure."""
    size = (lib().ltv_hm_scan_backward_chain_workspace_size if backward
            else lib().ltv_hm_scan_forward_chain_workspace_size)
    nbytes = size(dtype_code(dtype), B, T, NH, NKVH, Da, r)
    if nbytes == 0:
        return _NO_CHAIN
    check_chain_errors()
    buf = chain_workspace(device, nbytes)
    return ChainWorkspace(buf, buf.data_ptr(), buf.numel())


def chain_done(cw: ChainWorkspace) -> None:
    """After a library call that was given ``cw``: with LTV_CHAIN_SYNC_CHECK
    set (and outside graph capture), wait for it and raise if it failed."""
    if cw.buf is None or not chain_sync_check() or torch.cuda.is_current_stream_capturing():
        return
    torch.cuda.current_stream(cw.buf.device).synchronize()
    check_chain_errors()


def require_device(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(
                f"LTV HIP kernels need GPU tensors, got a tensor on {t.device}")


# ---------------------------------------------------------------------------
# optional per-call timing: HIP events recorded on the launch stream around
# each library call while a recorder is active (used by bench.py)
# ---------------------------------------------------------------------------
class KernelRecorder:
    """Collects (name, start_event, end_event) for every instrumented call made
    while it is active.  Events are recorded on torch's current stream, which is
    the stream every op launches on."""

    def __init__(self):
        self.spans: list[tuple[str, TimingEvent, TimingEvent]] = []

    def __enter__(self):
        global _recorder
        _recorder = self
        return self

    def __exit__(self, *exc):
        global _recorder
        _recorder = None
        return False

    def durations_ms(self) -> dict[str, list[float]]:
        out: dict[str, list[float]] = {}
        for name, a, b in self.spans:
            out.setdefault(name, []).append(a.elapsed_time(b))
        return out


_recorder: KernelRecorder | None = None


# Timing events for the recorder, created through the HIP runtime this process
# already uses (torch's) with hipEventDisableSystemFence: a default event's
# system-scope fence writes back and invalidates the caches when it completes,
# which idles the GPU for about 10 us per record on MI355X and perturbs the
# next kernel.  These events only timestamp.
_HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000
_hip_rt = None


def _hip():
    global _hip_rt
    if _hip_rt is None:
        path = None
        with open("/proc/self/maps") as fh:
            for line in fh:
                if "libamdhip64" in line:
                    path = line.split()[-1]
                    break
        rt = ctypes.CDLL(path or "libamdhip64.so")
        rt.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(_c_vp), ctypes.c_uint]
        rt.hipEventRecord.argtypes = [_c_vp, _c_vp]
        rt.hipEventSynchronize.argtypes = [_c_vp]
        rt.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), _c_vp, _c_vp]
        rt.hipEventDestroy.argtypes = [_c_vp]
        _hip_rt = rt
    return _hip_rt


class TimingEvent:
    __slots__ = ("h",)

    def __init__(self):
        self.h = _c_vp()
        rc = _hip().hipEventCreateWithFlags(ctypes.byref(self.h), _HIP_EVENT_DISABLE_SYSTEM_FENCE)
        if rc != 0:
            raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")

    def record(self):
        rc = _hip().hipEventRecord(self.h, _c_vp(torch.cuda.current_stream().cuda_stream))
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def elapsed_time(self, end: "TimingEvent") -> float:
        rt = _hip()
        rt.hipEventSynchronize(end.h)
        ms = ctypes.c_float()
        rc = rt.hipEventElapsedTime(ctypes.byref(ms), self.h, end.h)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return ms.value

    def __del__(self):
        if self.h and _hip_rt is not None:
            _hip_rt.hipEventDestroy(self.h)


class span:
    """``with span("scan_fwd"): lib.call(...)`` -- no-op unless recording."""

    __slots__ = ("name", "ev")

    def __init__(self, name: str):
        self.name = name
        self.ev = None

    def __enter__(self):
        if _recorder is not None:
            a = TimingEvent()
            a.record()
            self.ev = a
        return self

    def __exit__(self, *exc):
        if self.ev is not None and _recorder is not None:
            b = TimingEvent()
            b.record()
            _recorder.spans.append((self.name, self.ev, b))
        return False
