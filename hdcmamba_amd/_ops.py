"""ctypes binding of libhdcmamba_hip.so and tensor-level wrappers.

The C ABI (include/hdcm.h) takes raw device pointers, element strides and a
hipStream_t.  These wrappers check tensors, allocate outputs and workspaces through
PyTorch's caching allocator and launch on torch's current stream.  There is no CPU
or fallback path: a missing library or a CPU tensor raises.
"""
from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_int64, c_size_t, c_void_p
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().with_name("libhdcmamba_hip.so")
ABI_VERSION = 2

HDCM_F32, HDCM_BF16 = 0, 1
_DTYPES = {torch.float32: HDCM_F32, torch.bfloat16: HDCM_BF16}

# name -> (restype, argtypes); mirrors include/hdcm.h
_PROTOS = {
    "hdcm_abi_version": (c_int, []),
    "hdcm_strerror": (ctypes.c_char_p, [c_int]),
    "hdcm_time_launches": (c_int, [c_void_p, c_void_p, c_int]),
    "hdcm_timed_launch_count": (c_int, []),
    "hdcm_set_option": (c_int, [c_int, c_int]),
    "hdcm_get_option": (c_int, [c_int]),
    "hdcm_norm_conv_fwd": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p,
                                   c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_float,
                                   c_int, c_void_p]),
    "hdcm_ssm_workspace_bytes": (c_size_t, [c_int64, c_int64, c_int64]),
    "hdcm_ssm_fwd": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_int64, c_void_p,
                             c_void_p, c_int64, c_void_p, c_size_t, c_int64, c_int64, c_int64, c_int, c_void_p]),
    "hdcm_ssm_fwd_noalloc": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_int64, c_void_p,
                                     c_void_p, c_int64, c_int64, c_int64, c_int64, c_int, c_void_p]),
    "hdcm_ssm_bwd_workspace_bytes": (c_size_t, [c_int64, c_int64, c_int64, c_int]),
    "hdcm_ssm_bwd": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                             c_void_p, c_void_p, c_size_t, c_int64, c_int64, c_int64, c_int, c_void_p]),
    "hdcm_gnorm_gate_bwd_workspace_bytes": (c_size_t, [c_int64, c_int64]),
    "hdcm_gnorm_gate_bwd": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_float, c_void_p,
                                    c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_void_p,
                                    c_size_t, c_int64, c_int64, c_int64, c_int, c_void_p]),
    "hdcm_slot_phi_prep": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_int64, c_int,
                                   c_void_p]),
    "hdcm_slot_phi_chain": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_int64, c_int,
                                    c_void_p]),
    "hdcm_slot_workspace_bytes": (c_size_t, [c_int64, c_int64, c_int64, c_int64, c_int64, c_int]),
    "hdcm_slot_state_fwd": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_size_t,
                                    c_int64, c_int64, c_int64, c_int64, c_int64, c_int, c_void_p]),
    "hdcm_slot_gate_fwd": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_float,
                                   c_void_p, c_size_t, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64,
                                   c_int64, c_int64, c_int64, c_int64, c_int64, c_int, c_void_p]),
    "hdcm_slot_attend_fwd": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p, c_int, c_void_p,
                                     c_size_t, c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_int64,
                                     c_int64, c_int64, c_int64, c_int, c_void_p]),
    "hdcm_rowln_fwd": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64,
                               c_int64, c_float, c_int, c_void_p]),
    "hdcm_rowln2_fwd": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_float, c_void_p,
                                c_void_p, c_float, c_int64, c_int64, c_int, c_void_p]),
    "hdcm_norm_conv_step_fwd": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p,
                                        c_void_p, c_void_p, c_int64, c_int64, c_int64, c_float, c_int,
                                        c_void_p]),
    "hdcm_mixer_step_fwd": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p,
                                    c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_float,
                                    c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64,
                                    c_int, c_void_p]),
    "hdcm_gnorm_gate_fwd": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p,
                                    c_float, c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int,
                                    c_void_p]),
    "hdcm_chunk_pos_advance": (c_int, [c_void_p, c_int64, c_void_p]),
    "hdcm_skinny_gemm_fwd": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64,
                                     c_void_p, c_int64, c_int64, c_int64, c_int64, c_int, c_void_p]),
    "hdcm_step_workspace_bytes": (c_size_t, []),
    "hdcm_norm_conv_in_proj_step_fwd": (c_int, [c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p,
                                                c_void_p, c_float, c_void_p, c_int64, c_void_p, c_int64, c_void_p,
                                                c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p, c_size_t,
                                                c_int, c_void_p]),
    "hdcm_gemm_fwd": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_int64,
                              c_int64, c_int, c_void_p]),
    "hdcm_rowln_gemm_fwd": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                    c_int64, c_int64, c_int64, c_float, c_int, c_void_p]),
    "hdcm_rowln_gemm_stats_fwd": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64,
                                          c_int64, c_void_p, c_int64, c_void_p, c_int64, c_int64, c_int64, c_int64,
                                          c_float, c_int, c_void_p]),
    "hdcm_row_sums_fwd": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int, c_void_p]),
    "hdcm_rowln_bwd_workspace_bytes": (c_size_t, [c_int64, c_int64]),
    "hdcm_rowln_bwd": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p,
                               c_void_p, c_void_p, c_size_t, c_int64, c_int64, c_float, c_int, c_void_p]),
    "hdcm_norm_conv_bwd_workspace_bytes": (c_size_t, [c_int64, c_int64, c_int64]),
    "hdcm_norm_conv_bwd": (c_int, [c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_void_p,
                                   c_void_p, c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p,
                                   c_void_p, c_size_t, c_int64, c_int64, c_int64, c_float, c_int, c_void_p]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Load libhdcmamba_hip.so (once) and declare its prototypes."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH.name} is not built; run `python -m hdcmamba_amd.build`")
        h = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _PROTOS.items():
            fn = getattr(h, name)
            fn.restype, fn.argtypes = res, args
        if h.hdcm_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH.name} ABI {h.hdcm_abi_version()} != expected {ABI_VERSION}")
        _lib = h
    return _lib


class HdcmError(RuntimeError):
    def __init__(self, op: str, code: int):
        super().__init__(f"{op}: {lib().hdcm_strerror(code).decode()} (status {code})")
        self.code = code


def _check(op: str, code: int) -> None:
    if code != 0:
        raise HdcmError(op, code)


def _dtype(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; expected float32 or bfloat16") from None


def _on_gpu(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError("hdcmamba_amd kernels need ROCm GPU tensors; got a tensor on "
                               f"{t.device} (there is no CPU path)")


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


_side_streams = {}


def side_stream(device) -> torch.cuda.Stream:
    """A second stream per device (default priority) for work that can overlap the
    current stream's kernels; callers fork and join it with wait_stream."""
    idx = torch.device(device).index
    if idx is None:
        idx = torch.cuda.current_device()
    s = _side_streams.get(idx)
    if s is None:
        s = _side_streams[idx] = torch.cuda.Stream(device=idx)
    return s


def _same(t: torch.Tensor, ref: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != ref.dtype:
        t = t.to(ref.dtype)
    if t.device != ref.device:
        raise RuntimeError(f"{name} is on {t.device}, expected {ref.device}")
    return t.contiguous()


def _rows2d(t: torch.Tensor, name: str):
    """(row stride) of a [..., W] tensor whose rows are uniformly strided."""
    if t.numel() == 0:  # no rows to address: any stride works, report a dense one
        return t.shape[-1]
    if t.stride(-1) != 1:
        raise RuntimeError(f"{name}: last dimension must be contiguous")
    rs = t.stride(-2) if t.dim() >= 2 else t.shape[-1]
    # all leading dims must collapse onto rows of stride rs
    expect = rs
    for d in range(t.dim() - 2, -1, -1):
        if t.shape[d] > 1 and t.stride(d) != expect:
            raise RuntimeError(f"{name}: leading dimensions must collapse to uniformly strided rows")
        expect *= t.shape[d]
    return rs


# ----------------------------------------------------------------------------- timing hook
def _hip_runtime() -> ctypes.CDLL:
    """The HIP runtime this process already uses (torch's copy, which libhdcmamba_hip.so
    binds to through the shared soname), with the event calls declared."""
    path = "libamdhip64.so.7"
    try:
        with open("/proc/self/maps") as f:
            for line in f:
                if "libamdhip64" in line:
                    path = line.split()[-1]
                    break
    except OSError:
        pass
    h = ctypes.CDLL(path)
    h.hipEventCreate.restype = c_int
    h.hipEventCreate.argtypes = [ctypes.POINTER(c_void_p)]
    h.hipEventDestroy.restype = c_int
    h.hipEventDestroy.argtypes = [c_void_p]
    h.hipEventSynchronize.restype = c_int
    h.hipEventSynchronize.argtypes = [c_void_p]
    h.hipEventElapsedTime.restype = c_int
    h.hipEventElapsedTime.argtypes = [ctypes.POINTER(c_float), c_void_p, c_void_p]
    return h


class _Timer:
    """Kernel durations of named calls (used by bench.py).

    For a call whose name is in ``active``, hdcm_time_launches arms event pairs for the
    call's kernels: the k-th kernel it launches records pair k from its own dispatch
    timestamps (begin, end), so no event packets enter the stream and each interval is
    exactly one kernel's execution."""

    max_launches = 8  # kernels per call that get events

    def __init__(self):
        self.active = set()
        self.events = {}
        self._rt = None
        self._armed = None

    def _event(self):
        if self._rt is None:
            self._rt = _hip_runtime()
        ev = c_void_p()
        if self._rt.hipEventCreate(ctypes.byref(ev)) != 0:
            raise RuntimeError("hipEventCreate failed")
        return ev.value

    def begin(self, name):
        if name not in self.active:
            return None
        n = self.max_launches
        starts = (c_void_p * n)(*[self._event() for _ in range(n)])
        stops = (c_void_p * n)(*[self._event() for _ in range(n)])
        _check("hdcm_time_launches", lib().hdcm_time_launches(starts, stops, n))
        return starts, stops

    def end(self, name, arrays):
        if arrays is None:
            return
        used = lib().hdcm_timed_launch_count()
        _check("hdcm_time_launches", lib().hdcm_time_launches(None, None, 0))
        starts, stops = arrays
        for k in range(used, self.max_launches):  # pairs no kernel recorded
            self._rt.hipEventDestroy(starts[k])
            self._rt.hipEventDestroy(stops[k])
        self.events.setdefault(name, []).append([(starts[k], stops[k]) for k in range(used)])

    def _elapsed(self, a, b):
        t = c_float()
        rc = self._rt.hipEventSynchronize(b) or self._rt.hipEventElapsedTime(ctypes.byref(t), a, b)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return t.value

    def collect(self):
        """{name: [[ms of kernel k of the call for k in its launches] per timed call]};
        releases the events."""
        torch.cuda.synchronize()
        out = {}
        for name, calls in self.events.items():
            out[name] = []
            for pairs in calls:
                out[name].append([self._elapsed(a, b) for a, b in pairs])
                for a, b in pairs:
                    self._rt.hipEventDestroy(a)
                    self._rt.hipEventDestroy(b)
        self.events = {}
        return out


timer = _Timer()

# launch options of the library (hdcm_set_option)
OPTIONS = {"ssm_spin_rounds": 1, "slot_seg_tiles": 2, "skinny_cols8_max_n": 3, "skinny_fold_tail": 4,
           "step_spin_rounds": 5}


class option:
    """Context manager that sets a library launch option and restores its previous value:
    ``with _ops.option("slot_seg_tiles", 8): ...``.  ssm_spin_rounds = polling rounds of the
    scan's look-back before it computes a missing total itself (0 forces that path);
    slot_seg_tiles = row tiles per slot segment (0 = automatic); skinny_cols8_max_n = widest
    skinny-GEMM output run with 8 columns per workgroup (0 = never); skinny_fold_tail = 1 runs
    the skinny GEMM's tiles past one round of resident workgroups as second tiles of the first
    workgroups (0 = a second round); step_spin_rounds = polling rounds of the fused decode front's
    GEMM workgroups for the conv rows before they count a timeout.  Launches read the value
    current when they are issued (a recorded graph keeps the value of its capture)."""

    def __init__(self, name, value):
        self.key = OPTIONS[name]
        self.value = int(value)

    def __enter__(self):
        self.old = lib().hdcm_get_option(self.key)
        _check("hdcm_set_option", lib().hdcm_set_option(self.key, self.value))
        return self

    def __exit__(self, *exc):
        _check("hdcm_set_option", lib().hdcm_set_option(self.key, self.old))
        return False


# ----------------------------------------------------------------------------- wrappers
def norm_conv(x, ln_w, ln_b, conv_w, conv_b, eps, out=None):
    """LayerNorm + causal depthwise conv: x [B,L,D] -> out [B,L,D] (x.dtype)."""
    _on_gpu(x)
    if x.dim() != 3:
        raise RuntimeError("norm_conv expects x of shape [B, L, D]")
    B, L, D = x.shape
    ln_w = _same(ln_w, x, "ln_w")
    ln_b = _same(ln_b, x, "ln_b")
    conv_b = _same(conv_b, x, "conv_b")
    conv_w = _same(conv_w.reshape(D, 4), x, "conv_w")
    if x.stride(2) != 1:
        x = x.contiguous()
    if out is None:
        out = torch.empty(B, L, D, device=x.device, dtype=x.dtype)
    ev = timer.begin("norm_conv")
    _check("hdcm_norm_conv_fwd", lib().hdcm_norm_conv_fwd(
        x.data_ptr(), x.stride(0), x.stride(1), ln_w.data_ptr(), ln_b.data_ptr(), conv_w.data_ptr(),
        conv_b.data_ptr(), out.data_ptr(), out.stride(0), out.stride(1), B, L, D, float(eps),
        _dtype(x), _stream(x)))
    timer.end("norm_conv", ev)
    return out


def norm_conv_bwd(grad_out, x, ln_w, ln_b, conv_w, eps):
    """Gradients of norm_conv: returns dx (x.dtype, [B,L,D]) and fp32 d_ln_w [D],
    d_ln_b [D], d_conv_w [D,4], d_conv_b [D]."""
    _on_gpu(grad_out, x)
    B, L, D = x.shape
    ln_w = _same(ln_w, x, "ln_w")
    ln_b = _same(ln_b, x, "ln_b")
    conv_w = _same(conv_w.reshape(D, 4), x, "conv_w")
    grad_out = _same(grad_out, x, "grad_out")
    if not grad_out.is_contiguous():  # e.g. the expanded gradient of a sum
        grad_out = grad_out.contiguous()
    if x.stride(2) != 1:
        x = x.contiguous()
    dx = torch.empty(B, L, D, device=x.device, dtype=x.dtype)
    f32 = dict(device=x.device, dtype=torch.float32)
    d_ln_w, d_ln_b, d_conv_b = torch.empty(D, **f32), torch.empty(D, **f32), torch.empty(D, **f32)
    d_conv_w = torch.empty(D, 4, **f32)
    nbytes = lib().hdcm_norm_conv_bwd_workspace_bytes(B, L, D)
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=x.device)
    _check("hdcm_norm_conv_bwd", lib().hdcm_norm_conv_bwd(
        grad_out.data_ptr(), grad_out.stride(0), grad_out.stride(1), x.data_ptr(), x.stride(0), x.stride(1),
        ln_w.data_ptr(), ln_b.data_ptr(), conv_w.data_ptr(), dx.data_ptr(), dx.stride(0), dx.stride(1),
        d_ln_w.data_ptr(), d_ln_b.data_ptr(), d_conv_w.data_ptr(), d_conv_b.data_ptr(), ws.data_ptr(), nbytes,
        B, L, D, float(eps), _dtype(x), _stream(x)))
    return dx, d_ln_w, d_ln_b, d_conv_w, d_conv_b


_ssm_ws = {}       # (device index, stream) -> the scan's persistent workspace
_ssm_ws_kept = []  # replaced workspaces stay allocated: a recorded graph may still use them


def _ssm_workspace(device, nbytes):
    """The scan's workspace for the current stream of `device`: zero-filled once, then reused
    by every call on that stream (the kernel keeps it consistent; calls on one stream are
    ordered, calls on different streams get different workspaces)."""
    stream = torch.cuda.current_stream(device)
    key = (stream.device.index, stream.cuda_stream)
    ws = _ssm_ws.get(key)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("ssm: the scan's workspace must exist before graph capture; run the "
                               "forward once outside capture first")
        if ws is not None:
            _ssm_ws_kept.append(ws)
        ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
        _ssm_ws[key] = ws
    return ws


def _stats_arg(row_stats, part, rows, nparts):
    """Pointer to part ``part`` and part stride (in pairs) of the partial row statistics
    ``row_stats`` ([P, rows, 2] fp32, contiguous: the rows of one part adjacent), or (None, 0)."""
    if row_stats is None:
        return None, 0
    if (row_stats.dtype != torch.float32 or not row_stats.is_contiguous() or row_stats.dim() != 3
            or row_stats.shape[1] != rows or row_stats.shape[2] != 2 or part + nparts > row_stats.shape[0]):
        raise ValueError(f"row_stats must be a contiguous fp32 [>= {part + nparts}, {rows}, 2] tensor")
    return row_stats.data_ptr() + 8 * part * rows, rows


def ssm_stats_parts(d_state):
    """Pairs per row the scan writes into row_stats (one per 32-channel block)."""
    return -(-d_state // 32)


def ssm(projs, A_log, d_state, y, h0=None, h_final=None, row_stats=None, stats_part=0):
    """Selective scan; writes y [B,L,ds] (may be a column slice of a wider buffer).  With
    ``row_stats`` ([P, B*L, 2] fp32), the sum and sum of squares of each row's stored values
    per 32-channel block go to parts stats_part, stats_part + 1, ..."""
    _on_gpu(projs, y)
    B, L, _ = projs.shape
    A_log = _same(A_log, projs, "A_log")
    prs = _rows2d(projs, "projs")
    yrs = _rows2d(y, "y")
    nbytes = lib().hdcm_ssm_workspace_bytes(B, L, d_state)
    ws = _ssm_workspace(projs.device, nbytes)
    if h0 is not None:
        h0 = h0.float().contiguous()
    sp, srs = _stats_arg(row_stats, stats_part, B * L, ssm_stats_parts(d_state))
    ev = timer.begin("ssm")
    _check("hdcm_ssm_fwd", lib().hdcm_ssm_fwd(
        projs.data_ptr(), prs, A_log.data_ptr(), h0.data_ptr() if h0 is not None else None,
        y.data_ptr(), yrs, h_final.data_ptr() if h_final is not None else None, sp, srs, ws.data_ptr(), nbytes,
        B, L, d_state, _dtype(projs), _stream(projs)))
    timer.end("ssm", ev)
    return y


def ssm_noalloc(projs, A_log, d_state, y, h0=None, h_final=None):
    """ssm() on the library's fixed per-GPU scratch instead of an allocated workspace
    (hdcm_ssm_fwd_noalloc): this wrapper and the call allocate nothing on the device.
    Calls that overlap on one GPU share the scratch and race."""
    _on_gpu(projs, y)
    B, L, _ = projs.shape
    if A_log.dtype != projs.dtype or A_log.device != projs.device or not A_log.is_contiguous():
        raise RuntimeError("ssm_noalloc: A_log must be a contiguous tensor of projs' dtype and device")
    for name, t in (("h0", h0), ("h_final", h_final)):
        if t is not None and (t.dtype != torch.float32 or not t.is_contiguous()):
            raise RuntimeError(f"ssm_noalloc: {name} must be a contiguous fp32 tensor")
    _check("hdcm_ssm_fwd_noalloc", lib().hdcm_ssm_fwd_noalloc(
        projs.data_ptr(), _rows2d(projs, "projs"), A_log.data_ptr(), h0.data_ptr() if h0 is not None else None,
        y.data_ptr(), _rows2d(y, "y"), h_final.data_ptr() if h_final is not None else None, None, 0, B, L, d_state,
        _dtype(projs), _stream(projs)))
    return y


def ssm_bwd(projs, A_log, d_state, h, gy, dprojs):
    """Gradient of ssm (zero start state): d dt_raw, d x, d b into dprojs[..., :3*ds] (in
    place) and returns d A_log (fp32 [ds]).  h is the forward's y, gy its gradient."""
    _on_gpu(projs, h, gy, dprojs)
    B, L, _ = projs.shape
    A_log = _same(A_log, projs, "A_log")
    for name, t in (("h", h), ("gy", gy), ("dprojs", dprojs)):
        if t.dtype != projs.dtype:
            raise RuntimeError(f"ssm_bwd: {name} must have projs' dtype")
    dA = torch.empty(d_state, device=projs.device, dtype=torch.float32)
    nbytes = lib().hdcm_ssm_bwd_workspace_bytes(B, L, d_state, _dtype(projs))
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=projs.device)
    _check("hdcm_ssm_bwd", lib().hdcm_ssm_bwd(
        projs.data_ptr(), _rows2d(projs, "projs"), A_log.data_ptr(), h.data_ptr(), _rows2d(h, "h"), gy.data_ptr(),
        _rows2d(gy, "gy"), dprojs.data_ptr(), _rows2d(dprojs, "dprojs"), dA.data_ptr(), ws.data_ptr(), ws.numel(),
        B, L, d_state, _dtype(projs), _stream(projs)))
    return dA


def gnorm_gate_bwd(y, gate, gn_w, gn_b, eps, dout, num_heads, dy, dgate):
    """Gradient of the slot GroupNorm + gate on [B,L,dm] views: writes dy and dgate (in
    place; column slices allowed) and returns (d gn_w, d gn_b) fp32."""
    _on_gpu(y, gate, dout, dy, dgate)
    B, L, dm = y.shape
    gn_w, gn_b = _same(gn_w, y, "gn_w"), _same(gn_b, y, "gn_b")
    f32 = dict(device=y.device, dtype=torch.float32)
    dgw, dgb = torch.empty(dm, **f32), torch.empty(dm, **f32)
    nbytes = lib().hdcm_gnorm_gate_bwd_workspace_bytes(dm, num_heads)
    ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=y.device)
    _check("hdcm_gnorm_gate_bwd", lib().hdcm_gnorm_gate_bwd(
        y.data_ptr(), _rows2d(y, "y"), gate.data_ptr(), _rows2d(gate, "gate"), gn_w.data_ptr(), gn_b.data_ptr(),
        float(eps), dout.data_ptr(), _rows2d(dout, "dout"), dy.data_ptr(), _rows2d(dy, "dy"), dgate.data_ptr(),
        _rows2d(dgate, "dgate"), dgw.data_ptr(), dgb.data_ptr(), ws.data_ptr(), ws.numel(), B * L, dm, num_heads,
        _dtype(y), _stream(y)))
    return dgw, dgb


def slot_phi_prep(projs, q_col, d_model, z):
    """z[..., dm:4dm] = [v | phi(k) | phi(q)] from the q, k, v blocks of projs."""
    _on_gpu(projs, z)
    B, L, _ = projs.shape
    _check("hdcm_slot_phi_prep", lib().hdcm_slot_phi_prep(
        projs.data_ptr(), _rows2d(projs, "projs"), q_col, z.data_ptr(), _rows2d(z, "z"), B * L, d_model,
        _dtype(projs), _stream(projs)))
    return z


def slot_phi_chain(projs, q_col, d_model, dprojs):
    """In place: the q, k blocks of dprojs (gradients of phi(q), phi(k)) times phi'(q), phi'(k)."""
    _on_gpu(projs, dprojs)
    B, L, _ = projs.shape
    _check("hdcm_slot_phi_chain", lib().hdcm_slot_phi_chain(
        projs.data_ptr(), _rows2d(projs, "projs"), q_col, dprojs.data_ptr(), _rows2d(dprojs, "dprojs"), B * L,
        d_model, _dtype(projs), _stream(projs)))
    return dprojs


SLOT_MAX_HEAD_DIM = 128  # widest head of the fused slot + gate kernels


def slot_workspace(projs, d_model, num_heads, chunk):
    B, L, _ = projs.shape
    nbytes = lib().hdcm_slot_workspace_bytes(B, L, d_model, num_heads, chunk, _dtype(projs))
    if nbytes == 0 and B * L > 0:
        raise HdcmError("hdcm_slot_workspace_bytes", -3)
    return torch.empty(max(nbytes, 16), dtype=torch.uint8, device=projs.device)


def slot_state(projs, q_col, gamma, d_model, num_heads, chunk, ws, S0=None):
    """Segment-start states of the slot recurrence into ws."""
    _on_gpu(projs)
    B, L, _ = projs.shape
    gamma = _same(gamma, projs, "gamma")
    if S0 is not None:
        S0 = S0.float().contiguous()
    ev = timer.begin("slot_state")
    _check("hdcm_slot_state_fwd", lib().hdcm_slot_state_fwd(
        projs.data_ptr(), _rows2d(projs, "projs"), q_col, gamma.data_ptr(),
        S0.data_ptr() if S0 is not None else None, ws.data_ptr(), ws.numel(), B, L, d_model,
        num_heads, chunk, _dtype(projs), _stream(projs)))
    timer.end("slot_state", ev)
    return ws


def slot_attend(base, q_col, k_col, v_col, gamma, d_model, num_heads, chunk, phi, out, out_col, reverse=False,
                ws=None, chain=None):
    """Slot recurrence without GroupNorm/gate on column blocks of base [B,L,W] into
    out[..., out_col:out_col+d_model]; ``reverse`` walks every sequence from its last token.
    With ``chain`` ([B,L,W'] in out's column layout) each output is multiplied by phi'(z), z
    the value of chain at the output's row and column."""
    _on_gpu(base, out)
    B, L, _ = base.shape
    if out.dtype != base.dtype or out.shape[:2] != base.shape[:2]:
        raise RuntimeError("slot_attend: out must match base in dtype and [B, L]")
    if chain is not None and (chain.dtype != out.dtype or chain.shape[:2] != out.shape[:2]):
        raise RuntimeError("slot_attend: chain must match out in dtype and [B, L]")
    gamma = _same(gamma, base, "gamma")
    if ws is None:
        ws = slot_workspace(base, d_model, num_heads, chunk)
    brs, ors = _rows2d(base, "base"), _rows2d(out, "out")
    bptr, optr = base.data_ptr(), out.data_ptr()
    zrs = _rows2d(chain, "chain") if chain is not None else 0
    zptr = chain.data_ptr() if chain is not None else None
    if reverse and B * L > 0:  # start at the last row; negative row strides
        bptr += (B * L - 1) * brs * base.element_size()
        optr += (B * L - 1) * ors * out.element_size()
        brs, ors = -brs, -ors
        if chain is not None:
            zptr += (B * L - 1) * zrs * chain.element_size()
            zrs = -zrs
    ev = timer.begin("slot_attend")
    _check("hdcm_slot_attend_fwd", lib().hdcm_slot_attend_fwd(
        bptr, brs, q_col, k_col, v_col, gamma.data_ptr(), 1 if phi else 0, ws.data_ptr(), ws.numel(), optr, ors,
        out_col, zptr, zrs, B, L, d_model, num_heads, chunk, _dtype(base), _stream(base)))
    timer.end("slot_attend", ev)
    return out


def slot_gate(projs, q_col, gamma, gn_w, gn_b, gn_eps, ws, out, out_col, d_model, num_heads, chunk,
              S_final=None, row_stats=None, stats_part=0):
    """Slot memory + GroupNorm + sigmoid gate into out[..., out_col:out_col+d_model].  With
    ``row_stats`` ([P, B*L, 2] fp32), the sum and sum of squares of each row's stored values
    per head go to parts stats_part .. stats_part + num_heads - 1."""
    _on_gpu(projs, out)
    B, L, _ = projs.shape
    gamma = _same(gamma, projs, "gamma")
    gn_w = _same(gn_w, projs, "gn_w")
    gn_b = _same(gn_b, projs, "gn_b")
    sp, srs = _stats_arg(row_stats, stats_part, B * L, num_heads)
    ev = timer.begin("slot_gate")
    _check("hdcm_slot_gate_fwd", lib().hdcm_slot_gate_fwd(
        projs.data_ptr(), _rows2d(projs, "projs"), q_col, gamma.data_ptr(), gn_w.data_ptr(),
        gn_b.data_ptr(), float(gn_eps), ws.data_ptr(), ws.numel(), out.data_ptr(), _rows2d(out, "out"),
        out_col, S_final.data_ptr() if S_final is not None else None, sp, srs, B, L, d_model, num_heads, chunk,
        _dtype(projs), _stream(projs)))
    timer.end("slot_gate", ev)
    return out


def gnorm_gate(y1, y2, gate, gn_w, gn_b, gn_eps, num_heads, out, row_stats=None, stats_part=0):
    """GroupNorm per (token, head) of y1 + y2' (y2' = y2 with each head's halves exchanged; y2
    may be None) times sigmoid(gate), into ``out``; all [..., d_model] row views of one dtype.
    ``row_stats`` as in slot_gate."""
    _on_gpu(y1, gate, out)
    dm = y1.shape[-1]
    rows = y1.numel() // dm if dm else 0
    gn_w = _same(gn_w, y1, "gn_w")
    gn_b = _same(gn_b, y1, "gn_b")
    sp, srs = _stats_arg(row_stats, stats_part, rows, num_heads)
    ev = timer.begin("gnorm_gate")
    _check("hdcm_gnorm_gate_fwd", lib().hdcm_gnorm_gate_fwd(
        y1.data_ptr(), _rows2d(y1, "y1"), y2.data_ptr() if y2 is not None else None,
        _rows2d(y2, "y2") if y2 is not None else 0, gate.data_ptr(), _rows2d(gate, "gate"), gn_w.data_ptr(),
        gn_b.data_ptr(), float(gn_eps), out.data_ptr(), _rows2d(out, "out"), sp, srs, rows, dm, num_heads,
        _dtype(y1), _stream(y1)))
    timer.end("gnorm_gate", ev)
    return out


def layer_norm(x, w=None, b=None, eps=1e-5, out=None):
    """Row LayerNorm over the last dim (fp32 statistics); in-place when out is x."""
    _on_gpu(x)
    W = x.shape[-1]
    if w is not None:
        w = _same(w, x, "w")
        b = _same(b, x, "b")
    if out is None:
        out = torch.empty_like(x, memory_format=torch.contiguous_format)
    rows = x.numel() // W if W else 0
    ev = timer.begin("rowln")
    _check("hdcm_rowln_fwd", lib().hdcm_rowln_fwd(
        x.data_ptr(), _rows2d(x, "x"), out.data_ptr(), _rows2d(out, "out"),
        w.data_ptr() if w is not None else None, b.data_ptr() if b is not None else None,
        rows, W, float(eps), _dtype(x), _stream(x)))
    timer.end("rowln", ev)
    return out


def layer_norm2_ok(x) -> bool:
    """Whether layer_norm2 takes rows of x's width (up to 512 16-byte groups)."""
    return x.shape[-1] * x.element_size() <= 512 * 16


def layer_norm2(x, w1, b1, eps1, w2, b2, eps2, out=None):
    """layer_norm(layer_norm(x, w1, b1, eps1), w2, b2, eps2) in one pass, bit-identical to the
    two calls (the intermediate rounded to x's dtype as stored); in-place when out is x."""
    _on_gpu(x)
    W = x.shape[-1]
    w1, b1 = _same(w1, x, "w1"), _same(b1, x, "b1")
    w2, b2 = _same(w2, x, "w2"), _same(b2, x, "b2")
    if out is None:
        out = torch.empty_like(x, memory_format=torch.contiguous_format)
    rows = x.numel() // W if W else 0
    ev = timer.begin("rowln2")
    _check("hdcm_rowln2_fwd", lib().hdcm_rowln2_fwd(
        x.data_ptr(), _rows2d(x, "x"), out.data_ptr(), _rows2d(out, "out"), w1.data_ptr(), b1.data_ptr(),
        float(eps1), w2.data_ptr(), b2.data_ptr(), float(eps2), rows, W, _dtype(x), _stream(x)))
    timer.end("rowln2", ev)
    return out


def layer_norm_bwd(grad_out, x, w=None, eps=1e-5):
    """Gradient of layer_norm: (dx in x.dtype, dw fp32 or None, db fp32 or None)."""
    _on_gpu(grad_out, x)
    W = x.shape[-1]
    if grad_out.shape != x.shape or grad_out.dtype != x.dtype:
        raise RuntimeError("layer_norm_bwd: grad_out must match x in shape and dtype")
    grad_out, x = grad_out.contiguous(), x.contiguous()
    rows = x.numel() // W if W else 0
    dx = torch.empty_like(x, memory_format=torch.contiguous_format)
    dw = db = ws = None
    if w is not None:
        w = _same(w, x, "w")
        dw = torch.empty(W, device=x.device, dtype=torch.float32)
        db = torch.empty(W, device=x.device, dtype=torch.float32)
        ws = torch.empty(max(lib().hdcm_rowln_bwd_workspace_bytes(rows, W), 16), dtype=torch.uint8,
                         device=x.device)
    _check("hdcm_rowln_bwd", lib().hdcm_rowln_bwd(
        grad_out.data_ptr(), _rows2d(grad_out, "grad_out"), x.data_ptr(), _rows2d(x, "x"),
        w.data_ptr() if w is not None else None, dx.data_ptr(), _rows2d(dx, "dx"),
        dw.data_ptr() if dw is not None else None, db.data_ptr() if db is not None else None,
        ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0, rows, W, float(eps),
        _dtype(x), _stream(x)))
    return dx, dw, db


# ----------------------------------------------------------------------------- decode step
def norm_conv_step(x, ln_w, ln_b, conv_w, conv_b, eps, hist, out=None):
    """One token per batch row: x [B,D] -> out [B,D]; hist [B,3,D] (raw previous rows,
    x.dtype) is shifted in place."""
    _on_gpu(x, hist)
    B, D = x.shape
    ln_w = _same(ln_w, x, "ln_w")
    ln_b = _same(ln_b, x, "ln_b")
    conv_b = _same(conv_b, x, "conv_b")
    conv_w = _same(conv_w.reshape(D, 4), x, "conv_w")
    if hist.dtype != x.dtype or not hist.is_contiguous() or tuple(hist.shape) != (B, 3, D):
        raise RuntimeError("norm_conv_step: hist must be a contiguous [B,3,D] tensor of x's dtype")
    if x.stride(1) != 1:
        x = x.contiguous()
    if out is None:
        out = torch.empty(B, D, device=x.device, dtype=x.dtype)
    ev = timer.begin("norm_conv_step")
    _check("hdcm_norm_conv_step_fwd", lib().hdcm_norm_conv_step_fwd(
        x.data_ptr(), x.stride(0), ln_w.data_ptr(), ln_b.data_ptr(), conv_w.data_ptr(), conv_b.data_ptr(),
        hist.data_ptr(), out.data_ptr(), out.stride(0), B, D, float(eps), _dtype(x), _stream(x)))
    timer.end("norm_conv_step", ev)
    return out


_step_ws = {}  # device index -> the fused decode front's flag workspace


def step_workspace(device):
    """The fused decode front's workspace (call tag, arrivals, timeouts, row flags) of
    `device`: zero-filled once, then kept (the kernel keeps it consistent from call to call).
    One per device, shared by every stream: calls that overlap in time on one device race
    (a decode step, eager or replayed, runs on one stream at a time)."""
    dev = torch.device(device)
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    ws = _step_ws.get(key)
    if ws is None:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("decode step: the fused front's workspace must exist before graph capture; run "
                               "one step outside capture first")
        nbytes = int(lib().hdcm_step_workspace_bytes())
        ws = torch.zeros((nbytes + 255) // 256 * 256, dtype=torch.uint8, device=device)
        _step_ws[key] = ws
    return ws


def step_timeouts(device) -> int:
    """Waits of the fused decode front that gave up (the word at byte 128 of the workspace) on `device`;
    0 unless the GPU was shared with work that held back the conv rows."""
    ws = step_workspace(device)
    return int(ws[128:132].view(torch.int32).item())


def norm_conv_in_proj_step_ok(x, weight) -> bool:
    """Whether the fused decode front (hdcm_norm_conv_in_proj_step_fwd) takes x [B,D] and
    in_proj's weight [N,D]: bf16, 1 <= B <= 16, D % 32 == 0, D <= 2048."""
    B, D = x.shape
    return (x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16 and 1 <= B <= SKINNY_MAX_ROWS
            and D % 32 == 0 and D <= 2048 and weight.shape[-1] == D)


def norm_conv_in_proj_step(x, ln_w, ln_b, conv_w, conv_b, eps, hist, weight, bias, u=None, out=None):
    """norm_conv_step followed by skinny_linear(u, weight, bias) in one launch (the same values
    bit for bit): x [B,D] -> (u [B,D], out [B,N]); hist [B,3,D] is shifted in place."""
    _on_gpu(x, hist, weight)
    B, D = x.shape
    N = weight.shape[0]
    ln_w = _same(ln_w, x, "ln_w")
    ln_b = _same(ln_b, x, "ln_b")
    conv_b = _same(conv_b, x, "conv_b")
    conv_w = _same(conv_w.reshape(D, 4), x, "conv_w")
    if hist.dtype != x.dtype or not hist.is_contiguous() or tuple(hist.shape) != (B, 3, D):
        raise RuntimeError("norm_conv_in_proj_step: hist must be a contiguous [B,3,D] tensor of x's dtype")
    if x.stride(1) != 1 or x.stride(0) % 8:
        x = x.contiguous()
    w = weight if weight.is_contiguous() else weight.contiguous()
    if bias is not None:
        bias = _same(bias, x, "bias")
    if u is None:
        u = torch.empty(B, D, device=x.device, dtype=x.dtype)
    if out is None:
        out = torch.empty(B, N, device=x.device, dtype=x.dtype)
    ws = step_workspace(x.device)
    ev = timer.begin("norm_conv_in_proj_step")
    _check("hdcm_norm_conv_in_proj_step_fwd", lib().hdcm_norm_conv_in_proj_step_fwd(
        x.data_ptr(), x.stride(0), ln_w.data_ptr(), ln_b.data_ptr(), conv_w.data_ptr(), conv_b.data_ptr(),
        hist.data_ptr(), float(eps), u.data_ptr(), u.stride(0), w.data_ptr(), w.stride(0),
        bias.data_ptr() if bias is not None else None, out.data_ptr(), out.stride(0), B, D, N, ws.data_ptr(),
        ws.numel(), _dtype(x), _stream(x)))
    timer.end("norm_conv_in_proj_step", ev)
    return u, out


def mixer_step(projs, A_log, d_state, q_col, gamma, gn_w, gn_b, gn_eps, h, S_prev, S_intra, pos, chunk,
               out, d_model, num_heads, y_col=0, g_col=None, pos_dev=None):
    """One token per batch row of the SSM and the slot memory + GroupNorm gate.
    projs [B,P]; h [B,ds], S_prev / S_intra [B,H,hd,hd] fp32 contiguous, updated in place;
    pos = token offset in its chunk (or, with pos_dev, an int32 device scalar holding it).
    Writes out[:, y_col:y_col+ds] and out[:, g_col:g_col+dm]."""
    _on_gpu(projs, out, h, S_prev, S_intra)
    B = projs.shape[0]
    if g_col is None:
        g_col = y_col + d_state
    hd = d_model // num_heads
    for t, shape, name in ((h, (B, d_state), "h"), (S_prev, (B, num_heads, hd, hd), "S_prev"),
                           (S_intra, (B, num_heads, hd, hd), "S_intra")):
        if t.dtype != torch.float32 or not t.is_contiguous() or tuple(t.shape) != shape:
            raise RuntimeError(f"mixer_step: {name} must be a contiguous fp32 tensor of shape {shape}")
    A_log = _same(A_log, projs, "A_log")
    gamma = _same(gamma, projs, "gamma")
    gn_w = _same(gn_w, projs, "gn_w")
    gn_b = _same(gn_b, projs, "gn_b")
    ev = timer.begin("mixer_step")
    _check("hdcm_mixer_step_fwd", lib().hdcm_mixer_step_fwd(
        projs.data_ptr(), _rows2d(projs, "projs"), q_col, A_log.data_ptr(), h.data_ptr(), gamma.data_ptr(),
        S_prev.data_ptr(), S_intra.data_ptr(), int(pos), None if pos_dev is None else pos_dev.data_ptr(),
        int(chunk), gn_w.data_ptr(), gn_b.data_ptr(),
        float(gn_eps), out.data_ptr(), _rows2d(out, "out"), y_col, g_col, B, d_model, d_state, num_heads,
        _dtype(projs), _stream(projs)))
    timer.end("mixer_step", ev)
    return out


def chunk_pos_advance(pos_dev, chunk):
    """pos_dev (int32 device scalar) <- (pos_dev + 1) mod chunk, on the current stream."""
    _on_gpu(pos_dev)
    if pos_dev.dtype != torch.int32 or pos_dev.numel() != 1:
        raise RuntimeError("chunk_pos_advance: pos_dev must be a one-element int32 tensor")
    _check("hdcm_chunk_pos_advance", lib().hdcm_chunk_pos_advance(pos_dev.data_ptr(), int(chunk), _stream(pos_dev)))


# ----------------------------------------------------------------------------- decode projections
SKINNY_MAX_ROWS = 16
SKINNY_MAX_K = 3072


def _rows_view(t: torch.Tensor, K: int) -> torch.Tensor:
    """t [..., K] as a 2-D view with unit inner stride and 16-byte aligned rows (a copy if
    the layout does not allow one)."""
    t2 = t.reshape(-1, K)
    if t2.stride(-1) != 1 or (t2.shape[0] > 1 and t2.stride(0) % 8) or t2.data_ptr() % 16:
        t2 = t2.contiguous()
    return t2


def gemm(x, weight, bias=None, out=None):
    """x [..., K] @ weight[N, K]^T (+ bias[N]) -> [..., N] on the tiled bf16 MFMA GEMM (fp32
    accumulation, one rounding).  ``out`` may be a strided [..., N] view (unit inner stride)."""
    _on_gpu(x, weight)
    K = x.shape[-1]
    N = weight.shape[0]
    lead = x.shape[:-1]
    x2 = _rows_view(x, K)
    M = x2.shape[0]
    w = weight if weight.is_contiguous() else weight.contiguous()
    if out is None:
        out = torch.empty(*lead, N, device=x.device, dtype=x.dtype)
    o2 = out.view(-1, N)  # a view (never a copy): the kernel writes through it
    if bias is not None:
        bias = _same(bias, x, "bias")
    ev = timer.begin("gemm")
    _check("hdcm_gemm_fwd", lib().hdcm_gemm_fwd(
        x2.data_ptr(), x2.stride(0), w.data_ptr(), w.stride(0), bias.data_ptr() if bias is not None else None,
        o2.data_ptr(), o2.stride(0), M, N, K, _dtype(x), _stream(x)))
    timer.end("gemm", ev)
    return out


def rowln_gemm(c, weight, residual, eps=1e-5, out=None):
    """residual + LN(c) @ weight^T, LN the row LayerNorm without affine over c's last dim;
    the row statistics and the weight's row sums are computed inside the GEMM.  ``out`` may
    be ``residual``."""
    _on_gpu(c, weight, residual)
    K = c.shape[-1]
    N = weight.shape[0]
    c2 = _rows_view(c, K)
    M = c2.shape[0]
    w = weight if weight.is_contiguous() else weight.contiguous()
    r2 = residual.reshape(-1, N)
    if r2.stride(-1) != 1:
        raise ValueError("residual must have a unit inner stride")
    if out is None:
        out = torch.empty(*c.shape[:-1], N, device=c.device, dtype=c.dtype)
    o2 = out.view(-1, N)  # a view (never a copy): the kernel writes through it
    ev = timer.begin("rowln_gemm")
    _check("hdcm_rowln_gemm_fwd", lib().hdcm_rowln_gemm_fwd(
        c2.data_ptr(), c2.stride(0), w.data_ptr(), w.stride(0), r2.data_ptr(), r2.stride(0), o2.data_ptr(),
        o2.stride(0), M, N, K, float(eps), _dtype(c), _stream(c)))
    timer.end("rowln_gemm", ev)
    return out


def row_sums(weight, out=None):
    """fp32 [N] sums of the rows of a bf16 [N, K] weight (hdcm_row_sums_fwd), into ``out``
    when given."""
    _on_gpu(weight)
    w = weight if weight.is_contiguous() else weight.contiguous()
    N, K = w.shape
    sums = torch.empty(N, device=w.device, dtype=torch.float32) if out is None else out
    if sums.dtype != torch.float32 or not sums.is_contiguous() or sums.numel() != N:
        raise ValueError(f"row_sums: out must be a contiguous fp32 tensor of {N} values")
    _check("hdcm_row_sums_fwd", lib().hdcm_row_sums_fwd(w.data_ptr(), w.stride(0), N, K, sums.data_ptr(),
                                                        _dtype(w), _stream(w)))
    return sums


def rowln_gemm_stats(c, weight, w_sums, row_stats, residual, eps=1e-5, out=None):
    """rowln_gemm with the row statistics and the weight row sums supplied: ``row_stats``
    [P, rows, 2] fp32 holds per row P (sum, sum of squares) pairs of disjoint column blocks
    covering c's last dim (as ssm and slot_gate write them), ``w_sums`` = row_sums(weight).
    ``out`` may be ``residual``."""
    _on_gpu(c, weight, residual)
    K = c.shape[-1]
    N = weight.shape[0]
    c2 = _rows_view(c, K)
    M = c2.shape[0]
    w = weight if weight.is_contiguous() else weight.contiguous()
    r2 = residual.reshape(-1, N)
    if r2.stride(-1) != 1:
        raise ValueError("residual must have a unit inner stride")
    sp, stride = _stats_arg(row_stats, 0, M, 1)
    parts = row_stats.shape[0]
    if w_sums.dtype != torch.float32 or not w_sums.is_contiguous() or w_sums.numel() != N:
        raise ValueError(f"w_sums must be a contiguous fp32 tensor of {N} values")
    if out is None:
        out = torch.empty(*c.shape[:-1], N, device=c.device, dtype=c.dtype)
    o2 = out.view(-1, N)
    ev = timer.begin("rowln_gemm")
    _check("hdcm_rowln_gemm_stats_fwd", lib().hdcm_rowln_gemm_stats_fwd(
        c2.data_ptr(), c2.stride(0), w.data_ptr(), w.stride(0), w_sums.data_ptr(), sp, parts, stride, r2.data_ptr(),
        r2.stride(0), o2.data_ptr(), o2.stride(0), M, N, K, float(eps), _dtype(c), _stream(c)))
    timer.end("rowln_gemm", ev)
    return out


def rowln_stats_ok(c, N):
    """Whether rowln_gemm_stats takes c [.., K] with N outputs: bf16, more rows than the decode
    step kernels handle, and the 16-byte runs it needs (N a multiple of 8)."""
    K = c.shape[-1]
    rows = c.numel() // K if K else 0
    return c.dtype == torch.bfloat16 and rows > SKINNY_MAX_ROWS and N % 8 == 0 and K % 8 == 0


def skinny_ok(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """Whether linear(x, weight) at x's shape runs on the skinny decode GEMM: bf16, at most
    16 rows, K a multiple of 32 up to 3072."""
    K = x.shape[-1]
    rows = x.numel() // K if K else 0
    return (x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16 and rows <= SKINNY_MAX_ROWS
            and K % 32 == 0 and K <= SKINNY_MAX_K and weight.shape[-1] == K)


def skinny_linear(x, weight, bias=None, residual=None, out=None):
    """x [..., K] (at most 16 rows) @ weight[N, K]^T (+ bias[N]) (+ residual [..., N]) -> [..., N]
    on the skinny decode GEMM (bf16, fp32 accumulation).  ``out`` may be ``residual``."""
    _on_gpu(x, weight)
    K = x.shape[-1]
    N = weight.shape[0]
    lead = x.shape[:-1]
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    M = x2.shape[0]
    w = weight if weight.is_contiguous() else weight.contiguous()
    if out is None:
        out = torch.empty(*lead, N, device=x.device, dtype=x.dtype)
    o2 = out.view(-1, N)
    r2 = residual.reshape(-1, N) if residual is not None else None
    if bias is not None:
        bias = _same(bias, x, "bias")
    ev = timer.begin("skinny_gemm")
    _check("hdcm_skinny_gemm_fwd", lib().hdcm_skinny_gemm_fwd(
        x2.data_ptr(), x2.stride(0), w.data_ptr(), w.stride(0), bias.data_ptr() if bias is not None else None,
        r2.data_ptr() if r2 is not None else None, r2.stride(0) if r2 is not None else 0, o2.data_ptr(),
        o2.stride(0), M, N, K, _dtype(x), _stream(x)))
    timer.end("skinny_gemm", ev)
    return out
