"""ctypes binding of libffmoe.so (the C ABI declared in include/ffmoe.h).

The library is built in-tree by ``flashfusedmoe_amd.build``.  There is no
fallback: if it is missing or fails to load, every entry point raises.
"""

import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libffmoe.so")

# constants mirrored from include/ffmoe.h
ROW_DROPPED = -1
ROW_ALIAS0 = -2
GATING = {"softmax": 0, "sigmoid": 1}
ACTIVATION = {"swiglu": 0, "geglu": 1, "relu_squared": 2}
MAX_EXPERTS = 256
MAX_TOPK = 16
MAX_FUSED_GATE_E = 32
STAT_AUX, STAT_Z, STAT_IMBALANCE, STAT_DROP_FRAC, NUM_STATS = 0, 1, 2, 3, 4
ISTAT_MAX, ISTAT_MIN, ISTAT_DROPPED, NUM_ISTATS = 0, 1, 2, 4

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_F = ctypes.c_float

# name -> (restype, argtypes)
SIGNATURES = {
    "ffmoe_last_error": (ctypes.c_char_p, []),
    "ffmoe_version": (_I, []),
    "ffmoe_route_workspace_bytes": (ctypes.c_size_t, [_L, _I, _I]),
    "ffmoe_route_fwd": (_I, [_P, _P, _P, _P, _L, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P]),
    "ffmoe_route_fwd_ex": (_I, [_P, _P, _P, _P, _I, _I, _F, _I, _I, _P, _L, _I, _I, _I, _I, _I, _P, _P,
                                _P, _P, _P, _P]),
    "ffmoe_route_scan": (_I, [_L, _I, _I, _I, _I, _F, _F, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "ffmoe_permute": (_I, [_P, _P, _P, _P, _P, _L, _I, _I, _I, _I, _I, _P, _P, _P, _P]),
    "ffmoe_gemm_tile_rows": (_I, [_L, _I]),
    "ffmoe_set_lds_transpose": (_I, [_I]),
    "ffmoe_gemm_workspace_bytes": (_L, []),
    "ffmoe_gemm_check": (_I, [_P, _P]),
    "ffmoe_gemm_up_glu": (_I, [_P, _P, _P, _P, _I, _I, _L, _I, _I, _I, _P, _P, _P, _P]),
    "ffmoe_gemm_down": (_I, [_P, _P, _P, _P, _I, _I, _L, _I, _I, _P, _P, _P]),
    "ffmoe_gemm_up_down_shared": (_I, [_P, _P, _P, _P, _P, _I, _I, _L, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P]),
    "ffmoe_gemm_dgrad_wgrad_shared": (_I, [_P, _P, _P, _P, _P, _I, _I, _L, _I, _I, _P, _P, _P, _P, _P, _P]),
    "ffmoe_gemm_dgrad_glu": (_I, [_P, _P, _P, _P, _P, _I, _I, _L, _I, _I, _I, _P, _P, _P]),
    "ffmoe_gemm_dgrad": (_I, [_P, _P, _P, _P, _I, _I, _L, _I, _I, _P, _P, _P]),
    "ffmoe_gemm_wgrad": (_I, [_P, _P, _P, _I, _I, _I, _P, _P]),
    "ffmoe_gemm_up_glu_shared": (_I, [_P, _P, _P, _P, _I, _I, _L, _I, _I, _I, _P, _P, _P, _P, _P]),
    "ffmoe_gemm_down_shared": (_I, [_P, _P, _P, _P, _I, _I, _L, _I, _I, _P, _P, _P, _P]),
    "ffmoe_gemm_dgrad_glu_shared": (_I, [_P, _P, _P, _P, _P, _I, _I, _L, _I, _I, _I, _P, _P, _P, _P]),
    "ffmoe_gemm_dgrad_shared": (_I, [_P, _P, _P, _P, _I, _I, _L, _I, _I, _P, _P, _P, _P]),
    "ffmoe_gemm_wgrad_shared": (_I, [_P, _P, _P, _I, _I, _I, _P, _P, _P, _P]),
    "ffmoe_combine": (_I, [_P, _P, _P, _P, _L, _I, _I, _P, _P]),
    "ffmoe_dx_reduce": (_I, [_P, _P, _P, _P, _L, _I, _I, _I, _P, _P]),
    "ffmoe_gate_grad_workspace_bytes": (_L, [_L, _I, _I]),
    "ffmoe_gate_grad": (_I, [_P, _P, _L, _I, _I, _P, _P, _P]),
    "ffmoe_gate_logits_workspace_bytes": (_L, [_L, _I, _I]),
    "ffmoe_gate_logits": (_I, [_P, _P, _L, _I, _I, _P, _P, _P]),
    "ffmoe_gate_dx": (_I, [_P, _P, _L, _I, _I, _P, _P]),
    "ffmoe_gate_grad_noalloc_max_bytes": (_L, []),
    "ffmoe_gate_grad_noalloc": (_I, [_P, _P, _L, _I, _I, _P, _P]),
    "ffmoe_route_bwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _F, _L, _I, _I, _I,
                             _I, _I, _P, _P, _P, _P]),
    "ffmoe_route_bwd_ex": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _F, _L, _I, _I, _I, _I, _I,
                                _I, _P, _P, _I, _F, _P, _P, _P, _P]),
    "ffmoe_glu_fwd": (_I, [_P, _L, _I, _I, _P, _P]),
    "ffmoe_t_gemm_dense": (_I, [_I, _I, _I, _P, _P, _P, _I, _I, _I, _L, _L, _L, _I, _P]),
    "ffmoe_t_gemm_rows": (_I, [_I, _P, _P, _P, _P, _I, _L, _I, _I, _I, _P, _P]),
    "ffmoe_t_gemm_wgrad": (_I, [_I, _P, _P, _P, _I, _I, _I, _P, _P]),
    "ffmoe_t_glu_fwd": (_I, [_I, _P, _L, _I, _I, _I, _P, _P]),
    "ffmoe_t_glu_bwd": (_I, [_I, _P, _P, _L, _I, _I, _I, _P, _P]),
    "ffmoe_t_permute": (_I, [_I, _P, _P, _P, _P, _P, _L, _I, _I, _I, _I, _I, _P, _P, _P, _P]),
    "ffmoe_t_combine": (_I, [_I, _P, _P, _P, _P, _L, _I, _I, _P, _P]),
    "ffmoe_t_route_bwd": (_I, [_I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _F, _F, _L, _I, _I, _I, _I,
                               _I, _I, _P, _P, _I, _F, _P, _P, _P, _P]),
    "ffmoe_t_routing_scatter_padded": (_I, [_I, _P, _P, _P, _P, _L, _I, _I, _L, _I, _L, _P, _P, _P]),
    "ffmoe_t_scatter_rows": (_I, [_I, _P, _P, _P, _L, _I, _I, _L, _P, _P]),
    "ffmoe_route_logits_f32": (_I, [_P, _P, _I, _F, _I, _I, _L, _I, _I, _I, _I, _P, _P, _P, _P, _P]),
    "ffmoe_glu_bwd": (_I, [_P, _P, _L, _I, _I, _P, _P]),
    "ffmoe_scatter_rows": (_I, [_P, _P, _P, _L, _I, _I, _L, _P, _P]),
    "ffmoe_routing_scatter_padded": (_I, [_P, _P, _P, _P, _L, _I, _I, _L, _I, _L, _P, _P, _P]),
}

class DenseGroup(ctypes.Structure):
    """ffmoe_dense_group (include/ffmoe.h): a dense row group computed in
    the same launch as the routed experts (MoELayer's shared expert)."""
    _fields_ = [("a", _P), ("b", _P), ("up", _P), ("c", _P), ("c2", _P), ("rows", _L),
                ("activation", _I)]


def dense_group(a, b, c, rows, activation, up=None, c2=None):
    """A DenseGroup over tensors (None -> NULL); pass it with ctypes.byref."""
    return DenseGroup(ptr(a), ptr(b), ptr(up), ptr(c), ptr(c2), int(rows), int(activation))


_lib = None
_lock = threading.Lock()


class FFMoEError(RuntimeError):
    """A libffmoe entry point rejected its arguments or failed to launch."""


def load():
    """Loads libffmoe.so once and binds every entry point of include/ffmoe.h."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m flashfusedmoe_amd.build` "
                "(the fused MoE path has no non-HIP fallback)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    if t is None:
        return None
    return t.data_ptr()


def stream_ptr(device=None):
    return torch.cuda.current_stream(device).cuda_stream


# Optional observer of every entry-point call: hook(name, phase) with phase 0
# right before and 1 right after the call (a profiler records HIP events on
# the launch stream there).  None in normal use.
call_hook = None


def call(name, *args):
    """Calls an entry point and raises FFMoEError with the library's message
    when it returns nonzero."""
    lib = load()
    hook = call_hook
    if hook is not None:
        hook(name, 0)
    rc = getattr(lib, name)(*args)
    if hook is not None:
        hook(name, 1)
    if rc != 0:
        msg = lib.ffmoe_last_error().decode(errors="replace")
        raise FFMoEError(f"{name} failed: {msg}")
    return rc


def gemm_tile_rows(max_rows, E):
    """Row-tile height the grouped GEMMs use for max_rows rows over E experts."""
    return load().ffmoe_gemm_tile_rows(max_rows, E)


_GEMM_WS = {}


def gemm_workspace(device, stream):
    """The grouped GEMMs' persistent-schedule workspace for (device, stream):
    allocated zeroed once (its flags must start at zero; every GEMM call
    leaves them zero), reused by every later call on that stream."""
    import torch
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    ws = _GEMM_WS.get(key)
    if ws is None:
        with torch.cuda.device(key[0]):
            nbytes = int(load().ffmoe_gemm_workspace_bytes())
        if nbytes <= 0:
            raise FFMoEError("ffmoe_gemm_workspace_bytes failed: no device")
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        _GEMM_WS[key] = ws
    return ws


def check_gemm_workspaces():
    """Raises FFMoEError if a grouped GEMM on any cached workspace reported a
    timed-out stream-K wait (its output was wrong); the workspace is cleared
    first, so later calls are sound.  Synchronises each workspace's stream."""
    import torch
    for (dev, stream), ws in list(_GEMM_WS.items()):
        with torch.cuda.device(dev):
            call("ffmoe_gemm_check", ws.data_ptr(), stream)


def route_workspace_bytes(N, E, k):
    return int(load().ffmoe_route_workspace_bytes(N, E, k))


def set_lds_transpose(enable):
    return load().ffmoe_set_lds_transpose(1 if enable else 0)
