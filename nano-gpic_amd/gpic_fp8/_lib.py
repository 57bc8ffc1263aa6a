"""ctypes boundary to libgpic_fp8.so, the HIP kernels of the FP8 linear path (include/gpic_fp8.h).

There is no CPU path: a missing library, a CPU tensor or a failed launch raises RuntimeError.

torch is imported before the library is opened, so libgpic_fp8.so binds to the HIP runtime torch already loaded
(both are SONAME libamdhip64.so.7): torch's stream handles and device pointers are valid in our calls.
"""
import contextlib
import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libgpic_fp8.so")

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_sz = ctypes.c_size_t

# name -> (restype, argtypes), exactly the functions declared in include/gpic_fp8.h
SIGNATURES = {
    "gpic_fp8_version": (ctypes.c_char_p, []),
    "gpic_fp8_status_string": (ctypes.c_char_p, [_int]),
    "gpic_fp8_cast_workspace_bytes": (_sz, []),
    "gpic_fp8_set_single_pass": (None, [_int, _int]),
    "gpic_fp8_tcast": (_int, [_vp, _int, _i64, _vp, _vp, _vp, _vp]),
    "gpic_fp8_tcast_noalloc": (_int, [_vp, _int, _i64, _vp, _vp, _vp]),
    "gpic_fp8_tcast_t": (_int, [_vp, _int, _i64, _i64, _vp, _vp, _i64, _vp, _vp, _vp]),
    "gpic_fp8_tcast_t_group": (_int, [_int, _vp, _int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "gpic_fp8_tcast_heads": (_int, [_vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    "gpic_fp8_swiglu_tcast": (_int, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _vp]),
    "gpic_fp8_swiglu_tcast_t": (_int, [_vp, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _i64, _vp, _vp, _vp]),
    "gpic_fp8_swiglu_bwd": (_int, [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp]),
    "gpic_fp8_swiglu_bwd_t": (_int, [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp]),
    "gpic_fp8_res_mod_rmsnorm": (_int, [_vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64,
                                         ctypes.c_float, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "gpic_fp8_res_mod_rmsnorm_bwd_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "gpic_fp8_res_mod_rmsnorm_bwd": (_int, [_vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp, _i64, _i64, _i64,
                                             _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "gpic_fp8_gemm_workspace_bytes": (_sz, [_i64, _i64, _i64]),
    "gpic_fp8_gemm": (_int, [_vp, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp, _sz, _vp]),
    "gpic_fp8_gemm_mn": (_int, [_vp, _i64, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _vp, _sz, _vp]),
}

DTYPE_CODE = {torch.bfloat16: 0, torch.float32: 1}

_lib = None


def lib():
    """The loaded library (opened once). Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python nano-gpic_amd/gpic_fp8/build.py` "
                               "(hipcc, gfx950). The FP8 path has no CPU fallback.")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(status, what):
    if status != 0:
        msg = lib().gpic_fp8_status_string(status).decode()
        raise RuntimeError(f"{what} failed: {msg} (status {status})")


_IMPL = {}   # custom op -> the function it was made from


def custom_op(name):
    """torch.library.custom_op(name, mutates_args=()) that also keeps the function it wraps, for call()."""
    def deco(fn):
        op = torch.library.custom_op(name, mutates_args=())(fn)
        _IMPL[op] = fn
        return op
    return deco


def call(op, *args):
    """op(*args) for the path's own calls (the autograd Functions, one op inside another): outside torch.compile
    tracing the op's function runs directly, skipping the dispatcher (~10 us of host time per call, which bounds
    blocks of short kernels); under tracing the op itself, so a compiled graph holds the opaque custom op. Any other
    callable (a stand-in put in an op's place) is called as it is."""
    fn = None if torch.compiler.is_compiling() else _IMPL.get(op)
    return fn(*args) if fn is not None else op(*args)


def require_gpu(*tensors):
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(f"gpic_fp8 runs on the GPU only (HIP kernels); got a tensor on {t.device}")


# The current stream's raw handle without building a torch.cuda.Stream object (~1.5 us less host time per call)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _index(device):
    return device.index if device.index is not None else torch.cuda.current_device()


def stream_ptr(device):
    """The raw handle (hipStream_t) of `device`'s current stream."""
    index = _index(device)
    return _raw_stream(index) if _raw_stream is not None else torch.cuda.current_stream(index).cuda_stream


def on_device(device):
    """`device` made current for the calls inside, as torch.cuda.device(device) does, skipping the two device switches
    when it already is (the common case)."""
    if device.index is None or device.index == torch.cuda.current_device():
        return contextlib.nullcontext()
    return torch.cuda.device(device)


def ptr(t):
    return None if t is None else t.data_ptr()


def aligned(t):
    """t itself if its storage pointer is 16-byte aligned, else an aligned copy."""
    return t if t.data_ptr() % 16 == 0 else t.clone()


_WORKSPACES = {}   # (device index, stream handle) -> the cast workspace of that stream


def set_single_pass(enabled=True, wait_us=-1):
    """Single-pass casts on (default) or off, and the wait bound in microseconds (-1: the library default); see
    gpic_fp8_set_single_pass in include/gpic_fp8.h. The output bytes do not depend on either."""
    lib().gpic_fp8_set_single_pass(int(bool(enabled)), int(wait_us))


def _new_workspace(index, nbytes):
    """Device memory for a cast workspace, outside any CUDA-graph memory pool where that is possible. During a
    cudagraph-tree warm-up, torch serves every allocation of the current thread from the graph's private pool, and a
    workspace kept in this module's cache there would be live storage the trees do not account for (they refuse it).
    So it is allocated by a short-lived helper thread, whose allocations come from the ordinary pool. While the
    current stream is capturing (a first cast inside a torch.cuda.graph capture) a fresh device allocation elsewhere
    could break the capture, so the capture's own pool serves it and the graph keeps it alive."""
    dev = torch.device("cuda", index)
    if torch.cuda.is_current_stream_capturing():
        return torch.empty(nbytes // 4, dtype=torch.int32, device=dev)
    out = {}
    caller = torch.cuda.current_stream(dev)

    def alloc():
        # on the caller's stream: the caching allocator hands out a block only once the work queued on its stream
        # before its last free has run, so the block is free to be zeroed and used on that stream at once (on the
        # helper thread's default stream instead, kernels still running there could write over the fresh words)
        try:
            with torch.cuda.stream(caller):
                out["ws"] = torch.empty(nbytes // 4, dtype=torch.int32, device=dev)
        except BaseException as e:   # re-raised on the caller's thread
            out["err"] = e

    t = threading.Thread(target=alloc, name="gpic_fp8-workspace")
    t.start()
    t.join()
    if "err" in out:
        raise out["err"]
    return out["ws"]


_GEMM_WS = {}   # (device index, M, N, K) -> gpic_fp8_gemm_workspace_bytes (the plan is fixed per device and shape)


def gemm_workspace_bytes(device, M, N, K):
    key = (_index(device), M, N, K)
    n = _GEMM_WS.get(key)
    if n is None:
        n = _GEMM_WS[key] = lib().gpic_fp8_gemm_workspace_bytes(M, N, K)
    return n


def cast_workspace(device):
    """The cast workspace of `device`'s current stream: partial maxima, the SwiGLU sigmoid table and the single-pass
    casts' tagged partials with their call counter (an epoch word the kernels advance on the device). Created once per
    (device, stream) and kept: the counter must survive from call to call, and casts on different streams, which may
    overlap, get different workspaces. It is zeroed with a fill kernel on the stream that uses it, so under graph
    capture the fill is part of the graph (clearing it again on every replay, which the epoch scheme allows) and no
    memset node is recorded."""
    device = torch.device(device)
    index = _index(device)
    key = (index, stream_ptr(device))
    ws = _WORKSPACES.get(key)
    if ws is None:
        ws = _new_workspace(index, lib().gpic_fp8_cast_workspace_bytes())
        ws.zero_()
        _WORKSPACES[key] = ws
    return ws
