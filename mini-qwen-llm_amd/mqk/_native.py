"""ctypes binding of libmqk.so (the C ABI declared in include/mqk.h).

The library is loaded after ``torch`` so that it binds to the HIP runtime torch
already mapped (same soname), which keeps one runtime per process and lets
torch-allocated device pointers and torch streams be passed straight through.
A missing or unloadable library raises :class:`MqkNativeError`; nothing in
this package falls back to another implementation.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch  # (imported before the HIP library is mapped)

LIB_PATH = Path(os.environ.get("MQK_LIBRARY", Path(__file__).with_name("libmqk.so")))

MQK_OK = 0
MQK_SCALE_BF16 = 0
MQK_SCALE_FP16 = 1

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t

class PagedKV(ctypes.Structure):
    """struct mqk_paged_kv (include/mqk.h)."""
    _fields_ = [
        ("k_cache", ctypes.c_void_p),
        ("v_cache", ctypes.c_void_p),
        ("block_table", ctypes.c_void_p),
        ("bt_rows", ctypes.c_int64),
        ("bt_cols", ctypes.c_int64),
        ("num_blocks", ctypes.c_int64),
        ("block_size", ctypes.c_int32),
        ("kv_seq", ctypes.c_void_p),
        ("kv_pos", ctypes.c_void_p),
    ]


_KV = ctypes.POINTER(PagedKV)


class FusedExt(ctypes.Structure):
    """struct mqk_fused_ext (include/mqk.h)."""
    _fields_ = [
        ("cu_seqlens", ctypes.c_void_p),
        ("seq_pos0", ctypes.c_void_p),
        ("n_seqs", ctypes.c_int64),
        ("in_gamma", ctypes.c_void_p),
        ("in_eps", ctypes.c_float),
        ("kv", _KV),
    ]


_EXT = ctypes.POINTER(FusedExt)

# name -> (restype, argtypes); mirrors include/mqk.h.
SIGNATURES = {
    "mqk_version": (_I, []),
    "mqk_error_string": (ctypes.c_char_p, [_I]),
    "mqk_last_error_detail": (ctypes.c_char_p, []),
    "mqk_fused_qkv_rope_bf16": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P,     # x w_q w_k w_v q_gamma k_gamma cos sin positions
         _I64, _I64, _I64, _I, _I, _I,           # T S hidden Hq Hkv D
         _I64, _F, _P, _P, _P, _P, _SZ, _P],     # cos_rows eps q k v workspace ws_bytes stream
    ),
    "mqk_fused_qkv_rope_f32": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P,     # x w_q w_k w_v q_gamma k_gamma cos sin positions
         _I64, _I64, _I64, _I, _I, _I,           # T S hidden Hq Hkv D
         _I64, _F, _P, _P, _P, _P],              # cos_rows eps q k v stream
    ),
    "mqk_fused_qkv_rope_f16": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P,     # x w_q w_k w_v q_gamma k_gamma cos sin positions
         _I64, _I64, _I64, _I, _I, _I,           # T S hidden Hq Hkv D
         _I64, _F, _P, _P, _P, _P],              # cos_rows eps q k v stream
    ),
    "mqk_fused_qkv_rope_workspace_size": (_SZ, [_I64, _I, _I, _I64]),
    "mqk_fused_qkv_rope_workspace_size_hd": (_SZ, [_I64, _I, _I, _I64, _I]),
    "mqk_fused_qkv_rope_bf16_noalloc": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P,     # x w_q w_k w_v q_gamma k_gamma cos sin positions
         _I64, _I64, _I64, _I, _I, _I,           # T S hidden Hq Hkv D
         _I64, _F, _P, _P, _P, _P],              # cos_rows eps q k v stream
    ),
    "mqk_qk_norm_rope_bf16": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P,             # q_raw k_raw q_gamma k_gamma cos sin positions
         _I64, _I64, _I, _I, _I,                 # T S Hq Hkv D
         _I64, _F, _P, _P, _P],                  # cos_rows eps q_out k_out stream
    ),
    "mqk_w4a16_gemm": (
        _I, [_P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _P, _P],
    ),
    "mqk_w4a16_gemm_workspace_size": (_SZ, [_I64, _I64, _I64]),
    "mqk_w4a16_gemm_ex": (
        _I, [_P, _P, _P, _P, _I64, _I64, _I64, _I, _I, _P, _P, _SZ, _P],
    ),
    "mqk_fused_qkv_rope_w4a16": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P,  # x, (qw, sc, qz) x 3
         _I, _I,                                  # group scale_type
         _P, _P, _P, _P, _P,                      # q_gamma k_gamma cos sin positions
         _I64, _I64, _I64, _I, _I, _I,            # T S hidden Hq Hkv D
         _I64, _F, _P, _P, _P, _P, _SZ, _P],      # cos_rows eps q k v workspace ws_bytes stream
    ),
    "mqk_fused_qkv_rope_paged_bf16": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P,     # x w_q w_k w_v q_gamma k_gamma cos sin positions
         _I64, _I64, _I64, _I, _I, _I,           # T S hidden Hq Hkv D
         _I64, _F, _P, _P, _P, _KV, _P, _SZ, _P],  # cos_rows eps q k v kv workspace ws_bytes stream
    ),
    "mqk_fused_qkv_rope_paged_w4a16": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P,  # x, (qw, sc, qz) x 3
         _I, _I,                                  # group scale_type
         _P, _P, _P, _P, _P,                      # q_gamma k_gamma cos sin positions
         _I64, _I64, _I64, _I, _I, _I,            # T S hidden Hq Hkv D
         _I64, _F, _P, _P, _P, _KV, _P, _SZ, _P], # cos_rows eps q k v kv workspace ws_bytes stream
    ),
    "mqk_fused_qkv_rope_ex_workspace_size": (_SZ, [_I64, _I, _I, _I64, _EXT]),
    "mqk_fused_qkv_rope_ex_bf16": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P,     # x w_q w_k w_v q_gamma k_gamma cos sin positions
         _I64, _I64, _I64, _I, _I, _I,           # T S hidden Hq Hkv D
         _I64, _F, _P, _P, _P, _EXT, _P, _SZ, _P],  # cos_rows eps q k v ext workspace ws_bytes stream
    ),
    "mqk_fused_qkv_rope_ex_w4a16": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P,  # x, (qw, sc, qz) x 3
         _I, _I,                                  # group scale_type
         _P, _P, _P, _P, _P,                      # q_gamma k_gamma cos sin positions
         _I64, _I64, _I64, _I, _I, _I,            # T S hidden Hq Hkv D
         _I64, _F, _P, _P, _P, _EXT, _P, _SZ, _P],  # cos_rows eps q k v ext workspace ws_bytes stream
    ),
    "mqk_set_option": (_I, [ctypes.c_char_p, _I64]),
    "mqk_get_option": (_I64, [ctypes.c_char_p]),
    "mqk_tile_variants": (ctypes.c_char_p, []),
    "mqk_read_probe": (_I, [_P, _SZ, _I, _P, _P]),
    "mqk_clock_probe": (_I, [_P, _I, _P]),
}


class MqkNativeError(RuntimeError):
    """libmqk.so is missing, failed to load, or returned an error status."""


_lock = threading.Lock()
_lib = None


def library() -> ctypes.CDLL:
    """The loaded libmqk.so (loaded on first use)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise MqkNativeError(
                    f"libmqk.so not found at {LIB_PATH}; build it with "
                    "`python mini-qwen-llm_amd/csrc/build.py` (the mqk ops have no fallback path)")
            try:
                lib = ctypes.CDLL(str(LIB_PATH))
            except OSError as exc:
                raise MqkNativeError(f"cannot load {LIB_PATH}: {exc}") from exc
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def call(device: torch.device, fn, *args) -> int:
    """Run one native entry point with ``device`` as the current HIP device.

    libmqk launches on the calling thread's current device, so a caller whose
    tensors live on another GPU than the current one (one process driving
    several GPUs) still gets the kernels on the tensors' device, next to the
    stream and workspace that belong to it.  (The device is switched only when
    it differs: the switch costs more host time than a decode kernel's launch.)"""
    if torch.cuda.current_device() == device.index:
        return fn(*args)
    with torch.cuda.device(device):
        return fn(*args)


def stream_handle(device: torch.device) -> int:
    """The raw hipStream_t of torch's current stream on ``device`` (what
    ``torch.cuda.current_stream(device).cuda_stream`` returns, without building
    the stream object on every call)."""
    if _raw_stream is not None:
        return int(_raw_stream(device.index))
    return int(torch.cuda.current_stream(device).cuda_stream)


# (torch's own accessor of the raw current stream; absent in some builds)
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def check(status: int, what: str) -> None:
    """Raise :class:`MqkNativeError` for a non-zero mqk status."""
    if status == MQK_OK:
        return
    lib = library()
    msg = lib.mqk_error_string(status).decode()
    detail = lib.mqk_last_error_detail().decode()
    raise MqkNativeError(f"{what} failed: {msg} ({status}){': ' + detail if detail else ''}")


def set_option(name: str, value: int) -> None:
    check(library().mqk_set_option(name.encode(), int(value)), f"mqk_set_option({name})")


def get_option(name: str) -> int:
    return int(library().mqk_get_option(name.encode()))


def tile_variants() -> str:
    return library().mqk_tile_variants().decode()


def version() -> int:
    return int(library().mqk_version())


# ---------------------------------------------------------------------------
# Workspace: one zero-initialised device buffer per (device, stream).  The
# kernels leave its arrival counters at zero after each call, so it is zeroed
# only when allocated.  Keyed by stream because calls that may overlap must not
# share a workspace.
#
# A HIP graph captured on a stream keeps the workspace address it was captured
# with and writes partials and counters there on every replay -- whichever stream
# it is replayed on.  A replay on another stream therefore shares the capture
# stream's workspace: it must not overlap calls issued on the capture stream (or
# other replays of graphs captured there); order them with events, or capture on
# a stream that issues nothing else.  A buffer is
# therefore never released once a launch has used it: when a call needs more,
# the stream gets a new, larger buffer (at least twice the old size, so this
# happens a few times per stream at most) and the old one is retired, kept
# allocated and zero-countered for the life of the process, where graphs
# captured earlier still find it.  A buffer cannot be created during capture
# (its zero fill would run only at replay), so that raises instead: run the op
# once eagerly at the largest size before capturing.
# ---------------------------------------------------------------------------
_ws_lock = threading.Lock()
_workspaces: dict = {}
_retired: list = []


def workspace(device: torch.device, stream, nbytes: int):
    """The workspace of ``stream`` (a torch stream, or the raw handle of the
    device's current stream) with at least ``nbytes`` bytes; None for 0."""
    if nbytes <= 0:
        return None
    handle = stream if isinstance(stream, int) else int(stream.cuda_stream)
    key = (device.index, handle)
    buf = _workspaces.get(key)  # (the common case: an existing buffer that is large enough)
    if buf is not None and buf.numel() >= nbytes:
        return buf
    if isinstance(stream, int):
        stream = torch.cuda.current_stream(device)
        if int(stream.cuda_stream) != handle:
            raise MqkNativeError("a raw stream handle must be the device's current stream")
    with _ws_lock:
        buf = _workspaces.get(key)
        if buf is None or buf.numel() < nbytes:
            if torch.cuda.is_current_stream_capturing():
                raise MqkNativeError(
                    f"the mqk workspace of this stream must grow to {nbytes} bytes during HIP-graph "
                    "capture; run the op once eagerly on this stream at the largest size before capturing")
            old = 0 if buf is None else buf.numel()
            size = max(nbytes, 2 * old, 1 << 20)
            with torch.cuda.stream(stream):
                new = torch.zeros(size, dtype=torch.uint8, device=device)
            if buf is not None:
                _retired.append(buf)  # graphs captured earlier may still point at it
            _workspaces[key] = buf = new
        return buf


# Word of the workspace's statistics line that counts the heads the decode kernel
# finished on its recompute path (include/mqk.h: after the 1024 arrival counters).
_RECOMPUTE_WORD = 1024


def decode_recomputes(device=None, stream=None) -> int:
    """Heads the decode kernel has finished on its recompute path (some split of
    the head ran on another XCD than the grid assumes, e.g. on a partitioned
    GPU) in the workspace of ``stream`` (default: the current stream) since it
    was allocated; 0 before its first use.  Synchronises with that stream."""
    device = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    stream = torch.cuda.current_stream(device) if stream is None else stream
    with _ws_lock:
        buf = _workspaces.get((device.index, int(stream.cuda_stream)))
    if buf is None:
        return 0
    stream.synchronize()
    return int(buf[: 4 * (_RECOMPUTE_WORD + 1)].view(torch.int32)[_RECOMPUTE_WORD].item())


def retired_workspaces() -> int:
    """Number of superseded workspaces kept alive for graphs captured earlier."""
    return len(_retired)


def workspace_bytes() -> dict:
    """Device bytes the workspaces hold: ``{"current": ..., "retired": ...}`` (the
    buffers streams use now, and the superseded ones kept for captured graphs)."""
    with _ws_lock:
        return {"current": sum(b.numel() for b in _workspaces.values()),
                "retired": sum(b.numel() for b in _retired)}


def release_workspaces(retired_only: bool = True) -> int:
    """Drop the superseded workspaces (``retired_only``), or every workspace, and
    return the bytes released to torch's allocator.  Only for callers that know
    no HIP graph captured earlier still replays the op: a graph keeps the
    workspace address it was captured with, and a replay after its buffer was
    released writes freed memory.  A stream whose workspace was released gets a
    new zero-filled one at its next call (so not during capture)."""
    with _ws_lock:
        n = sum(b.numel() for b in _retired)
        _retired.clear()
        if not retired_only:
            n += sum(b.numel() for b in _workspaces.values())
            _workspaces.clear()
    return n


def blocks(heads: int, head_dim: int) -> int:
    """Heads -> the kernels' 128-column blocks (two heads per block at head_dim 64):
    the head counts the workspace-size queries take."""
    return heads * head_dim // 128


def fused_workspace_bytes(T: int, H_Q: int, H_KV: int, hidden: int, D: int, ext=None) -> int:
    """Workspace bytes of one fused call: the fused plan's over 128-column blocks
    (with ``ext``: the _ex query, which adds the input-norm scales), and for head
    sizes other than 64 and 128 at least what each projection's own plan needs."""
    lib = library()
    if ext is None:
        n = int(lib.mqk_fused_qkv_rope_workspace_size(T, blocks(H_Q, D), blocks(H_KV, D), hidden))
    else:
        n = int(lib.mqk_fused_qkv_rope_ex_workspace_size(T, blocks(H_Q, D), blocks(H_KV, D), hidden,
                                                         ctypes.byref(ext)))
    if D not in (64, 128):
        n = max(n, int(lib.mqk_fused_qkv_rope_workspace_size_hd(T, H_Q, H_KV, hidden, D)))
    return n


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()
