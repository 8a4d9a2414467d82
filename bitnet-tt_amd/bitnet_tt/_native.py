"""ctypes binding of libbtl.so, the gfx950 BitLinear library (include/btl.h).

The library is the only compute path of this package: every device operation
goes through it, and a missing or stale library raises instead of falling back
to anything else.  Tensors are passed as raw device pointers together with the
current HIP stream of the calling thread (``torch.cuda.current_stream()``), so
calls are stream-ordered and can be recorded into a HIP graph.
"""

from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
# BTL_LIBRARY names another build of the same library (the host-sanitizer
# build of tests/host_asan.sh); the default is the in-tree product build.
LIB_PATH = os.environ.get("BTL_LIBRARY") or os.path.join(_HERE, "_lib", "libbtl.so")

# Status codes and epilogue modes (include/btl.h).
BTL_OK = 0
STATUS_NAMES = {
    1: "BTL_ERR_NULL",
    2: "BTL_ERR_SHAPE",
    3: "BTL_ERR_ALIGN",
    4: "BTL_ERR_WORKSPACE",
    5: "BTL_ERR_ARG",
    6: "BTL_ERR_LAUNCH",
}
EPI_SCALE = 0
EPI_RELU2_MUL = 1
MAX_SEGMENTS = 4
MAX_K = 16384

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t



class LayerWeight(ctypes.Structure):
    """btl_layer_weight_t: one BitLinear of a btl_decode_step launch."""

    _fields_ = [
        ("wdev", ctypes.c_void_p),
        ("seg_scale", ctypes.c_float * MAX_SEGMENTS),
        ("seg_end", ctypes.c_int64 * MAX_SEGMENTS),
        ("nseg", ctypes.c_int),
        ("gamma", ctypes.c_void_p),
    ]


def layer_weight(w, gamma) -> LayerWeight:
    """LayerWeight of a PackedTernaryWeight and the RMSNorm gain of its input."""
    n = len(w.segment_scales)
    if not 1 <= n <= MAX_SEGMENTS:
        raise ValueError(f"1..{MAX_SEGMENTS} weight-scale segments are supported, got {n}")
    lw = LayerWeight()
    lw.wdev = w.data.data_ptr()
    for i in range(MAX_SEGMENTS):
        lw.seg_scale[i] = float(w.segment_scales[i]) if i < n else 0.0
        lw.seg_end[i] = int(w.segment_ends[i]) if i < n else 0
    lw.nseg = n
    lw.gamma = gamma.data_ptr()
    return lw


_LWP = ctypes.POINTER(LayerWeight)

# name -> (argtypes, restype); the exported C ABI, one entry per declaration.
EXPORTS = {
    "btl_last_error": ([], ctypes.c_char_p),
    "btl_version": ([], _I),
    "btl_check_coresident": ([_I64, _I64, _I64], _I),
    "btl_packed_tile_count": ([_I64, _I64], _I64),
    "btl_packed_dram_bytes": ([_I64, _I64], _I64),
    "btl_devlayout_words": ([_I64, _I64], _I64),
    "btl_act_bytes": ([_I64, _I64], _I64),
    "btl_choose_splitk": ([_I64, _I64, _I64, _I], _I),
    "btl_gemm_tiling": ([_I64, _I64, _I64, _I, _I, _P], _I),
    "btl_gemm_workspace_bytes": ([_I64, _I64, _I64, _I, _I], _I64),
    "btl_fused_workspace_bytes": ([_I64, _I64, _I64, _I, _I], _I64),
    "btl_fused_error_offset": ([], _I64),
    "btl_weight_quant_scratch_bytes": ([_I64], _I64),
    "btl_weight_quant_ternary": ([_P, _I64, _F, _P, _P, _P, _SZ, _P], _I),
    "btl_pack_tiles": ([_P, _I64, _I64, _P, _P], _I),
    "btl_unpack_tiles": ([_P, _I64, _I64, _P, _P], _I),
    "btl_repack": ([_P, _I64, _I64, _P, _P], _I),
    "btl_quant_absmax": ([_P, _I64, _I64, _I64, _P, _F, _P, _P, _P, _P, _P, _P, _P], _I),
    "btl_rmsnorm": ([_P, _I64, _I64, _I64, _P, _F, _P, _P], _I),
    "btl_gemm_i8t2": (
        [_P, _P, _P, _I64, _I64, _I64, _P, _P, _P, _I, _I, _P, _P, _P, _P, _SZ, _I, _P],
        _I,
    ),
    "btl_bitlinear_fused": (
        [_P, _I64, _I64, _I64, _P, _F, _P, _I64, _P, _P, _I, _I, _P, _P, _P, _P, _P, _SZ, _I, _P],
        _I,
    ),
    "btl_bitlinear_fused_noalloc": (
        [_P, _I64, _I64, _I64, _P, _F, _P, _I64, _P, _P, _I, _I, _P, _P, _P, _P, _P, _I, _P],
        _I,
    ),
    "btl_decode_step_workspace_bytes": ([_I64, _I64, _I64, _I64, _I64], _I64),
    "btl_decode_step_error_offset": ([], _I64),
    "btl_decode_step_prepare": ([_I64, _I64, _I64, _I64, _I64, _LWP, _P, _SZ], _I),
    "btl_decode_step": ([_I64, _I64, _I64, _I64, _I64, _F, _P, _P, _P, _P, _P, _SZ, _P], _I),
    "btl_decode_step_floor": ([_I64, _I64, _I64, _I64, _I64, _P, _SZ, _P], _I),
    "btl_decode_step_clear_share": ([_I, _I64, _P, _I64], _I),
    "btl_decode_step_attention_prepare": ([_I64, _I64, _I64, _I64, _I64, _P, _P, _P, _SZ], _I),
    "btl_decode_step_full": (
        [_I64, _I64, _I64, _I64, _I64, _F, _I64, _I64, _P, _P, _P, _I, _F, _P, _P, _P, _P, _P, _SZ, _P],
        _I,
    ),
    "btl_gemm_i8t2_dot4": ([_P, _P, _I64, _I64, _I64, _P, _P, _P], _I),
    "btl_lm_head_weight_bytes": ([_I64, _I64], _I64),
    "btl_lm_head_workspace_bytes": ([], _I64),
    "btl_lm_head_repack": ([_P, _I64, _I64, _P, _P], _I),
    "btl_lm_head": ([_P, _I64, _I64, _I64, _P, _P, _P, _P, _SZ, _P], _I),
    "btl_decode_attention_workspace_bytes": ([_I64, _I64, _I64, _I64], _I64),
    "btl_decode_attention_error_offset": ([_I64, _I64], _I64),
    "btl_decode_attention": ([_P, _I64, _I64, _I64, _I64, _I64, _P, _P, _P, _I, _F, _P, _P, _P, _P, _SZ, _P], _I),
}


class NativeLibraryError(RuntimeError):
    """libbtl.so is missing or unusable; there is no other compute path."""


_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    """Load libbtl.so once and declare every exported signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise NativeLibraryError(
                f"{LIB_PATH} is not built; build it with __graft_entry__.build() "
                "(hipcc --offload-arch=gfx950). The BitLinear path has no other backend."
            )
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in EXPORTS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def last_error() -> str:
    msg = lib().btl_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    if rc != BTL_OK:
        raise RuntimeError(f"{what} failed with {STATUS_NAMES.get(rc, rc)}: {last_error()}")


def ptr(t) -> ctypes.c_void_p | None:
    """Device pointer of a tensor (None passes NULL)."""
    if t is None:
        return None
    return ctypes.c_void_p(t.data_ptr())


def require_cuda(t, name: str) -> None:
    if t is None:
        return
    if not t.is_cuda:
        raise ValueError(
            f"{name} must be a tensor on a ROCm GPU device; the BitLinear path runs only "
            "through the gfx950 kernels"
        )
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def stream_of(device) -> ctypes.c_void_p:
    import torch

    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def segments_arrays(scales, ends):
    """Host arrays for the per-segment epilogue scales."""
    n = len(scales)
    if not 1 <= n <= MAX_SEGMENTS:
        raise ValueError(f"1..{MAX_SEGMENTS} weight-scale segments are supported, got {n}")
    sc = (ctypes.c_float * n)(*[float(s) for s in scales])
    en = (ctypes.c_int64 * n)(*[int(e) for e in ends])
    return sc, en, n


# Per (device, stream) workspace.  Calls on one stream are ordered, so they
# can share it; the activation kernel of every fused call clears the split-K
# counters it uses.
_workspaces: dict = {}


def has_workspace(device, nbytes: int, kind: str = "bitlinear") -> bool:
    """True when the current stream already owns a workspace of nbytes."""
    import torch

    buf = _workspaces.get((kind, _device_key(device), torch.cuda.current_stream(device).cuda_stream))
    return buf is not None and buf.numel() >= nbytes


# Byte offsets of the sticky error words each workspace holds (a bounded wait
# of a kernel that ran out sets one; see check_errors).
_error_words: dict = {}
# What a workspace was prepared for (data_ptr -> owner object), for launches
# whose workspace holds host-prepared state (the decode step's weight table).
_prepared_for: dict = {}


# Host-side set-up to redo after a workspace has been zero-filled by
# check_errors (data_ptr -> callable), for workspaces whose start state is not
# all zeros (the decode step's weight table and operand tiles).
_reset_hooks: dict = {}


def workspace_prepared_for(buf):
    return _prepared_for.get(buf.data_ptr())


def set_workspace_reset(buf, fn) -> None:
    _reset_hooks[buf.data_ptr()] = fn


def set_workspace_prepared_for(buf, owner) -> None:
    _prepared_for[buf.data_ptr()] = owner


def _device_key(device) -> str:
    import torch

    d = torch.device(device)
    if d.index is None:
        d = torch.device(d.type, torch.cuda.current_device())
    return str(d)


def workspace(device, nbytes: int, kind: str = "bitlinear", error_offset: int | None = None):
    """Zero-filled device workspace of at least nbytes for the current stream.

    kind separates workspaces whose layouts differ ("bitlinear" for
    btl_bitlinear_fused / btl_gemm_i8t2, "step" for btl_decode_step).  A
    workspace that grows is replaced by a fresh zero-filled one; the old one
    is released in stream order, after the calls that used it.
    ``error_offset`` registers the byte offset of a sticky error word inside
    the workspace, which :func:`check_errors` reads."""
    import torch

    stream = torch.cuda.current_stream(device)
    key = (kind, _device_key(device), stream.cuda_stream)
    buf = _workspaces.get(key)
    if buf is None or buf.numel() < nbytes:
        if buf is not None:
            _prepared_for.pop(buf.data_ptr(), None)
            _reset_hooks.pop(buf.data_ptr(), None)
        size = max(int(nbytes), 1 << 20)
        buf = torch.zeros(size, dtype=torch.uint8, device=device)
        _prepared_for.pop(buf.data_ptr(), None)
        _reset_hooks.pop(buf.data_ptr(), None)
        _workspaces[key] = buf
    if error_offset is not None:
        _error_words.setdefault(key, set()).add(int(error_offset))
    return buf


def check_errors(device=None) -> None:
    """Raise RuntimeError if any kernel on ``device`` set its sticky error word.

    The kernels that hand data between workgroups of one launch (the fused
    decode BitLinear, the decode step, decode attention) never hang: a wait
    that exceeds its spin limit sets a sticky error word in the call's
    workspace and the kernel finishes with invalid outputs.  This reads every
    registered error word of the device's workspaces (all streams) after a
    device synchronisation.  When one is set, the affected workspaces are
    zero-filled in place (the start state of their launch counters) and the
    host-side set-up registered for them (set_workspace_reset: the decode
    step's weight table and operand tiles) is redone, so later calls and
    graphs captured on them work again; RuntimeError names them: the outputs
    of the calls since the last check are not valid."""
    import torch

    dev = _device_key(device if device is not None else "cuda")
    keys = [k for k in _workspaces if k[1] == dev and _error_words.get(k)]
    if not keys:
        return
    torch.cuda.synchronize(dev)
    bad = []
    for key in keys:
        buf = _workspaces[key]
        for off in sorted(_error_words[key]):
            word = int(buf[off:off + 4].view(torch.int32).item())
            if word:
                bad.append((key, off, word))
    if not bad:
        return
    for key in {b[0] for b in bad}:
        _workspaces[key].zero_()
        torch.cuda.synchronize(dev)
        hook = _reset_hooks.get(_workspaces[key].data_ptr())
        if hook is not None:
            hook()
        else:
            _prepared_for.pop(_workspaces[key].data_ptr(), None)
    torch.cuda.synchronize(dev)
    what = ", ".join(f"{k[0]} workspace (stream {k[2]:#x}) word at byte {off} = {w}" for k, off, w in bad)
    raise RuntimeError(
        f"a kernel on {dev} set its error word ({what}): a bounded wait ran out, or a decode-attention position "
        "was out of range; the outputs of the calls since the last check are invalid, and the workspaces have "
        "been reset"
    )


def gemm_tiling(M: int, K: int, N: int, epilogue: int = EPI_SCALE, rowsum_given: bool = True) -> dict:
    """The tiling btl_gemm_i8t2 runs for a shape (a planning query)."""
    info = (ctypes.c_int32 * 6)()
    check(lib().btl_gemm_tiling(M, K, N, epilogue, int(bool(rowsum_given)), info), "btl_gemm_tiling")
    kind = ("decode", "tiles", "wide")[info[0]]
    return {"kind": kind, "rows": info[1], "col_tiles": info[2], "splitk": info[3], "k_groups": info[4],
            "tiles_per_wave": info[5]}
