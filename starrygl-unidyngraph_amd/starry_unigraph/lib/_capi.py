"""ctypes binding of libstarrygl_mi355x.so (the C ABI in include/starrygl_mi355x.h).

The library is the only compute path: when it is missing, or when no GPU is
visible, every entry point raises ``RuntimeError``. There is no CPU fallback.
Device buffers are torch tensors (the caching allocator owns them); work is
enqueued on torch's current stream for the tensor's device.
"""
from __future__ import annotations

import ctypes
import os
import struct
import threading

import torch  # loads the HIP runtime first, so the library binds to the same one

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_NAME = "libstarrygl_mi355x.so"
LIB_PATH = os.path.join(_HERE, LIB_NAME)
ABI_VERSION = 22

SGL_DERR_NODE_RANGE = 1
SGL_DERR_EID_RANGE = 2
SGL_DERR_STALE_NODE_BITS = 4
SGL_FIXED_SHIFT = 40    # fractional bits of the predictor's int64 gradient accumulators
SGL_DONE_WORDS = 1088   # int32 words of sgl_predictor's completion counter
SGL_DONE_RANGE_WORD = 32   # its word that flags a value outside the fixed-point range
SGL_COMPACT_NOALLOC_MAX_QUERIES = 1 << 24   # sgl_recent_compact_noalloc's limit
SGL_LINK_METRICS_MAX_SCORES = 8192   # sgl_link_metrics' limit on positive + negative scores

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_sz = ctypes.c_size_t

# the attention's dropout arguments: p_att, p_out, seed, rng_step, pass, sv_sdrop
_DROP = [ctypes.c_float, ctypes.c_float, ctypes.c_uint64, _vp, _i32, _vp]

# name -> (restype, argtypes); mirrors include/starrygl_mi355x.h
SIGNATURES: dict[str, tuple] = {
    "sgl_abi_version": (ctypes.c_int, []),
    "sgl_last_error": (ctypes.c_char_p, []),
    "sgl_host_device_pointer": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)]),
    "sgl_tcsr_workspace_bytes": (_sz, [_i64, _i64]),
    "sgl_tcsr_build": (ctypes.c_int, [_i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp, _vp]),
    "sgl_recent_sample": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _vp, ctypes.c_int, _vp, _i64, _vp, _vp, _i32, _i32,
                                         _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "sgl_recent_sample_packed": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _vp, ctypes.c_int, _vp, _i64, _vp, _vp,
                                                _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "sgl_compact_workspace_bytes": (_sz, [_i64]),
    "sgl_recent_compact": (ctypes.c_int, [_i64, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz,
                                          _vp]),
    "sgl_recent_compact_noalloc": (ctypes.c_int, [_i64, _i32] + [_vp] * 11),
    "sgl_node_bits_words": (_i64, [_i64]),
    "sgl_negatives_from_draws": (ctypes.c_int, [_i64, _vp, _vp, _i64, _vp, _vp, _vp, _vp]),
    "sgl_batch_prepare": (ctypes.c_int, [_i64, _i64] + [_vp] * 24),
    "sgl_batch_prepare_metrics": (ctypes.c_int, [_i64, _i64] + [_vp] * 23 + [_i32, _i32, _vp, _vp, _vp, _vp, _vp,
                                                                              _i32, _vp, _vp, _vp, _vp]),
    "sgl_memory_update_lds_bytes": (_sz, [_i32, _i32]),
    "sgl_memory_update_bf16_tile_rows": (_i32, [_i32, _i32, _i64]),
    "sgl_memory_update": (ctypes.c_int, [_i32, _i32, _i32, _i64] + [_vp] * 25),
    "sgl_memory_update_bf16": (ctypes.c_int, [_i32, _i32, _i32, _i64] + [_vp] * 26),
    "sgl_gru_packed_elems": (_i64, [_i32, _i32]),
    "sgl_gru_pack_bf16": (ctypes.c_int, [_i32, _i32] + [_vp] * 6),
    "sgl_memory_commit": (ctypes.c_int, [_i32, _i64] + [_vp] * 11),
    "sgl_time_projection_forward": (ctypes.c_int, [_i32, _i64, _vp, _vp, _vp, ctypes.c_float, ctypes.c_float,
                                                   _vp, _vp, _vp, _vp]),
    "sgl_time_projection_backward": (ctypes.c_int, [_i32, _i64, _vp, _vp, _vp, ctypes.c_float, ctypes.c_float]
                                     + [_vp] * 8),
    "sgl_memory_gather": (ctypes.c_int, [_i32, _i64] + [_vp] * 8),
    "sgl_conv_tile_rows": (_i32, [_i32] * 4),
    "sgl_conv_backward_tile_rows": (_i32, [_i32] * 5),
    "sgl_edge_rows": (ctypes.c_int, [_i32] * 4 + [_i64] + [_vp] * 8),
    "sgl_conv_forward": (ctypes.c_int, [_i32] * 5 + [_i64] + [_vp] * 29 + _DROP + [_vp, _vp]),
    "sgl_conv_backward": (ctypes.c_int, [_i32] * 5 + [_i64] + [_vp] * 39 + _DROP + [_vp, _vp]),
    "sgl_dropout_masks": (ctypes.c_int, [_i64, _i32, _i32, _i32, ctypes.c_float, ctypes.c_float, ctypes.c_uint64,
                                         _vp, _i32, _vp, _vp, _vp]),
    "sgl_predictor": (ctypes.c_int, [_i64, _i32, _i64, _i32] + [_vp] * 20 + [_i64, _vp, _vp, _vp]),
    "sgl_link_metrics_work_doubles": (_i64, [_i32]),
    "sgl_link_metrics": (ctypes.c_int, [_i32, _i32, _vp, _vp, _vp, _vp, _vp, _i32, _vp, _vp, _vp, _vp]),
    "sgl_adam_step": (ctypes.c_int, [_i64] + [_vp] * 6 + [ctypes.c_float] * 5 + [_vp]),
    "sgl_adam_advance": (ctypes.c_int, [_vp, _vp, _vp]),
    "sgl_time_next_launch": (ctypes.c_int, [_vp, _vp]),
    "sgl_plan_op_kind": (_i32, [ctypes.c_char_p, _vp]),
    "sgl_plan_run": (ctypes.c_int, [_vp, _i32, _i32, _vp, _vp, _vp] + [ctypes.c_uint32] * 2 + [_i32, _vp, _vp]),
    "sgl_grad_adam": (ctypes.c_int, [_vp, _vp, _i32] + [_vp] * 5 + [_i32] + [_vp] * 2 + [ctypes.c_float] * 4
                      + [_vp, _vp]),
    "sgl_grad_shadows": (ctypes.c_int, [_vp, _vp, _i32, _vp, _vp, _vp]),
    "sgl_adam_coef": (ctypes.c_int, [_i32] + [_vp] * 3 + [ctypes.c_float] * 3 + [_vp] * 3),
}

_lock = threading.Lock()
_lib = None


def load_library(path: str | None = None) -> ctypes.CDLL:
    """Load (once) and type the C-ABI library. Raises RuntimeError if absent."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or LIB_PATH
        if not os.path.exists(p):
            raise RuntimeError(
                f"{LIB_NAME} not found at {p}: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "or `make -C starrygl-unidyngraph_amd/csrc`")
        lib = ctypes.CDLL(p)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        v = lib.sgl_abi_version()
        if v != ABI_VERSION:
            raise RuntimeError(f"{LIB_NAME} ABI version {v} != expected {ABI_VERSION}")
        if path is None:
            _lib = lib
        return lib


def lib() -> ctypes.CDLL:
    return _lib if _lib is not None else load_library()


def require_gpu(device=None) -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("starry_unigraph MI355X path needs a GPU (torch.cuda.is_available() is False); "
                           "there is no CPU fallback")
    if device is None:
        return torch.device("cuda", torch.cuda.current_device())
    d = torch.device(device)
    if d.type != "cuda":
        raise RuntimeError(f"device {d} is not a GPU; the MI355X path has no CPU fallback")
    return d if d.index is not None else torch.device("cuda", torch.cuda.current_device())


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().sgl_last_error()
        raise RuntimeError(f"{what}: {msg.decode() if msg else 'error code %d' % rc}")


def host_device_pointer(t: torch.Tensor) -> int:
    """The device-visible address of a pinned host tensor's first element
    (sgl_host_device_pointer), for a kernel that reads it in place."""
    if not t.is_pinned():
        raise RuntimeError("host_device_pointer: the tensor is not in pinned host memory")
    out = ctypes.c_void_p()
    check(lib().sgl_host_device_pointer(ctypes.c_void_p(t.data_ptr()), ctypes.byref(out)), "sgl_host_device_pointer")
    return int(out.value)


def ptr(t: torch.Tensor | None) -> int | None:
    """Device address of a tensor's first element; for an empty view the
    address inside its (non-empty) storage, so the C side never sees NULL for
    an array that merely has no elements this call."""
    if t is None:
        return None
    if t.numel() == 0:
        return t.untyped_storage().data_ptr() + t.storage_offset() * t.element_size()
    return t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
_dev_index: dict = {}


def stream_of(device: torch.device) -> int:
    """The current HIP stream of ``device`` (its raw handle). torch's
    current_stream() resolves the device through several Python layers on
    every call; the index is resolved once per device here."""
    if _raw_stream is None:
        return torch.cuda.current_stream(device).cuda_stream
    idx = _dev_index.get(device)
    if idx is None:
        idx = _dev_index[device] = torch.cuda._get_device_index(device, optional=True)
    return _raw_stream(idx)


class GradJob(ctypes.Structure):
    """struct sgl_grad_job of include/starrygl_mi355x.h (no bf16 copies
    unless sh_off / sht_off are given)."""
    _fields_ = [("x1", _vp), ("x2", _vp), ("s1", _i64), ("s2", _i64), ("off", _i64), ("ps1", _i64), ("ps2", _i64),
                ("ldo", _i32), ("rows", _i32), ("cols", _i32), ("kind", _i32), ("seg", _i32),
                ("r_fixed", _i32), ("r_extra", _i32), ("tiles_b", _i32), ("tile0", _i32), ("npass", _i32),
                ("sh_off", _i64), ("sht_off", _i64), ("sh_ld", _i32), ("sht_ld", _i32)]

    def __init__(self, **kw):
        kw.setdefault("sh_off", -1)
        kw.setdefault("sht_off", -1)
        super().__init__(**kw)


class Bf16Weights(ctypes.Structure):
    """struct sgl_bf16_weights of include/starrygl_mi355x.h."""
    _fields_ = [(n, _vp) for n in ("wq", "wk", "wv", "wout", "wkt", "wvt", "wot", "ws", "wd", "wst", "wdt")] + \
               [(n, _i32) for n in ("ld_q", "ld_c", "ld_o", "ld_h", "hp", "ld_d")]


SGL_OP_MAX_ARGS = 64


class Op(ctypes.Structure):
    """struct sgl_op of include/starrygl_mi355x.h (one recorded call)."""
    _fields_ = [("kind", _i32), ("nargs", _i32), ("a", ctypes.c_uint64 * SGL_OP_MAX_ARGS)]


_recording: list | None = None


class record:
    """Within ``with record() as calls:``, :func:`call` appends (name, args
    without the stream) to ``calls`` instead of launching."""

    def __enter__(self) -> list:
        global _recording
        if _recording is not None:
            raise RuntimeError("launch recordings do not nest")
        _recording = []
        return _recording

    def __exit__(self, *exc) -> None:
        global _recording
        _recording = None


def call(name: str, *args) -> int:
    """Call entry point ``name`` (its arguments end with the stream), or
    record the call when a recording is active (then 0 is returned; the
    entry point's checks run when the plan is replayed)."""
    rec = _recording
    if rec is not None:
        rec.append((name, args[:-1]))
        return 0
    return getattr(lib(), name)(*args)


def _slot(v, t) -> int:
    if v is None:
        return 0
    if t is ctypes.c_float:
        return struct.unpack("<I", struct.pack("<f", float(v)))[0]
    if t is _vp:
        if isinstance(v, ctypes.Array):
            return ctypes.addressof(v)
        if isinstance(v, ctypes.c_void_p):
            return v.value or 0
        return int(v) & 0xFFFFFFFFFFFFFFFF
    return int(v) & 0xFFFFFFFFFFFFFFFF


def pack_ops(calls: list) -> ctypes.Array:
    """Recorded calls -> an sgl_op array for sgl_plan_run (the recorded
    arguments must stay alive, e.g. host pointer arrays, as long as it is
    replayed)."""
    L = lib()
    ops = (Op * max(len(calls), 1))()
    for i, (name, args) in enumerate(calls):
        n = _i32(0)
        kind = L.sgl_plan_op_kind(name.encode(), ctypes.byref(n))
        argtypes = SIGNATURES[name][1][:-1]
        if kind < 0 or n.value != len(argtypes) or len(args) != len(argtypes):
            raise RuntimeError(f"{name}: not a plannable call ({len(args)} arguments recorded)")
        ops[i].kind = kind
        ops[i].nargs = n.value
        for j, (v, t) in enumerate(zip(args, argtypes)):
            ops[i].a[j] = _slot(v, t)
    return ops


class ErrorFlag:
    """A device int32 that kernels OR SGL_DERR_* bits into."""

    def __init__(self, device: torch.device):
        self.t = torch.zeros(1, dtype=torch.int32, device=device)

    def reset(self) -> None:
        self.t.zero_()

    def raise_if_set(self, what: str) -> None:
        v = int(self.t.item())
        if v:
            parts = []
            if v & SGL_DERR_NODE_RANGE:
                parts.append("node id out of range [0, num_nodes)")
            if v & SGL_DERR_EID_RANGE:
                parts.append("edge id out of range [0, 2^31)")
            if v & SGL_DERR_STALE_NODE_BITS:
                parts.append("node bitmap not clear at the batch preparation (a previous step's memory commit "
                             "did not run); the batch was given no roots")
            self.reset()
            raise RuntimeError(f"{what}: " + "; ".join(parts))


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
