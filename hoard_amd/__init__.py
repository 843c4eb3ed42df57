"""hoard_amd -- MI355X-native MoE expert stage of bgallon-dev/hoard.

The product is libhoard_moe.so (C++ orchestrator + HIP kernels for gfx950)
behind the C ABI in include/hoard_moe.h.  This module is ctypes plumbing for
tests and the bench: it loads the in-tree library and raises if it has not
been built -- there is no fallback path.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libhoard_moe.so"

TYPE_F32 = 0
TYPE_Q3_K = 11
TYPE_Q4_K = 12
TYPE_Q5_K = 13
TYPE_Q6_K = 14
BLOCK_BYTES = {TYPE_Q3_K: 110, TYPE_Q4_K: 144, TYPE_Q5_K: 176, TYPE_Q6_K: 210}

OK = 0
ERR_INVALID = -1
ERR_UNSUPPORTED = -2
ERR_HIP = -3
ERR_OOM = -4
ERR_STATE = -5
ERR_IO = -6


class HoardError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"hoard error {code}: {msg}")
        self.code = code


class MoeCfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in (
        "n_embd", "n_expert", "n_used", "n_ff", "n_ff_shexp", "n_layer", "renorm", "pool_k",
        "max_tokens")]


class LayerWeights(ctypes.Structure):
    _fields_ = [
        ("router", ctypes.c_void_p),
        ("gate_type", ctypes.c_int32), ("up_type", ctypes.c_int32), ("down_type", ctypes.c_int32),
        ("gate", ctypes.c_void_p), ("up", ctypes.c_void_p), ("down", ctypes.c_void_p),
        ("sh_gate_type", ctypes.c_int32), ("sh_up_type", ctypes.c_int32), ("sh_down_type", ctypes.c_int32),
        ("sh_gate", ctypes.c_void_p), ("sh_up", ctypes.c_void_p), ("sh_down", ctypes.c_void_p),
        ("sh_gate_inp", ctypes.c_void_p),
    ]


class MoeStats(ctypes.Structure):
    _fields_ = [
        ("reqs", ctypes.c_uint64), ("hits", ctypes.c_uint64), ("misses", ctypes.c_uint64),
        ("bytes_h2d", ctypes.c_uint64), ("tokens", ctypes.c_uint64),
        ("expert_hist", ctypes.c_uint64 * 1024), ("last_unique", ctypes.c_int32),
    ]


KERNEL_ROUTER, KERNEL_GATEUP, KERNEL_DOWN, KERNEL_DECODE, KERNEL_BATCHED, KERNEL_LAYER = 0, 1, 2, 3, 4, 5
KERNEL_NAMES = {KERNEL_ROUTER: "router", KERNEL_GATEUP: "gateup", KERNEL_DOWN: "down_combine",
                KERNEL_DECODE: "decode_persistent", KERNEL_BATCHED: "batched_experts", KERNEL_LAYER: "layer_fused"}
TRACE_PHASES = 12
OPT_PERSISTENT_DECODE = 1
OPT_PERSISTENT_AVAILABLE = 2
OPT_POOL_NAIVE = 3
OPT_DECODE_KERNEL = 4
OPT_DECODE_KERNELS_AVAILABLE = 5
OPT_LAYER_KERNELS = 6
OPT_DECODE_LAUNCH = 7
OPT_WAIT_LIMIT_US = 8
OPT_FAIL_UPLOAD = 9
OPT_LAYER_FUSED = 10
DECODE_AUTO, DECODE_XCD, DECODE_SPREAD = 0, 1, 2


class KernelTimes(ctypes.Structure):
    _fields_ = [("launches", ctypes.c_uint64 * 8), ("total_ms", ctypes.c_double * 8)]


class StoreLayer(ctypes.Structure):
    _fields_ = [("off", ctypes.c_uint64 * 3), ("stride", ctypes.c_uint64 * 3)]


class StoreCfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("readers", "ram_experts", "direct", "pinned")]


class StoreStats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in ("requests", "ram_hits", "file_reads", "bytes_read", "read_ns")] + \
               [("direct", ctypes.c_int32), ("ram_experts", ctypes.c_int32)]


_P = ctypes.c_void_p
_I = ctypes.c_int
# name -> (restype, argtypes); every symbol the public headers declare
ABI = {
    "hoard_last_error": (ctypes.c_char_p, []),
    "hoard_moe_create": (_I, [ctypes.POINTER(MoeCfg), ctypes.POINTER(_P)]),
    "hoard_moe_destroy": (None, [_P]),
    "hoard_moe_set_layer_weights": (_I, [_P, _I, ctypes.POINTER(LayerWeights)]),
    "hoard_moe_route": (_I, [_P, _I, _P, _P, _P, _P]),
    "hoard_moe_ffn_combine": (_I, [_P, _I, _P, _P, _P, _P, _P, _P]),
    "hoard_moe_layer": (_I, [_P, _I, _P, _P, _P, _P, _P, _P]),
    "hoard_moe_decode": (_I, [_P, _I, _I, _P, ctypes.c_float, _P]),
    "hoard_moe_profile": (_I, [_P, _I]),
    "hoard_moe_profile_read": (_I, [_P, ctypes.POINTER(KernelTimes)]),
    "hoard_moe_set_option": (_I, [_P, _I, _I]),
    "hoard_moe_get_option": (_I, [_P, _I, ctypes.POINTER(ctypes.c_int)]),
    "hoard_moe_sync_check": (_I, [_P]),
    "hoard_moe_phase_trace": (_I, [_P, _I]),
    "hoard_moe_phase_trace_read": (_I, [_P, _P, ctypes.c_size_t, ctypes.POINTER(ctypes.c_int)]),
    "hoard_moe_fused_trace_read": (_I, [_P, _P, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]),
    "hoard_moe_pool_ensure": (_I, [_P, _I, _P, _P, _P, _P, _P]),
    "hoard_moe_forward_batched": (_I, [_P, _I, _I, _P, _P, _P, _P, _P, _P]),
    "hoard_moe_forward_batched_noalloc": (_I, [_P, _I, _I, _P, _P, _P, _P, _P, _P]),
    "hoard_moe_ffn_combine_batched": (_I, [_P, _I, _I, _P, _P, _P, _P, _P, _P]),
    "hoard_moe_pool_ensure_batched": (_I, [_P, _I, _I, _P, _P, _P, _P, _P]),
    "hoard_moe_get_stats": (_I, [_P, ctypes.POINTER(MoeStats)]),
    "hoard_moe_reset_stats": (_I, [_P]),
    "hoard_gguf_open": (_I, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "hoard_gguf_close": (None, [_P]),
    "hoard_gguf_arch": (ctypes.c_char_p, [_P]),
    "hoard_gguf_moe_cfg": (_I, [_P, ctypes.POINTER(MoeCfg)]),
    "hoard_gguf_rms_eps": (ctypes.c_float, [_P]),
    "hoard_gguf_layer_weights": (_I, [_P, _I, ctypes.POINTER(LayerWeights)]),
    "hoard_gguf_tensor": (_I, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int64),
                               ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(_P)]),
    "hoard_gguf_store_layers": (_I, [_P, ctypes.POINTER(StoreLayer), _I]),
    "hoard_store_open": (_I, [ctypes.c_char_p, _I, _I, ctypes.POINTER(StoreLayer), ctypes.POINTER(StoreCfg),
                              ctypes.POINTER(_P)]),
    "hoard_store_close": (None, [_P]),
    "hoard_store_fetch": (_I, [_P, _I, _I, _P, _P, _P]),
    "hoard_store_get_stats": (_I, [_P, ctypes.POINTER(StoreStats)]),
    "hoard_store_reset_stats": (_I, [_P]),
    "hoard_moe_attach_store": (_I, [_P, _P]),
    "hoard_slot_lru_create": (_I, [_I, _I, _I, _I, ctypes.POINTER(_P)]),
    "hoard_slot_lru_access": (_I, [_P, _I, _P, _I, _P, _P]),
    "hoard_slot_lru_destroy": (None, [_P]),
    "hoard_synth_key": (ctypes.c_uint64, [ctypes.c_uint32] * 5),
    "hoard_synth_fill_blocks": (_I, [_I, ctypes.c_uint64, _P, ctypes.c_size_t, ctypes.c_float]),
    "hoard_synth_fill_normal": (None, [ctypes.c_uint64, _P, ctypes.c_size_t, ctypes.c_float]),
    "hoard_synth_fill_experts": (_I, [_I, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                      ctypes.c_uint32, _I, _I, _I, _P, ctypes.c_float]),
    "hoard_synth_expert_bytes": (ctypes.c_size_t, [_I, _I, _I]),
}

_lib = None


def load_library(path: Path | None = None) -> ctypes.CDLL:
    """Load the in-tree libhoard_moe.so; raise if it was never built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    try:
        # torch bundles its own libamdhip64 and finds it by a name that does not
        # match the one this library links; loading torch first keeps a single
        # HIP runtime in the process whichever module the caller imports first.
        import torch  # noqa: F401
    except ImportError:
        pass
    if not p.exists():
        raise HoardError(ERR_STATE, f"{p} is not built: run __graft_entry__.build() "
                                    "(or python -m hoard_amd.build) first")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in ABI.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != OK:
        raise HoardError(rc, load_library().hoard_last_error().decode())


def row_bytes(qtype: int, cols: int) -> int:
    return (cols // 256) * BLOCK_BYTES[qtype]


def expert_bytes(qtype: int, rows: int, cols: int) -> int:
    return rows * row_bytes(qtype, cols)
