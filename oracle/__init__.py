"""ctypes bindings for the CPU oracle (libmoe_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline.  The
product (hoard_amd/) never imports it.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libmoe_oracle.so"

TYPE_Q3_K = 11
TYPE_Q4_K = 12
TYPE_Q5_K = 13
TYPE_Q6_K = 14
BLOCK_BYTES = {TYPE_Q3_K: 110, TYPE_Q4_K: 144, TYPE_Q5_K: 176, TYPE_Q6_K: 210}
Q8K_DTYPE = np.dtype([("d", "<f4"), ("qs", "i1", 256), ("bsums", "<i2", 16)])
assert Q8K_DTYPE.itemsize == 292


class LayerCfg(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in (
        "n_embd", "n_expert", "n_used", "n_ff", "n_ff_shexp", "renorm",
        "gate_type", "up_type", "down_type", "sh_gate_type", "sh_up_type", "sh_down_type")]


class LayerW(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "router", "gate", "up", "down", "sh_gate", "sh_up", "sh_down", "sh_gate_inp")]


_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_SIGS = {
    "orc_fp16_to_fp32": (_F, [ctypes.c_uint16]),
    "orc_fp32_to_fp16": (ctypes.c_uint16, [_F]),
    "orc_nearest_int": (_I, [_F]),
    "orc_dequant_q4_K": (None, [_P, _P]),
    "orc_dequant_q6_K": (None, [_P, _P]),
    "orc_dequant_q3_K": (None, [_P, _P]),
    "orc_dequant_q5_K": (None, [_P, _P]),
    "orc_dequant_row": (None, [_I, _P, _I, _P]),
    "orc_quantize_q8_K": (None, [_P, _I, _P]),
    "orc_sizeof_q8_K": (ctypes.c_size_t, []),
    "orc_vec_dot_f32": (_F, [_I, _P, _P]),
    "orc_vec_dot_q4_K_q8_K": (_F, [_I, _P, _P]),
    "orc_vec_dot_q6_K_q8_K": (_F, [_I, _P, _P]),
    "orc_vec_dot_q3_K_q8_K": (_F, [_I, _P, _P]),
    "orc_vec_dot_q5_K_q8_K": (_F, [_I, _P, _P]),
    "orc_vec_dot_q_q8_K": (_F, [_I, _I, _P, _P]),
    "orc_mul_mat_q": (None, [_I, _P, _I, _I, _P, _P]),
    "orc_mul_mat_q8": (None, [_I, _P, _I, _I, _P, _P]),
    "orc_silu": (_F, [_F]),
    "orc_sigmoid": (_F, [_F]),
    "orc_route": (None, [_I, _I, _I, _I, _P, _P, _P, _P, _P]),
    "orc_expert_ffn": (None, [_I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P]),
    "orc_moe_layer": (None, [ctypes.POINTER(LayerCfg), ctypes.POINTER(LayerW), _P, _P, _P, _P, _P]),
    "orc_moe_ffn_combine": (None, [ctypes.POINTER(LayerCfg), ctypes.POINTER(LayerW), _P, _P, _P, _P, _P]),
    "orc_moe_layer_batched": (None, [ctypes.POINTER(LayerCfg), ctypes.POINTER(LayerW), _I, _P, _P, _P,
                                     _P, _P]),
    "orc_rms_norm": (None, [_I, _P, _F, _P]),
    "orc_num_threads": (_I, []),
    "orc_set_num_threads": (None, [_I]),
}

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        l_ = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(l_, name)
            fn.restype, fn.argtypes = res, args
        _lib = l_
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


def fp16_to_fp32(h: int) -> float:
    return lib().orc_fp16_to_fp32(h)


def fp32_to_fp16(f: float) -> int:
    return lib().orc_fp32_to_fp16(f)


def nearest_int(f: float) -> int:
    return lib().orc_nearest_int(f)


def dequant(qtype: int, data: np.ndarray, n: int) -> np.ndarray:
    data = _u8(data)
    out = np.empty(n, dtype=np.float32)
    lib().orc_dequant_row(qtype, _p(data), n, _p(out))
    return out


def quantize_q8k(x: np.ndarray) -> np.ndarray:
    x = _f32(x)
    out = np.zeros(x.size // 256, dtype=Q8K_DTYPE)
    lib().orc_quantize_q8_K(_p(x), x.size, _p(out))
    return out


def dequant_q8k(q: np.ndarray) -> np.ndarray:
    return (q["qs"].astype(np.float64) * q["d"].astype(np.float64)[:, None]).reshape(-1)


def vec_dot_f32(x: np.ndarray, y: np.ndarray) -> float:
    x, y = _f32(x), _f32(y)
    return lib().orc_vec_dot_f32(x.size, _p(x), _p(y))


def vec_dot_q(qtype: int, row: np.ndarray, q8: np.ndarray) -> float:
    row = _u8(row)
    return lib().orc_vec_dot_q_q8_K(qtype, q8.size * 256, _p(row), _p(q8))


def mul_mat_q(qtype: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    w, x = _u8(w), _f32(x)
    out = np.empty(rows, dtype=np.float32)
    lib().orc_mul_mat_q(qtype, _p(w), rows, cols, _p(x), _p(out))
    return out


def silu(x: float) -> float:
    return lib().orc_silu(x)


def sigmoid(x: float) -> float:
    return lib().orc_sigmoid(x)


def route(w_router: np.ndarray, fx: np.ndarray, n_expert: int, n_used: int, renorm: int):
    w_router, fx = _f32(w_router), _f32(fx)
    sel = np.empty(n_used, dtype=np.int32)
    wsel = np.empty(n_used, dtype=np.float32)
    probs = np.empty(n_expert, dtype=np.float32)
    lib().orc_route(fx.size, n_expert, n_used, renorm, _p(w_router), _p(fx), _p(sel), _p(wsel), _p(probs))
    return sel, wsel, probs


def rms_norm(x: np.ndarray, eps: float) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    lib().orc_rms_norm(x.size, _p(x), eps, _p(out))
    return out


def layer_cfg(shape) -> LayerCfg:
    return LayerCfg(shape.n_embd, shape.n_expert, shape.n_used, shape.n_ff, shape.n_ff_shexp,
                    shape.renorm, shape.gate_type, shape.up_type, shape.down_type,
                    shape.sh_gate_type, shape.sh_up_type, shape.sh_down_type)


def layer_w(hl) -> LayerW:
    return LayerW(_p(hl.router), _p(hl.gate), _p(hl.up), _p(hl.down), _p(hl.sh_gate),
                  _p(hl.sh_up), _p(hl.sh_down), _p(hl.sh_gate_inp))


def moe_layer(hl, fx: np.ndarray, res: np.ndarray):
    """Full stage for one token on a host layer (hoard_amd.workloads.HostLayer)."""
    s = hl.shape
    fx, res = _f32(fx), _f32(res)
    out = np.empty(s.n_embd, dtype=np.float32)
    sel = np.empty(s.n_used, dtype=np.int32)
    wsel = np.empty(s.n_used, dtype=np.float32)
    cfg, w = layer_cfg(s), layer_w(hl)
    lib().orc_moe_layer(ctypes.byref(cfg), ctypes.byref(w), _p(fx), _p(res), _p(out), _p(sel), _p(wsel))
    return out, sel, wsel


def moe_ffn_combine(hl, fx: np.ndarray, sel: np.ndarray, wsel: np.ndarray, res: np.ndarray):
    s = hl.shape
    fx, res, wsel = _f32(fx), _f32(res), _f32(wsel)
    sel = np.ascontiguousarray(sel, dtype=np.int32)
    out = np.empty(s.n_embd, dtype=np.float32)
    cfg, w = layer_cfg(s), layer_w(hl)
    lib().orc_moe_ffn_combine(ctypes.byref(cfg), ctypes.byref(w), _p(fx), _p(sel), _p(wsel), _p(res), _p(out))
    return out


def moe_layer_batched(hl, fx: np.ndarray, res: np.ndarray):
    s = hl.shape
    fx, res = _f32(fx), _f32(res)
    m = fx.shape[0]
    out = np.empty((m, s.n_embd), dtype=np.float32)
    sel = np.empty((m, s.n_used), dtype=np.int32)
    wsel = np.empty((m, s.n_used), dtype=np.float32)
    cfg, w = layer_cfg(s), layer_w(hl)
    lib().orc_moe_layer_batched(ctypes.byref(cfg), ctypes.byref(w), m, _p(fx), _p(res), _p(out), _p(sel),
                                _p(wsel))
    return out, sel, wsel


def expert_ffn(n_embd, n_ff, gate_type, up_type, down_type, gate, up, down, fx):
    """One expert: returns (y[n_embd], h[n_ff])."""
    q8 = quantize_q8k(fx)
    y = np.empty(n_embd, dtype=np.float32)
    h = np.empty(n_ff, dtype=np.float32)
    gate, up, down = _u8(gate), _u8(up), _u8(down)
    lib().orc_expert_ffn(n_embd, n_ff, gate_type, up_type, down_type, _p(gate), _p(up), _p(down), _p(q8),
                         _p(y), _p(h))
    return y, h
