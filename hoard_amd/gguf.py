"""The expert stage's weights from a GGUF file, through include/hoard_gguf.h.

    g = GGUFWeights("model.gguf")
    cfg = g.cfg()                      # hoard_moe_cfg from the file's metadata
    w = g.layer_weights(l)             # hoard_layer_weights into the mapping
    lib.hoard_moe_set_layer_weights(handle, l, ctypes.byref(w))

Counterpart of the reference's load_model (src/run_moe_stream.cpp:119-186).
"""
from __future__ import annotations

import ctypes
from pathlib import Path

from . import LayerWeights, MoeCfg, check, load_library


class GGUFWeights:
    def __init__(self, path: str | Path):
        self.lib = load_library()
        self.h = ctypes.c_void_p()
        check(self.lib.hoard_gguf_open(str(path).encode(), ctypes.byref(self.h)))

    def close(self) -> None:
        if self.h:
            self.lib.hoard_gguf_close(self.h)
            self.h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def arch(self) -> str:
        return self.lib.hoard_gguf_arch(self.h).decode()

    def cfg(self) -> MoeCfg:
        c = MoeCfg()
        check(self.lib.hoard_gguf_moe_cfg(self.h, ctypes.byref(c)))
        return c

    def rms_eps(self) -> float:
        return float(self.lib.hoard_gguf_rms_eps(self.h))

    def layer_weights(self, layer: int) -> LayerWeights:
        w = LayerWeights()
        check(self.lib.hoard_gguf_layer_weights(self.h, layer, ctypes.byref(w)))
        return w

    def shape(self):
        """The stage's shape descriptor (workloads.Shape) from the metadata and
        layer 0's tensor types; weight_set -1 marks it as not synthetic."""
        from .workloads import Shape
        c, w = self.cfg(), self.layer_weights(0)
        kw = {}
        if c.n_ff_shexp:
            kw = dict(n_ff_shexp=c.n_ff_shexp, sh_gate_type=w.sh_gate_type, sh_up_type=w.sh_up_type,
                      sh_down_type=w.sh_down_type)
        return Shape(self.arch(), -1, c.n_embd, c.n_expert, c.n_used, c.n_ff, c.renorm, w.gate_type, w.up_type,
                     w.down_type, c.n_layer, **kw)

    def tensor(self, name: str):
        """(ggml type, ne[4], bytes, address) of a tensor in the mapping."""
        t = ctypes.c_int32()
        ne = (ctypes.c_int64 * 4)()
        nb = ctypes.c_size_t()
        p = ctypes.c_void_p()
        check(self.lib.hoard_gguf_tensor(self.h, name.encode(), ctypes.byref(t), ne, ctypes.byref(nb),
                                         ctypes.byref(p)))
        return t.value, list(ne), nb.value, p.value
