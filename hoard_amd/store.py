"""The storage tier (include/hoard_store.h): expert bytes streamed from the
model file through a bounded RAM tier, by a pool of parallel readers.

    st = ExpertStore.from_gguf("model.gguf", readers=8, ram_experts=1024)
    parts, hits = st.fetch(layer, [3, 17, 40])   # addresses of gate/up/down bytes
    stage = MoEStage.from_gguf("model.gguf", pool_k=16, store=st)

Counterpart of the reference's DirectIO and RamTier (src/run_qwen35.cpp:99-148)
and its three-tier fetch (:596-638).
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

from . import StoreCfg, StoreLayer, StoreStats, check, load_library


class ExpertStore:
    def __init__(self, path: str | Path, layers, n_expert: int, readers: int = 8, ram_experts: int = 0,
                 direct: bool = True, pinned: bool = True):
        """layers: a sequence of ((gate, up, down) file offsets, (gate, up, down) strides)."""
        self.lib = load_library()
        arr = (StoreLayer * len(layers))()
        for i, (off, stride) in enumerate(layers):
            arr[i].off[:] = list(off)
            arr[i].stride[:] = list(stride)
        self.layers = [(tuple(a.off), tuple(a.stride)) for a in arr]
        self.n_layer, self.n_expert = len(layers), n_expert
        cfg = StoreCfg(readers, ram_experts, int(direct), int(pinned))
        self.h = ctypes.c_void_p()
        check(self.lib.hoard_store_open(str(path).encode(), len(layers), n_expert, arr, ctypes.byref(cfg),
                                        ctypes.byref(self.h)))

    @classmethod
    def from_gguf(cls, path: str | Path, **kw) -> "ExpertStore":
        from .gguf import GGUFWeights
        with GGUFWeights(path) as g:
            c = g.cfg()
            arr = (StoreLayer * c.n_layer)()
            check(g.lib.hoard_gguf_store_layers(g.h, arr, c.n_layer))
            layers = [(tuple(a.off), tuple(a.stride)) for a in arr]
        return cls(path, layers, c.n_expert, **kw)

    def close(self) -> None:
        if self.h:
            self.lib.hoard_store_close(self.h)
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

    def fetch(self, layer: int, ids):
        """([(gate, up, down) addresses] per id, hit flags)."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        n = ids.size
        parts = (ctypes.c_void_p * (3 * max(n, 1)))()
        hit = np.zeros(max(n, 1), dtype=np.uint8)
        check(self.lib.hoard_store_fetch(self.h, layer, n, ids.ctypes.data, parts, hit.ctypes.data))
        return [tuple(parts[3 * j + i] for i in range(3)) for j in range(n)], hit[:n].astype(bool)

    def stats(self) -> StoreStats:
        s = StoreStats()
        check(self.lib.hoard_store_get_stats(self.h, ctypes.byref(s)))
        return s

    def reset_stats(self) -> None:
        check(self.lib.hoard_store_reset_stats(self.h))
