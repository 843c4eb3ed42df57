"""Python handle over the C ABI, with torch providing device memory and streams.

torch is plumbing here: it allocates the activation buffers the ABI reads and
writes and hands over its current HIP stream.  Every computation is a call
into libhoard_moe.so.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import check, load_library


def _torch():
    import torch  # deferred: the CPU-only tests never need a device
    return torch


class MoEStage:
    """One hoard_moe handle.  layers: {layer index: workloads.HostLayer}."""

    def __init__(self, shape, n_layer: int | None = None, layers=None, pool_k: int = 0,
                 max_tokens: int = 1):
        torch = _torch()
        if not torch.cuda.is_available():
            raise RuntimeError("MoEStage needs a HIP device")
        self.lib = load_library()
        self.shape = shape
        self.cfg = shape.cfg(n_layer, pool_k, max_tokens)
        self.h = ctypes.c_void_p()
        torch.cuda.init()
        check(self.lib.hoard_moe_create(ctypes.byref(self.cfg), ctypes.byref(self.h)))
        for li, hl in (layers or {}).items():
            self.set_layer(li, hl)

    @classmethod
    def from_gguf(cls, path, layers=None, pool_k: int = 0, max_tokens: int = 1, store=None) -> "MoEStage":
        """A stage holding the expert stage of every layer in `layers` (default:
        all) of a GGUF file.  The weights are copied in, so the file is closed
        before this returns.  With `store` (a hoard_amd.store.ExpertStore over
        the same file) and pool_k > 0, slot misses stream from the store instead
        of a pinned copy of every expert; the store must outlive the stage."""
        from .gguf import GGUFWeights
        with GGUFWeights(path) as g:
            shape = g.shape()
            st = cls(shape, pool_k=pool_k, max_tokens=max_tokens)
            try:
                if store is not None:
                    check(st.lib.hoard_moe_attach_store(st.h, store.h))
                    st.store = store
                for l in range(shape.n_layer) if layers is None else layers:
                    w = g.layer_weights(l)
                    check(st.lib.hoard_moe_set_layer_weights(st.h, l, ctypes.byref(w)))
            except Exception:
                st.close()
                raise
            st.rms_eps = g.rms_eps()
        return st

    def close(self):
        if self.h:
            self.lib.hoard_moe_destroy(self.h)
            self.h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_layer(self, layer: int, hl) -> None:
        w = hl.weights()
        check(self.lib.hoard_moe_set_layer_weights(self.h, layer, ctypes.byref(w)))

    # -- device helpers ------------------------------------------------------
    @staticmethod
    def stream():
        return ctypes.c_void_p(_torch().cuda.current_stream().cuda_stream)

    @staticmethod
    def dev(a, dtype=None):
        torch = _torch()
        t = torch.as_tensor(np.ascontiguousarray(a))
        if dtype is not None:
            t = t.to(dtype)
        return t.to("cuda")

    @staticmethod
    def ptr(t):
        return ctypes.c_void_p(t.data_ptr())

    # -- ABI calls (numpy in, numpy out; synchronous) ------------------------
    def route(self, layer: int, fx: np.ndarray):
        torch = _torch()
        s = self.shape
        fx_d = self.dev(fx)
        sel = torch.empty(s.n_used, dtype=torch.int32, device="cuda")
        w = torch.empty(s.n_used, dtype=torch.float32, device="cuda")
        check(self.lib.hoard_moe_route(self.h, layer, self.ptr(fx_d), self.ptr(sel), self.ptr(w), self.stream()))
        torch.cuda.synchronize()
        return sel.cpu().numpy(), w.cpu().numpy()

    def ffn_combine(self, layer: int, fx, ids, w, res):
        torch = _torch()
        fx_d, ids_d, w_d, res_d = self.dev(fx), self.dev(ids, torch.int32), self.dev(w), self.dev(res)
        out = torch.empty_like(res_d)
        check(self.lib.hoard_moe_ffn_combine(self.h, layer, self.ptr(fx_d), self.ptr(ids_d), self.ptr(w_d),
                                             self.ptr(res_d), self.ptr(out), self.stream()))
        torch.cuda.synchronize()
        return out.cpu().numpy()

    def layer(self, layer: int, fx, res):
        torch = _torch()
        s = self.shape
        fx_d, res_d = self.dev(fx), self.dev(res)
        out = torch.empty_like(res_d)
        sel = torch.empty(s.n_used, dtype=torch.int32, device="cuda")
        w = torch.empty(s.n_used, dtype=torch.float32, device="cuda")
        check(self.lib.hoard_moe_layer(self.h, layer, self.ptr(fx_d), self.ptr(res_d), self.ptr(out),
                                       self.ptr(sel), self.ptr(w), self.stream()))
        torch.cuda.synchronize()
        return out.cpu().numpy(), sel.cpu().numpy(), w.cpu().numpy()

    def forward_batched(self, layer: int, fx, res):
        """M tokens at once: fx, res [M][n_embd] -> out [M][n_embd], sel, w [M][n_used]."""
        torch = _torch()
        fx_d, res_d = self.dev(fx), self.dev(res)
        M = fx_d.shape[0]
        out = torch.empty_like(res_d)
        sel = torch.empty((M, self.shape.n_used), dtype=torch.int32, device="cuda")
        w = torch.empty((M, self.shape.n_used), dtype=torch.float32, device="cuda")
        check(self.lib.hoard_moe_forward_batched(self.h, layer, M, self.ptr(fx_d), self.ptr(res_d), self.ptr(out),
                                                 self.ptr(sel), self.ptr(w), self.stream()))
        torch.cuda.synchronize()
        return out.cpu().numpy(), sel.cpu().numpy(), w.cpu().numpy()

    def ffn_combine_batched(self, layer: int, fx, ids, w, res):
        """Caller's selection for M tokens: fx, res [M][n_embd]; ids, w [M][n_used]."""
        torch = _torch()
        fx_d, res_d = self.dev(fx), self.dev(res)
        ids_d, w_d = self.dev(ids, torch.int32), self.dev(w)
        out = torch.empty_like(res_d)
        check(self.lib.hoard_moe_ffn_combine_batched(self.h, layer, fx_d.shape[0], self.ptr(fx_d), self.ptr(ids_d),
                                                     self.ptr(w_d), self.ptr(res_d), self.ptr(out), self.stream()))
        torch.cuda.synchronize()
        return out.cpu().numpy()

    def pool_ensure_batched(self, layer: int, sel):
        """Slots for the ids sel (token-major), taken one after the other."""
        sel_h = np.ascontiguousarray(np.ravel(sel), dtype=np.int32)
        slots_h = np.zeros(sel_h.size, dtype=np.int32)
        check(self.lib.hoard_moe_pool_ensure_batched(self.h, layer, sel_h.size, sel_h.ctypes.data,
                                                     slots_h.ctypes.data, None, self.stream(), None))
        return slots_h.reshape(np.shape(sel))

    def pool_ensure(self, layer: int, sel, copy_stream=None):
        """Makes the experts sel resident in this layer's slots; returns the slots
        (host) and a device tensor holding them, ordered on the current stream."""
        torch = _torch()
        sel_h = np.ascontiguousarray(sel, dtype=np.int32)
        slots_h = np.zeros(self.shape.n_used, dtype=np.int32)
        slots_d = torch.empty(self.shape.n_used, dtype=torch.int32, device="cuda")
        cs = ctypes.c_void_p(copy_stream.cuda_stream) if copy_stream is not None else None
        check(self.lib.hoard_moe_pool_ensure(self.h, layer, sel_h.ctypes.data, slots_h.ctypes.data,
                                             self.ptr(slots_d), self.stream(), cs))
        return slots_h, slots_d

    def ffn_combine_dev(self, layer: int, fx_d, ids_d, w_d, res_d, out_d) -> None:
        """hoard_moe_ffn_combine on device tensors, asynchronous on the current stream."""
        check(self.lib.hoard_moe_ffn_combine(self.h, layer, self.ptr(fx_d), self.ptr(ids_d), self.ptr(w_d),
                                             self.ptr(res_d), self.ptr(out_d), self.stream()))

    def stats(self):
        from . import MoeStats
        st = MoeStats()
        check(self.lib.hoard_moe_get_stats(self.h, ctypes.byref(st)))
        return st

    def reset_stats(self) -> None:
        check(self.lib.hoard_moe_reset_stats(self.h))

    def set_option(self, option: int, value: int) -> None:
        check(self.lib.hoard_moe_set_option(self.h, option, value))

    def get_option(self, option: int) -> int:
        v = ctypes.c_int()
        check(self.lib.hoard_moe_get_option(self.h, option, ctypes.byref(v)))
        return v.value

    def sync_check(self) -> None:
        check(self.lib.hoard_moe_sync_check(self.h))

    def decode(self, x, layer_begin: int, layer_end: int, eps: float):
        torch = _torch()
        x_d = self.dev(x)
        check(self.lib.hoard_moe_decode(self.h, layer_begin, layer_end, self.ptr(x_d), ctypes.c_float(eps),
                                        self.stream()))
        torch.cuda.synchronize()
        return x_d.cpu().numpy()
