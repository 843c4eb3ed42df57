"""Synthetic MoE-layer workloads of the shapes the stage is measured on.

Five shapes (all hidden 2048; ff = expert intermediate):
  olmoe      OLMoE-1B-7B: 64 experts, top-8, no renorm, ff 1024, all Q4_K.
  qwen3_30b  Qwen3-30B-A3B: 128 experts, top-8, renorm, ff 768, Q4_K gate/up, Q6_K down, 48 layers.
  qwen3_next Qwen3-Next-80B-A3B: 512 experts, top-10, renorm, ff 512, plus a sigmoid-gated
             shared expert (ff 512), Q4_K gate/up, Q6_K down, 48 layers.
Router weights f32 ~ N(0, 0.02); quant blocks random with fp16 d/dmin ~ |N(0, 0.01)|;
hidden x ~ N(0, 1) and fx = rms_norm(x, 1e-6).  Every byte comes from the
library's counter-based generator (include/hoard_synth.h) keyed by
(weight set, seed, layer, tensor, expert), so tests and the bench regenerate
identical layers independently.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import TYPE_Q3_K, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, LayerWeights, MoeCfg, expert_bytes, load_library

ROUTER, GATE, UP, DOWN, SH_GATE, SH_UP, SH_DOWN, SH_GATE_INP, HIDDEN = range(9)
RMS_EPS = 1e-6
DSTD = 0.01
ROUTER_STD = 0.02


@dataclass(frozen=True)
class Shape:
    name: str
    weight_set: int
    n_embd: int
    n_expert: int
    n_used: int
    n_ff: int
    renorm: int
    gate_type: int
    up_type: int
    down_type: int
    n_layer: int
    n_ff_shexp: int = 0
    sh_gate_type: int = TYPE_Q4_K
    sh_up_type: int = TYPE_Q4_K
    sh_down_type: int = TYPE_Q6_K

    def cfg(self, n_layer: int | None = None, pool_k: int = 0, max_tokens: int = 1) -> MoeCfg:
        return MoeCfg(self.n_embd, self.n_expert, self.n_used, self.n_ff, self.n_ff_shexp,
                      n_layer or self.n_layer, self.renorm, pool_k, max_tokens)

    def expert_bytes(self) -> int:
        return (expert_bytes(self.gate_type, self.n_ff, self.n_embd)
                + expert_bytes(self.up_type, self.n_ff, self.n_embd)
                + expert_bytes(self.down_type, self.n_embd, self.n_ff))

    def shared_bytes(self) -> int:
        if not self.n_ff_shexp:
            return 0
        return (expert_bytes(self.sh_gate_type, self.n_ff_shexp, self.n_embd)
                + expert_bytes(self.sh_up_type, self.n_ff_shexp, self.n_embd)
                + expert_bytes(self.sh_down_type, self.n_embd, self.n_ff_shexp)
                + 4 * self.n_embd)

    def bytes_per_token_layer(self, unique_experts: int | None = None, tokens: int = 1) -> int:
        """Algorithmic HBM bytes: selected experts once, shared expert, router W, x in and out."""
        u = self.n_used if unique_experts is None else unique_experts
        return (u * self.expert_bytes() + self.shared_bytes() + 4 * self.n_expert * self.n_embd
                + tokens * 2 * 4 * self.n_embd)

    def flops_per_token_layer(self) -> int:
        routed = self.n_used * 2 * 3 * self.n_ff * self.n_embd
        shared = 2 * 3 * self.n_ff_shexp * self.n_embd if self.n_ff_shexp else 0
        return routed + shared + 2 * self.n_expert * self.n_embd


OLMOE = Shape("olmoe", 0, 2048, 64, 8, 1024, 0, TYPE_Q4_K, TYPE_Q4_K, TYPE_Q4_K, 1)
QWEN3_30B = Shape("qwen3_30b", 1, 2048, 128, 8, 768, 1, TYPE_Q4_K, TYPE_Q4_K, TYPE_Q6_K, 48)
QWEN3_NEXT = Shape("qwen3_next", 2, 2048, 512, 10, 512, 1, TYPE_Q4_K, TYPE_Q4_K, TYPE_Q6_K, 48,
                   n_ff_shexp=512)
# Q5_K down experts: Qwen3.5-35B-A3B (qwen35moe; n_ff 512, 8 of 256 experts, 40 layers,
# a 512-wide shared expert), and OLMoE in its Q3_K_M form (Q3_K gate/up, Q5_K down);
# types and expert sizes as listed in the reference's notes/FEASIBILITY.md:75,77.
QWEN35 = Shape("qwen35", 3, 2048, 256, 8, 512, 1, TYPE_Q4_K, TYPE_Q4_K, TYPE_Q5_K, 40, n_ff_shexp=512)
OLMOE_Q3 = Shape("olmoe_q3", 4, 2048, 64, 8, 1024, 0, TYPE_Q3_K, TYPE_Q3_K, TYPE_Q5_K, 16)
SHAPES = {s.name: s for s in (OLMOE, QWEN3_30B, QWEN3_NEXT, QWEN35, OLMOE_Q3)}


@dataclass
class HostLayer:
    """One layer's weights in host memory, GGUF layout."""
    shape: Shape
    router: np.ndarray
    gate: np.ndarray
    up: np.ndarray
    down: np.ndarray
    sh_gate: np.ndarray | None = None
    sh_up: np.ndarray | None = None
    sh_down: np.ndarray | None = None
    sh_gate_inp: np.ndarray | None = None

    def weights(self) -> LayerWeights:
        s = self.shape
        p = lambda a: a.ctypes.data if a is not None else None  # noqa: E731
        return LayerWeights(p(self.router), s.gate_type, s.up_type, s.down_type,
                            p(self.gate), p(self.up), p(self.down),
                            s.sh_gate_type, s.sh_up_type, s.sh_down_type,
                            p(self.sh_gate), p(self.sh_up), p(self.sh_down), p(self.sh_gate_inp))

    def stride(self, which: str) -> int:
        s = self.shape
        return {"gate": expert_bytes(s.gate_type, s.n_ff, s.n_embd),
                "up": expert_bytes(s.up_type, s.n_ff, s.n_embd),
                "down": expert_bytes(s.down_type, s.n_embd, s.n_ff)}[which]


def _experts(lib, qtype, shape, seed, layer, tensor, rows, cols):
    buf = np.empty(shape.n_expert * expert_bytes(qtype, rows, cols), dtype=np.uint8)
    rc = lib.hoard_synth_fill_experts(qtype, shape.weight_set, seed, layer, tensor, shape.n_expert,
                                      rows, cols, buf.ctypes.data, DSTD)
    assert rc == 0
    return buf


def _single(lib, qtype, shape, seed, layer, tensor, rows, cols):
    buf = np.empty(expert_bytes(qtype, rows, cols), dtype=np.uint8)
    key = lib.hoard_synth_key(shape.weight_set, seed, layer, tensor, 0)
    rc = lib.hoard_synth_fill_blocks(qtype, key, buf.ctypes.data, rows * (cols // 256), DSTD)
    assert rc == 0
    return buf


def normal(key: int, n: int, std: float) -> np.ndarray:
    lib = load_library()
    out = np.empty(n, dtype=np.float32)
    lib.hoard_synth_fill_normal(key, out.ctypes.data, n, std)
    return out


def _some_experts(lib, qtype, shape, seed, layer, tensor, rows, cols, experts):
    """Full-size tensor with only `experts` generated (the rest zero)."""
    stride = expert_bytes(qtype, rows, cols)
    buf = np.zeros(shape.n_expert * stride, dtype=np.uint8)
    for e in experts:
        key = lib.hoard_synth_key(shape.weight_set, seed, layer, tensor, int(e))
        rc = lib.hoard_synth_fill_blocks(qtype, key, buf[e * stride:].ctypes.data, rows * (cols // 256), DSTD)
        assert rc == 0
    return buf


def make_router(shape: Shape, seed: int, layer: int) -> np.ndarray:
    lib = load_library()
    return normal(lib.hoard_synth_key(shape.weight_set, seed, layer, ROUTER, 0),
                  shape.n_expert * shape.n_embd, ROUTER_STD)


def make_layer(shape: Shape, seed: int, layer: int, experts=None) -> HostLayer:
    """One synthetic layer; with `experts`, only those experts are generated
    (byte-identical to the full layer there) and the others are left zero."""
    lib = load_library()
    ws = shape.weight_set
    router = make_router(shape, seed, layer)
    if experts is None:
        gen = lambda q, t, r, c: _experts(lib, q, shape, seed, layer, t, r, c)  # noqa: E731
    else:
        gen = lambda q, t, r, c: _some_experts(lib, q, shape, seed, layer, t, r, c, experts)  # noqa: E731
    hl = HostLayer(
        shape, router,
        gen(shape.gate_type, GATE, shape.n_ff, shape.n_embd),
        gen(shape.up_type, UP, shape.n_ff, shape.n_embd),
        gen(shape.down_type, DOWN, shape.n_embd, shape.n_ff))
    if shape.n_ff_shexp:
        f = shape.n_ff_shexp
        hl.sh_gate = _single(lib, shape.sh_gate_type, shape, seed, layer, SH_GATE, f, shape.n_embd)
        hl.sh_up = _single(lib, shape.sh_up_type, shape, seed, layer, SH_UP, f, shape.n_embd)
        hl.sh_down = _single(lib, shape.sh_down_type, shape, seed, layer, SH_DOWN, shape.n_embd, f)
        hl.sh_gate_inp = normal(lib.hoard_synth_key(ws, seed, layer, SH_GATE_INP, 0), shape.n_embd,
                                ROUTER_STD)
    return hl


def fill_layer(hl: HostLayer, seed: int, layer: int) -> HostLayer:
    """Regenerate another layer into hl's existing buffers (no new host pages)."""
    lib = load_library()
    s, ws = hl.shape, hl.shape.weight_set
    lib.hoard_synth_fill_normal(lib.hoard_synth_key(ws, seed, layer, ROUTER, 0), hl.router.ctypes.data,
                                hl.router.size, ROUTER_STD)
    for buf, q, t, r, c in ((hl.gate, s.gate_type, GATE, s.n_ff, s.n_embd),
                            (hl.up, s.up_type, UP, s.n_ff, s.n_embd),
                            (hl.down, s.down_type, DOWN, s.n_embd, s.n_ff)):
        assert lib.hoard_synth_fill_experts(q, ws, seed, layer, t, s.n_expert, r, c, buf.ctypes.data, DSTD) == 0
    if s.n_ff_shexp:
        f = s.n_ff_shexp
        for buf, q, t, r, c in ((hl.sh_gate, s.sh_gate_type, SH_GATE, f, s.n_embd),
                                (hl.sh_up, s.sh_up_type, SH_UP, f, s.n_embd),
                                (hl.sh_down, s.sh_down_type, SH_DOWN, s.n_embd, f)):
            key = lib.hoard_synth_key(ws, seed, layer, t, 0)
            assert lib.hoard_synth_fill_blocks(q, key, buf.ctypes.data, r * (c // 256), DSTD) == 0
        lib.hoard_synth_fill_normal(lib.hoard_synth_key(ws, seed, layer, SH_GATE_INP, 0),
                                    hl.sh_gate_inp.ctypes.data, s.n_embd, ROUTER_STD)
    return hl


def rms_norm(x: np.ndarray, eps: float = RMS_EPS) -> np.ndarray:
    """ggml_rms_norm: mean of x*x accumulated in double, scale = 1/sqrtf(mean + eps)."""
    x = np.asarray(x, dtype=np.float32)
    sq = (x * x).astype(np.float64)
    mean = np.float32(np.sum(sq) / x.size)
    scale = np.float32(1.0) / np.sqrt(np.float32(mean + np.float32(eps)), dtype=np.float32)
    return (x * scale).astype(np.float32)


def make_hidden(shape: Shape, seed: int, layer: int, token: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """(fx, res): res ~ N(0, 1), fx = rms_norm(res)."""
    lib = load_library()
    res = normal(lib.hoard_synth_key(shape.weight_set, seed, layer, HIDDEN, token), shape.n_embd, 1.0)
    return rms_norm(res), res


def as_ptr(a: np.ndarray) -> ctypes.c_void_p:
    return ctypes.c_void_p(a.ctypes.data)


@dataclass
class RoutingTrace:
    """Per (token, layer): the n_used selected experts and their weights."""
    sel: np.ndarray  # int32 [tokens, n_layer, n_used]
    w: np.ndarray    # float32 [tokens, n_layer, n_used], each row sums to 1


def routing_trace(shape: Shape, seed: int, tokens: int = 512, n_layer: int | None = None,
                  zipf_s: float = 0.8, reuse_p: float = 0.4, window: int = 4) -> RoutingTrace:
    """Seeded synthetic routing for the slot-pool workload: per layer, expert
    popularity follows Zipf(zipf_s) over a random ranking of the experts; each
    of a token's picks instead reuses, with probability reuse_p, an expert the
    same layer selected in the previous `window` tokens.  Picks are distinct
    within a token.  Weights are normalised Exp(1) draws."""
    n_layer = n_layer or shape.n_layer
    E, k = shape.n_expert, shape.n_used
    rng = np.random.Generator(np.random.PCG64(0x7A1F0000 + seed))
    ranks = [rng.permutation(E) for _ in range(n_layer)]
    p = 1.0 / np.arange(1, E + 1, dtype=np.float64) ** zipf_s
    cdf = np.cumsum(p / p.sum())
    sel = np.zeros((tokens, n_layer, k), dtype=np.int32)
    for t in range(tokens):
        for layer in range(n_layer):
            recent = sorted(set(sel[max(0, t - window):t, layer].ravel().tolist())) if t else []
            picked: list[int] = []
            while len(picked) < k:
                pool = [e for e in recent if e not in picked]
                if pool and rng.random() < reuse_p:
                    e = pool[int(rng.integers(len(pool)))]
                else:
                    e = int(ranks[layer][min(int(np.searchsorted(cdf, rng.random(), side="right")), E - 1)])
                    if e in picked:
                        continue
                picked.append(e)
            sel[t, layer] = picked
    w = rng.exponential(1.0, size=(tokens, n_layer, k)).astype(np.float32)
    w /= w.sum(axis=2, keepdims=True)
    return RoutingTrace(sel, w.astype(np.float32))
