"""The resident paths under HIP graph capture: hoard_moe_layer, the
per-layer decode and the batched forward (kernel launches only: no copies,
memsets or allocations once the handle is set up and each entry point has run
once) captured into a graph, replayed
several times with the program's own eager work and synchronisations between
replays, each replay bit-identical to the eager launches, and the eager result
at the parity bar against the oracle."""
import ctypes

import numpy as np
import pytest

import hoard_amd as H
import parity
from hoard_amd import workloads as W

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

N_LAYER = 2
REPLAYS = 4
M = 16


@pytest.fixture(scope="module")
def stage():
    from hoard_amd.runtime import MoEStage
    shape = W.QWEN3_30B
    layers = {l: W.make_layer(shape, 11, l) for l in range(N_LAYER)}
    st = MoEStage(shape, n_layer=N_LAYER, layers=layers, max_tokens=M)
    st.set_option(H.OPT_PERSISTENT_DECODE, 0)
    yield shape, layers, st
    st.close()


def _replays_match(g, reset, outputs, eager, what):
    for r in range(REPLAYS):
        reset()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outputs, eager):
            assert torch.equal(o.view(torch.int32), e.view(torch.int32)), (what, r)
        # eager work of the program's own between replays
        torch.empty(1 << 16, device="cuda").normal_().sum().item()


def test_layer_chain_captured(orc, stage):
    shape, layers, st = stage
    D, k = shape.n_embd, shape.n_used
    fx, res = W.make_hidden(shape, 11, 0, 0)
    fx_d, res_d = st.dev(fx), st.dev(res)
    out = [torch.empty(D, device="cuda") for _ in range(N_LAYER)]
    sel = [torch.empty(k, dtype=torch.int32, device="cuda") for _ in range(N_LAYER)]
    w = [torch.empty(k, device="cuda") for _ in range(N_LAYER)]
    s = torch.cuda.Stream()

    def chain():  # layer l takes layer l-1's output as its normed input and residual
        sp = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for l in range(N_LAYER):
            a = fx_d if l == 0 else out[l - 1]
            r = res_d if l == 0 else out[l - 1]
            H.check(st.lib.hoard_moe_layer(st.h, l, st.ptr(a), st.ptr(r), st.ptr(out[l]), st.ptr(sel[l]),
                                           st.ptr(w[l]), sp))

    print("graph: eager layer chain", flush=True)
    with torch.cuda.stream(s):
        chain()
    torch.cuda.synchronize()
    eager = [t.clone() for t in out + sel + w]
    # the eager result against the oracle
    x_h, r_h = fx, res
    for l in range(N_LAYER):
        ref, sel_o, _ = orc.moe_layer(layers[l], x_h, r_h)
        assert np.array_equal(sel[l].cpu().numpy(), sel_o), l
        parity.assert_parity(out[l].cpu().numpy(), ref, f"layer chain {l}")
        x_h = r_h = out[l].cpu().numpy()
    print("graph: capture and replay", flush=True)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        chain()
    torch.cuda.synchronize()

    def reset():
        for t in out + w:
            t.fill_(float("nan"))
        for t in sel:
            t.fill_(-1)

    _replays_match(g, reset, out + sel + w, eager, "layer chain")


def test_decode_captured(orc, stage):
    shape, layers, st = stage
    _, x = W.make_hidden(shape, 11, 0, 1)
    x0 = st.dev(x)
    xd = x0.clone()
    s = torch.cuda.Stream()

    def step():
        H.check(st.lib.hoard_moe_decode(st.h, 0, N_LAYER, st.ptr(xd), ctypes.c_float(W.RMS_EPS),
                                        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))

    print("graph: eager per-layer decode", flush=True)
    with torch.cuda.stream(s):
        step()
    torch.cuda.synchronize()
    st.sync_check()
    eager = xd.clone()
    ref = x
    for l in range(N_LAYER):
        ref, _, _ = orc.moe_layer(layers[l], orc.rms_norm(ref, W.RMS_EPS), ref)
    parity.assert_parity(eager.cpu().numpy(), ref, "per-layer decode")
    print("graph: capture and replay decode", flush=True)
    xd.copy_(x0)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step()
    torch.cuda.synchronize()
    _replays_match(g, lambda: xd.copy_(x0), [xd], [eager], "decode")
    st.sync_check()


def test_batched_forward_captured(orc, stage):
    shape, layers, st = stage
    D, k = shape.n_embd, shape.n_used
    toks = [W.make_hidden(shape, 11, 1, 20 + t) for t in range(M)]
    fx_d = st.dev(np.stack([f for f, _ in toks]))
    res_d = st.dev(np.stack([r for _, r in toks]))
    out = torch.empty(M, D, device="cuda")
    sel = torch.empty(M, k, dtype=torch.int32, device="cuda")
    w = torch.empty(M, k, device="cuda")
    s = torch.cuda.Stream()

    def step():
        H.check(st.lib.hoard_moe_forward_batched(st.h, 1, M, st.ptr(fx_d), st.ptr(res_d), st.ptr(out), st.ptr(sel),
                                                 st.ptr(w), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)))

    print(f"graph: eager batched forward, M={M}", flush=True)
    with torch.cuda.stream(s):
        step()
    torch.cuda.synchronize()
    eager = [out.clone(), sel.clone(), w.clone()]
    for t, (fx, res) in enumerate(toks):
        ref, sel_o, _ = orc.moe_layer(layers[1], fx, res)
        assert np.array_equal(sel[t].cpu().numpy(), sel_o), t
        parity.assert_parity(out[t].cpu().numpy(), ref, f"batched token {t}")
    print("graph: capture and replay batched forward", flush=True)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step()
    torch.cuda.synchronize()

    def reset():
        out.fill_(float("nan"))
        w.fill_(float("nan"))
        sel.fill_(-1)

    _replays_match(g, reset, [out, sel, w], eager, "batched forward")


@pytest.mark.parametrize("kernel", [1, 2], ids=["xcd", "spread"])
def test_one_launch_decode_plain_launch_captured(orc, kernel):
    """The one-launch decode as a plain launch under capture: its sequence tags
    live in device memory, so every replay (with eager decodes on the same handle
    in between, which move the same tags) gives the eager bits.  Under capture
    with the cooperative launch, automatic mode records the per-layer kernels and
    forced mode refuses before launching anything."""
    from hoard_amd.runtime import MoEStage
    shape = W.QWEN3_30B
    nl = 4
    layers = {l: W.make_layer(shape, 12, l) for l in range(nl)}
    st = MoEStage(shape, n_layer=nl, layers=layers)
    try:
        st.set_option(H.OPT_DECODE_KERNEL, kernel)
        st.set_option(H.OPT_PERSISTENT_DECODE, 2)
        st.set_option(H.OPT_DECODE_LAUNCH, 1)
        _, x = W.make_hidden(shape, 12, 0, 0)
        x0 = st.dev(x)
        xd = x0.clone()
        other = st.dev(W.make_hidden(shape, 12, 0, 1)[1])
        s = torch.cuda.Stream()

        def decode(buf):
            return st.lib.hoard_moe_decode(st.h, 0, nl, st.ptr(buf), ctypes.c_float(W.RMS_EPS),
                                           ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))

        print(f"graph: eager one-launch decode, kernel {kernel}", flush=True)
        with torch.cuda.stream(s):
            H.check(decode(xd))
        torch.cuda.synchronize()
        st.sync_check()
        eager = xd.clone()
        ref = x
        for l in range(nl):
            ref, _, _ = orc.moe_layer(layers[l], orc.rms_norm(ref, W.RMS_EPS), ref)
        parity.assert_parity(eager.cpu().numpy(), ref, "one-launch decode")
        print("graph: capture and replay the plain launch", flush=True)
        xd.copy_(x0)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            H.check(decode(xd))
        torch.cuda.synchronize()

        def reset():
            xd.copy_(x0)
            o = other.clone()
            H.check(decode(o))  # an eager launch between replays moves the device tags too

        _replays_match(g, reset, [xd], [eager], "plain one-launch decode")
        st.sync_check()
        # cooperative launch under capture: auto mode records the per-layer kernels
        st.set_option(H.OPT_DECODE_LAUNCH, 0)
        st.set_option(H.OPT_PERSISTENT_DECODE, 1)
        print("graph: cooperative launch under capture, auto mode", flush=True)
        xd.copy_(x0)
        g2 = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g2, stream=s):
            H.check(decode(xd))
        torch.cuda.synchronize()
        xd.copy_(x0)
        torch.cuda.synchronize()
        g2.replay()
        torch.cuda.synchronize()
        parity.assert_parity(xd.cpu().numpy(), ref, "per-layer kernels recorded in place of the cooperative launch")
        st.set_option(H.OPT_PERSISTENT_DECODE, 2)
        g3 = torch.cuda.CUDAGraph()
        rc = None
        with torch.cuda.graph(g3, stream=s):
            rc = decode(xd)
        torch.cuda.synchronize()
        assert rc == H.ERR_UNSUPPORTED
    finally:
        st.close()
