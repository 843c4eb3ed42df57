// C++ orchestrator behind the C ABI in include/hoard_moe.h.
//
// Mirrors the reference's per-layer stage order (src/run_moe_stream.cpp:
// router tail :353-373 -> slot fetch :379-421 -> graph B :424-445 -> combine
// :447) with every step a device launch on the caller's stream.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "hoard_moe.h"
#include "kernels.h"
#include "slot_lru.h"
#include "store_impl.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

#define HIP_TRY(expr)                                                                        \
    do {                                                                                     \
        hipError_t e_ = (expr);                                                              \
        if (e_ != hipSuccess) return fail(HOARD_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

constexpr size_t kTailPad = 4096;  // kernels read whole 1 KB chunks past the end of a staged run
// Slot uploads in flight at once (the caller's copy stream and two more): on
// the 128-expert pool workload 3 streams move 46.9 GB/s of host-to-HBM traffic
// against 45.5 for 2; a fourth adds nothing.
constexpr int kUpStreams = 3;

bool quant_type_ok(int t) {
    return t == HOARD_TYPE_Q4_K || t == HOARD_TYPE_Q6_K || t == HOARD_TYPE_Q5_K || t == HOARD_TYPE_Q3_K;
}

size_t mat_bytes(int type, int rows, int cols) {
    return (size_t)rows * (size_t)(cols / 256) * hoard::block_bytes(type);
}

struct Layer {
    bool loaded = false;
    float *router = nullptr;
    int gate_type = 0, up_type = 0, down_type = 0;
    size_t gstride = 0, ustride = 0, dstride = 0;  // bytes between consecutive experts (or slots)
    size_t gbytes = 0, ubytes = 0, dbytes = 0;     // bytes of one expert's matrix
    uint8_t *gate = nullptr, *up = nullptr, *down = nullptr;
    int sh_gate_type = 0, sh_up_type = 0, sh_down_type = 0;
    uint8_t *sh_gate = nullptr, *sh_up = nullptr, *sh_down = nullptr;
    float *sh_gate_inp = nullptr;
    // pool_k > 0: gate/up/down above point into K slots of one record
    // [gate | up | down] each (stride = record size), so a miss is one copy from
    // the pinned host masters, laid out the same way per expert (the
    // reference's RAM tier, here never evicted)
    uint8_t *slots = nullptr;
    uint8_t *host_experts = nullptr;
    hipEvent_t copied[kUpStreams] = {};  // last uploads into this layer's slots, per upload stream
    hipEvent_t last_use = nullptr;  // last FFN reading this layer's slots (compute stream)
    bool used = false;              // last_use has been recorded
    int32_t *slot_stage = nullptr;  // pinned staging of the slot ids handed to the device
    hipEvent_t staged = nullptr;    // the staging copy has been consumed
    bool stage_pending = false;
};

}  // namespace

struct hoard_moe {
    hoard_moe_cfg cfg{};
    int device = 0;
    std::vector<Layer> layers;
    // per-call device scratch
    float *fx = nullptr;          // [max_tokens][n_embd]
    float *logits = nullptr;      // [max_tokens][n_expert]
    unsigned *counters = nullptr; // [max_tokens]
    int32_t *sel = nullptr;       // [max_tokens][n_used]
    float *wsel = nullptr;        // [max_tokens][n_used]
    float *sgate = nullptr;       // [max_tokens]
    float *hbuf = nullptr;        // [n_used+1][hstride]
    int hstride = 0;
    hoard_moe_stats stats{};
    // per-launch event pairs while profiling is enabled
    bool profiling = false;
    struct Mark {
        int kind;
        hipEvent_t a, b;
    };
    std::vector<Mark> marks;
    std::vector<hipEvent_t> event_pool;
    // persistent stacked decode
    bool persistent_shape_ok = false;  // shape/device admit a one-launch decode
    bool xcd_ok = false;               // ... the expert-per-XCD kernel
    bool spread_ok = false;            // ... the rows-spread kernel
    int persistent_mode = 1;           // HOARD_OPT_PERSISTENT_DECODE value
    int decode_kernel = 0;             // HOARD_OPT_DECODE_KERNEL value
    bool layer_kernels = true;         // HOARD_OPT_LAYER_KERNELS: instantiated per-layer kernels
    bool layer_fused = true;           // HOARD_OPT_LAYER_FUSED: one launch per layer where it applies
    bool chip_ok = false;              // gfx950 with 8 XCDs of 32 CUs, every expert resident
    unsigned long long *fctr = nullptr;  // the one-launch layer's counters, then its error word
    uint64_t *flgw = nullptr;            // its tagged logits, one copy per XCD
    uint64_t *fht = nullptr;             // its tagged h, [n_used+1][hstride]
    uint32_t *fq8d = nullptr;            // its Q8_K(h) blocks, [n_used+1][hstride/256][kFusedQ8Words]
    uint64_t *fq8f = nullptr;            // their flags (tagged words), [8][128]
    uint64_t *fsgt = nullptr;            // its tagged shared-expert gate
    unsigned long long *ftrace = nullptr;  // its phase stamps while tracing
    size_t ftrace_words = 0, ftrace_last = 0;
    bool coop_launch = true;           // HOARD_OPT_DECODE_LAUNCH 0: cooperative one-launch decode
    long long wait_ticks = 20000000;   // HOARD_OPT_WAIT_LIMIT_US: bound of the decode's waits (100 MHz ticks)
    hoard::DecodeLayer *d_table = nullptr;  // per-layer pointers of the one-launch decode, kept current
    uint64_t *pX = nullptr, *pLG = nullptr, *pH = nullptr, *pY = nullptr;
    uint64_t *sX = nullptr, *sLG = nullptr, *sH = nullptr, *sY = nullptr;  // spread kernel's exchange words
    unsigned *sflags = nullptr;                                             // its tickets
    unsigned *pflags = nullptr;        // tickets
    int *perr = nullptr;
    unsigned *seqw = nullptr;          // device: sequence base + finished count, [0..1] expert-per-XCD kernel,
                                       // [32..33] rows-spread kernel
    unsigned long long *ptrace = nullptr;  // phase stamps of the last traced decode
    // expert slot pool (pool_k > 0)
    hoard::SlotLru lru;
    bool pool_naive = false;
    int pool_ids_cap = 0;             // ids one pool step takes: min(max_tokens, 512) x n_used
    std::vector<int32_t> pool_slots;  // host scratch of a pool step, pool_ids_cap entries each
    std::vector<uint8_t> pool_miss;
    std::vector<int32_t> pool_mids;
    std::vector<int> pool_mj;
    int32_t *pin_sel = nullptr;     // pinned [n_used]: device-routed ids read back on the on-demand path
    int32_t *slot_ids = nullptr;    // device [n_used]: slots of the on-demand path
    hipStream_t copy_x[kUpStreams - 1] = {};  // upload streams besides the caller's: copies in flight
                                              // together hide each one's set-up
    int fail_upload = 0;            // HOARD_OPT_FAIL_UPLOAD: the n-th slot upload from now fails (test hook)
    hoard::Store *store = nullptr;  // storage tier serving slot misses (attached), else pinned masters
    bool weights_set = false;       // a layer's weights were set (a store attaches before that)
    // batched path (allocated on first use)
    uint8_t *b_q8x = nullptr, *b_q8h = nullptr;
    float *b_h = nullptr, *b_y = nullptr;
    int *b_ints = nullptr;          // group count, then the arrays of batched_layout
    unsigned *b_hist = nullptr;     // [E]
    unsigned *b_counters = nullptr; // route kernel's completion counters
    int *b_layout_ysrc = nullptr, *b_layout_bad = nullptr;  // caller-id arrays within b_ints
    bool hist_pending = false;      // a batched call ran since the histogram was last read
    const unsigned *hist_src = nullptr;  // the last batched call's histogram and group count
    const int *nu_src = nullptr;
    unsigned *nab_stats = nullptr;  // the allocation-free call's histogram [n_expert] and group count,
                                    // copied out of the shared fixed array (allocated at creation)
    size_t trace_layers = 0;
    bool tracing = false;
    int trace_last = 0;  // layers covered by the last traced decode

    ~hoard_moe() {
        for (auto &m : marks) {
            hipEventDestroy(m.a);
            hipEventDestroy(m.b);
        }
        for (auto e : event_pool) hipEventDestroy(e);
        for (auto &L : layers) free_layer(L);
        hipFree(fx);
        hipFree(logits);
        hipFree(counters);
        hipFree(sel);
        hipFree(wsel);
        hipFree(sgate);
        hipFree(hbuf);
        hipFree(d_table);
        hipFree(pX);
        hipFree(pLG);
        hipFree(pH);
        hipFree(pY);
        hipFree(sX);
        hipFree(sLG);
        hipFree(sH);
        hipFree(sY);
        hipFree(sflags);
        hipFree(pflags);
        hipFree(perr);
        hipFree(seqw);
        hipFree(fctr);
        hipFree(flgw);
        hipFree(fht);
        hipFree(fq8d);
        hipFree(fq8f);
        hipFree(fsgt);
        hipFree(ftrace);
        hipFree(ptrace);
        hipHostFree(pin_sel);
        hipFree(slot_ids);
        for (auto cx : copy_x)
            if (cx) hipStreamDestroy(cx);
        hipFree(b_q8x);
        hipFree(b_q8h);
        hipFree(b_h);
        hipFree(b_y);
        hipFree(b_ints);
        hipFree(b_hist);
        hipFree(b_counters);
        hipFree(nab_stats);
    }
    static void free_layer(Layer &L) {
        for (auto ev : L.copied)
            if (ev) hipEventDestroy(ev);
        if (L.last_use) hipEventDestroy(L.last_use);
        if (L.staged) hipEventDestroy(L.staged);
        hipHostFree(L.host_experts);
        hipHostFree(L.slot_stage);
        if (L.slots) {
            hipFree(L.slots);
            L.gate = L.up = L.down = nullptr;  // views into slots
        }
        hipFree(L.router);
        hipFree(L.gate);
        hipFree(L.up);
        hipFree(L.down);
        hipFree(L.sh_gate);
        hipFree(L.sh_up);
        hipFree(L.sh_down);
        hipFree(L.sh_gate_inp);
        L = Layer{};
    }
};

namespace {

int dev_alloc(void **p, size_t n) {
    hipError_t e = hipMalloc(p, n);
    if (e != hipSuccess) {
        *p = nullptr;
        (void)hipGetLastError();
        return fail(HOARD_ERR_OOM, "hipMalloc(%zu): %s", n, hipGetErrorString(e));
    }
    return HOARD_OK;
}

int upload(void **dst, const void *src, size_t n, size_t alloc) {
    int rc = dev_alloc(dst, alloc);
    if (rc) return rc;
    HIP_TRY(hipMemcpy(*dst, src, n, hipMemcpyHostToDevice));
    return HOARD_OK;
}

int check_layer(hoard_moe *h, int layer) {
    if (!h) return fail(HOARD_ERR_INVALID, "null handle");
    if (layer < 0 || layer >= h->cfg.n_layer) return fail(HOARD_ERR_INVALID, "layer %d out of range", layer);
    if (!h->layers[layer].loaded) return fail(HOARD_ERR_STATE, "layer %d has no weights", layer);
    HIP_TRY(hipSetDevice(h->device));
    return HOARD_OK;
}

hoard::MatDesc mat(const uint8_t *base, size_t stride, int type, int rows, int cols, int n_ids) {
    hoard::MatDesc m;
    m.base = base;
    m.stride = stride;
    m.type = type;
    m.rows = rows;
    m.cols = cols;
    m.n_ids = n_ids;
    return m;
}

hipEvent_t take_event(hoard_moe *h) {
    if (!h->event_pool.empty()) {
        hipEvent_t e = h->event_pool.back();
        h->event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

// Brackets one launch with an event pair when profiling; no-op otherwise.
struct KernelMark {
    hoard_moe *h;
    int kind;
    hipStream_t s;
    hipEvent_t a = nullptr;
    KernelMark(hoard_moe *h_, int kind_, hipStream_t s_) : h(h_), kind(kind_), s(s_) {
        if (h->profiling && (a = take_event(h))) hipEventRecord(a, s);
    }
    ~KernelMark() {
        if (!a) return;
        hipEvent_t b = take_event(h);
        if (!b) {
            h->event_pool.push_back(a);
            return;
        }
        hipEventRecord(b, s);
        h->marks.push_back({kind, a, b});
    }
};

int run_route(hoard_moe *h, const Layer &L, const float *xin, int is_residual, float eps, int32_t *sel,
              float *w, hipStream_t s) {
    const hoard_moe_cfg &c = h->cfg;
    hoard::RouterArgs a{};
    a.xin = xin;
    a.fx_out = h->fx;
    a.eps = eps;
    a.xin_is_residual = is_residual;
    a.w = L.router;
    a.n = c.n_embd;
    a.E = c.n_expert;
    a.k = c.n_used;
    a.renorm = c.renorm;
    a.M = 1;
    a.logits = h->logits;
    a.counters = h->counters;
    a.sel = sel;
    a.wsel = w;
    const bool fast = h->layer_kernels && hoard::layer_route_ok(a) &&
                      ((reinterpret_cast<uintptr_t>(xin) | reinterpret_cast<uintptr_t>(L.router)) & 15) == 0;
    KernelMark mark(h, HOARD_KERNEL_ROUTER, s);
    HIP_TRY(fast ? hoard::launch_layer_route(a, s) : hoard::launch_router(a, s));
    return HOARD_OK;
}

int run_ffn(hoard_moe *h, const Layer &L, const float *fx, const int32_t *ids, const float *w,
            const float *res, float *out, hipStream_t s) {
    const hoard_moe_cfg &c = h->cfg;
    const int n_ids = c.pool_k > 0 ? c.pool_k : c.n_expert;  // ids are slots in pool mode
    const bool sh = c.n_ff_shexp > 0;
    hoard::GateUpArgs g{};
    g.fx = fx;
    g.ids = ids;
    g.gate = mat(L.gate, L.gstride, L.gate_type, c.n_ff, c.n_embd, n_ids);
    g.up = mat(L.up, L.ustride, L.up_type, c.n_ff, c.n_embd, n_ids);
    if (sh) {
        g.sh_gate = mat(L.sh_gate, 0, L.sh_gate_type, c.n_ff_shexp, c.n_embd, 1);
        g.sh_up = mat(L.sh_up, 0, L.sh_up_type, c.n_ff_shexp, c.n_embd, 1);
        g.sh_gate_inp = L.sh_gate_inp;
    }
    g.sgate = h->sgate;
    g.n_embd = c.n_embd;
    g.k = c.n_used;
    g.h = h->hbuf;
    g.hstride = h->hstride;
    hoard::DownArgs d{};
    d.h = h->hbuf;
    d.hstride = h->hstride;
    d.ids = ids;
    d.w = w;
    d.down = mat(L.down, L.dstride, L.down_type, c.n_embd, c.n_ff, n_ids);
    if (sh) d.sh_down = mat(L.sh_down, 0, L.sh_down_type, c.n_embd, c.n_ff_shexp, 1);
    d.sgate = h->sgate;
    d.n_embd = c.n_embd;
    d.k = c.n_used;
    d.res = res;
    d.out = out;
    const bool fast = h->layer_kernels && hoard::layer_ffn_ok(g, d);
    hipError_t e;
    {
        KernelMark mark(h, HOARD_KERNEL_GATEUP, s);
        e = fast ? hoard::launch_layer_gateup(g, s) : hoard::launch_gateup(g, s);
    }
    if (e != hipSuccess) return fail(HOARD_ERR_HIP, "gate/up launch: %s", hipGetErrorString(e));
    {
        KernelMark mark(h, HOARD_KERNEL_DOWN, s);
        e = fast ? hoard::launch_layer_down(d, s) : hoard::launch_down_combine(d, s);
    }
    if (e != hipSuccess) return fail(HOARD_ERR_HIP, "down/combine launch: %s", hipGetErrorString(e));
    return HOARD_OK;
}

// The whole layer in one launch (router, gate/up and down workgroups in the
// order they start, layer.hip) where the shape and handle admit it: every
// expert resident, a shared expert as wide as the routed ones.  *done reports
// whether it ran.  xin is fx, or with rms the residual x whose rms_norm is fx.
int run_layer_fused(hoard_moe *h, const Layer &L, const float *xin, int rms, float eps, const float *res, float *out,
                    int32_t *sel, float *w, hipStream_t s, bool *done) {
    *done = false;
    const hoard_moe_cfg &c = h->cfg;
    if (!h->layer_fused || !h->layer_kernels || !h->chip_ok || c.pool_k > 0) return HOARD_OK;
    if (c.n_ff_shexp > 0 && c.n_ff_shexp != c.n_ff) return HOARD_OK;
    hoard::FusedLayerArgs a{};
    a.xin = xin;
    a.rms = rms;
    a.eps = eps;
    a.res = res;
    a.out = out;
    a.sel = sel;
    a.wsel = w;
    a.router = L.router;
    a.gate = mat(L.gate, L.gstride, L.gate_type, c.n_ff, c.n_embd, c.n_expert);
    a.up = mat(L.up, L.ustride, L.up_type, c.n_ff, c.n_embd, c.n_expert);
    a.down = mat(L.down, L.dstride, L.down_type, c.n_embd, c.n_ff, c.n_expert);
    if (c.n_ff_shexp > 0) {
        a.sh_gate = mat(L.sh_gate, 0, L.sh_gate_type, c.n_ff_shexp, c.n_embd, 1);
        a.sh_up = mat(L.sh_up, 0, L.sh_up_type, c.n_ff_shexp, c.n_embd, 1);
        a.sh_down = mat(L.sh_down, 0, L.sh_down_type, c.n_embd, c.n_ff_shexp, 1);
        a.sh_gate_inp = L.sh_gate_inp;
    }
    a.n_embd = c.n_embd;
    a.E = c.n_expert;
    a.k = c.n_used;
    a.renorm = c.renorm;
    a.lgw = h->flgw;
    a.ht = h->fht;
    a.q8d = h->fq8d;
    a.q8f = h->fq8f;
    a.sgt = h->fsgt;
    a.ctr = h->fctr;
    a.err = reinterpret_cast<int *>(h->fctr + hoard::kFusedCounterWords);
    a.wait_ticks = h->wait_ticks;
    if (!hoard::fused_layer_ok(a)) return HOARD_OK;
    if (h->tracing) {
        // the stamp buffer may be (re)allocated here, which a capturing stream must not see
        hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
        HIP_TRY(hipStreamIsCapturing(s, &capture));
        if (capture != hipStreamCaptureStatusNone)
            return fail(HOARD_ERR_UNSUPPORTED, "one-launch layer: phase tracing is not captured");
        // phase stamps of this launch: [workgroup][kFusedStamps] (read with hoard_moe_fused_trace_read)
        const size_t words = (size_t)hoard::fused_layer_groups(a) * hoard::kFusedStamps;
        if (h->ftrace_words < words) {
            hipFree(h->ftrace);
            h->ftrace = nullptr;
            if (int rc = dev_alloc((void **)&h->ftrace, words * sizeof(unsigned long long))) return rc;
            h->ftrace_words = words;
        }
        a.trace = h->ftrace;
        h->ftrace_last = words;
    }
    {
        KernelMark mark(h, HOARD_KERNEL_LAYER, s);
        HIP_TRY(hoard::launch_fused_layer(a, s));
    }
    *done = true;
    return HOARD_OK;
}

// Slot pool step for one layer: LRU bookkeeping on the host, uploads of the
// missed experts on copy_stream (after the previous FFN that read this layer's
// slots), and `stream` made to wait for them.  slot_dev (optional) receives
// the slot ids through a pinned staging copy on `stream`.
// ids one pool step takes: a batch of up to 512 tokens (the batched entry
// points' limit) times n_used
int pool_ids_cap(const hoard_moe_cfg &c) {
    return std::min(c.max_tokens, hoard::kBatchedMaxTokensLarge) * c.n_used;
}

// One slot upload.  HOARD_OPT_FAIL_UPLOAD counts down to an upload that fails
// as a refused hipMemcpyAsync would, before anything is issued.
hipError_t slot_upload(hoard_moe *h, void *dst, const void *src, size_t n, hipStream_t s) {
    if (h->fail_upload > 0 && --h->fail_upload == 0) return hipErrorOutOfMemory;
    return hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, s);
}

// A pool step that failed part-way: wait for the uploads it issued, then
// forget the layer's slot residency.
void pool_abandon(hoard_moe *h, int layer, const hipStream_t *up) {
    for (int i = 0; i < kUpStreams; ++i)
        (void)hipStreamSynchronize(up[i]);
    (void)hipGetLastError();
    h->lru.reset_layer(layer);
}

int pool_ensure(hoard_moe *h, int layer, const int32_t *sel, int n, bool sequential, int32_t *slot_host,
                int32_t *slot_dev, hipStream_t s, hipStream_t cs) {
    const hoard_moe_cfg &c = h->cfg;
    Layer &L = h->layers[layer];
    for (int j = 0; j < n; ++j)
        if (sel[j] < 0 || sel[j] >= c.n_expert) return fail(HOARD_ERR_INVALID, "expert id %d out of range", sel[j]);
    if (n > h->pool_ids_cap) return fail(HOARD_ERR_INVALID, "%d ids in one pool step (at most %d)", n, h->pool_ids_cap);
    int32_t *slots = h->pool_slots.data();
    uint8_t *miss = h->pool_miss.data();
    if (sequential)
        h->lru.access_sequential(layer, sel, n, slots, miss);
    else
        h->lru.access(layer, sel, n, h->pool_naive, slots, miss);
    int n_miss = 0;
    for (int j = 0; j < n; ++j) n_miss += miss[j];
    // From here on the LRU maps the missed slots to their new experts: a failure
    // before their uploads are issued leaves the slots holding other bytes, so
    // the layer's residency is forgotten (every slot is a miss next time), and
    // the uploads already issued are waited for, so none lands after a later
    // upload into the same slot.
#define POOL_TRY(expr)                                                                           \
    do {                                                                                         \
        hipError_t e_ = (expr);                                                                  \
        if (e_ != hipSuccess) {                                                                  \
            pool_abandon(h, layer, up);                                                          \
            return fail(HOARD_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_));                  \
        }                                                                                        \
    } while (0)
    // misses are dealt round-robin to the caller's copy stream and the internal
    // ones; each first waits until the last FFN reading this layer's slots is done
    hipStream_t up[kUpStreams];
    up[0] = cs;
    for (int i = 1; i < kUpStreams; ++i) up[i] = h->copy_x[i - 1];
    const int n_up = n_miss < kUpStreams ? (n_miss > 0 ? n_miss : 1) : kUpStreams;
    if (n_miss && L.used)
        for (int i = 0; i < n_up; ++i) POOL_TRY(hipStreamWaitEvent(up[i], L.last_use, 0));
    int m = 0;
    if (h->store) {
        // storage tier: the RAM tier serves or reads the missed experts (reads in
        // parallel, on the host), then each is uploaded from its RAM entry,
        // which is fenced until the upload is done
        int32_t *mids = h->pool_mids.data();
        int *mj = h->pool_mj.data(), nm = 0;
        for (int j = 0; j < n; ++j)
            if (miss[j]) {
                mj[nm] = j;
                mids[nm++] = sel[j];
            }
        std::vector<hoard::StoreEntry> ent((size_t)n);
        if (nm) {
            if (int rc = h->store->fetch(layer, nm, mids, ent.data(), nullptr)) {
                h->lru.reset_layer(layer);  // the missed slots were not filled: forget the layer's residency
                return rc;                  // the store has set the error text
            }
        }
        const size_t rec = L.gstride;
        for (int i = 0; i < nm; ++i) {
            uint8_t *dst = L.slots + (size_t)slots[mj[i]] * rec;
            hipStream_t us = up[m++ % n_up];
            POOL_TRY(slot_upload(h, dst, ent[i].part[0], L.gbytes, us));
            POOL_TRY(slot_upload(h, dst + L.gbytes, ent[i].part[1], L.ubytes, us));
            POOL_TRY(slot_upload(h, dst + L.gbytes + L.ubytes, ent[i].part[2], L.dbytes, us));
            if (int rc = h->store->fence(ent[i].slot, us)) {
                pool_abandon(h, layer, up);
                return rc;
            }
        }
        for (int j = 0; j < n; ++j) {
            h->stats.reqs += 1;
            h->stats.hits += miss[j] ? 0 : 1;
            h->stats.misses += miss[j] ? 1 : 0;
            h->stats.bytes_h2d += miss[j] ? rec : 0;
        }
    } else {
        for (int j = 0; j < n; ++j) {
            h->stats.reqs += 1;
            if (!miss[j]) {
                h->stats.hits += 1;
                continue;
            }
            const size_t e = (size_t)sel[j], sl = (size_t)slots[j], rec = L.gstride;  // one [g|u|d] record
            POOL_TRY(slot_upload(h, L.slots + sl * rec, L.host_experts + e * rec, rec, up[m++ % n_up]));
            h->stats.misses += 1;
            h->stats.bytes_h2d += rec;
        }
    }
    if (n_miss) {
        for (int i = 0; i < n_up; ++i) {
            POOL_TRY(hipEventRecord(L.copied[i], up[i]));
            POOL_TRY(hipStreamWaitEvent(s, L.copied[i], 0));
        }
    }
#undef POOL_TRY
    if (slot_host) std::memcpy(slot_host, slots, sizeof(int32_t) * n);
    if (slot_dev) {
        if (L.stage_pending) HIP_TRY(hipEventSynchronize(L.staged));  // previous ids consumed
        std::memcpy(L.slot_stage, slots, sizeof(int32_t) * n);
        HIP_TRY(hipMemcpyAsync(slot_dev, L.slot_stage, sizeof(int32_t) * n, hipMemcpyHostToDevice, s));
        HIP_TRY(hipEventRecord(L.staged, s));
        L.stage_pending = true;
    }
    return HOARD_OK;
}

// Marks the end of an FFN that read `layer`'s slots (pool mode).
int pool_mark_use(hoard_moe *h, int layer, hipStream_t s) {
    if (h->cfg.pool_k == 0) return HOARD_OK;
    Layer &L = h->layers[layer];
    HIP_TRY(hipEventRecord(L.last_use, s));
    L.used = true;
    return HOARD_OK;
}

// On-demand pool step after a device-side route: the selection is read back
// (the reference's D2H of sel, :367), then the slots are ensured.
int pool_after_route(hoard_moe *h, int layer, const int32_t *sel_dev, int32_t *slot_dev, hipStream_t s) {
    HIP_TRY(hipMemcpyAsync(h->pin_sel, sel_dev, sizeof(int32_t) * h->cfg.n_used, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipStreamSynchronize(s));
    return pool_ensure(h, layer, h->pin_sel, h->cfg.n_used, false, nullptr, slot_dev, s, s);
}

// The one-launch decodes need 8 XCDs x 32 CUs (one workgroup per CU).  The
// expert-per-XCD kernel takes k = 8 routed experts (one per XCD) of E <= 128
// with no shared expert; the rows-spread kernel takes the instantiated
// {n_embd, n_ff, k, E, shared} shapes.  Otherwise hoard_moe_decode launches the
// per-layer kernels.
constexpr int kPersistentCus = 256;

hoard::SpreadArgs spread_shape(const hoard_moe_cfg &c) {
    hoard::SpreadArgs a{};
    a.n_embd = c.n_embd;
    a.n_ff = c.n_ff;
    a.E = c.n_expert;
    a.k = c.n_used;
    a.shared = c.n_ff_shexp > 0 ? 1 : 0;
    a.d_type = a.sh_d_type = -1;  // any: the layers' types are checked at launch
    return a;
}

int persistent_setup(hoard_moe *h) {
    const hoard_moe_cfg &c = h->cfg;
    int cus = 0;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, h->device) != hipSuccess) return fail(HOARD_ERR_HIP, "device properties");
    cus = prop.multiProcessorCount;
    const bool arch_ok = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 && cus == kPersistentCus && c.pool_k == 0;
    h->chip_ok = arch_ok;
    h->xcd_ok = arch_ok && c.n_embd == 2048 && c.n_used == 8 && c.n_expert % 32 == 0 && c.n_expert <= 128 &&
                c.n_ff % 256 == 0 && c.n_ff <= 1024 && c.n_ff_shexp == 0;
    h->spread_ok = arch_ok && (c.n_ff_shexp == 0 || c.n_ff_shexp == c.n_ff) &&
                   hoard::spread_shape_compiled(spread_shape(c));
    h->persistent_shape_ok = h->xcd_ok || h->spread_ok;
    int rc = 0;
    if (h->persistent_shape_ok) {
        rc = dev_alloc((void **)&h->d_table, sizeof(hoard::DecodeLayer) * c.n_layer);
        rc = rc ? rc : dev_alloc((void **)&h->perr, sizeof(int));
        rc = rc ? rc : dev_alloc((void **)&h->seqw, 64 * sizeof(unsigned));
        if (rc) return rc;
        HIP_TRY(hipMemset(h->d_table, 0, sizeof(hoard::DecodeLayer) * c.n_layer));
        HIP_TRY(hipMemset(h->perr, 0, sizeof(int)));
        // sequence tags start at 1, so zeroed exchange words never read as current
        unsigned init[64] = {};
        init[0] = init[32] = 1u;
        HIP_TRY(hipMemcpy(h->seqw, init, sizeof init, hipMemcpyHostToDevice));
    }
    if (h->xcd_ok) {
        const size_t nX = (size_t)2 * 8 * c.n_embd, nLG = (size_t)8 * c.n_expert, nH = (size_t)8 * c.n_ff;
        rc = rc ? rc : dev_alloc((void **)&h->pX, sizeof(uint64_t) * nX);
        rc = rc ? rc : dev_alloc((void **)&h->pLG, sizeof(uint64_t) * nLG);
        rc = rc ? rc : dev_alloc((void **)&h->pH, sizeof(uint64_t) * nH);
        rc = rc ? rc : dev_alloc((void **)&h->pY, sizeof(uint64_t) * nX);
        const size_t flag_words = (size_t)8 * 32;
        rc = rc ? rc : dev_alloc((void **)&h->pflags, flag_words * sizeof(unsigned));
        if (rc) return rc;
        HIP_TRY(hipMemset(h->pX, 0, sizeof(uint64_t) * nX));
        HIP_TRY(hipMemset(h->pLG, 0, sizeof(uint64_t) * nLG));
        HIP_TRY(hipMemset(h->pH, 0, sizeof(uint64_t) * nH));
        HIP_TRY(hipMemset(h->pY, 0, sizeof(uint64_t) * nX));
        HIP_TRY(hipMemset(h->pflags, 0, flag_words * sizeof(unsigned)));
    }
    if (h->spread_ok) {
        const size_t units = (size_t)c.n_used + (c.n_ff_shexp > 0 ? 1 : 0);
        const size_t nX = (size_t)8 * c.n_embd, nLG = (size_t)256 * c.n_expert;
        const size_t nH = units * c.n_ff, nY = units * c.n_embd, nF = (size_t)8 * 32;
        rc = rc ? rc : dev_alloc((void **)&h->sX, sizeof(uint64_t) * nX);
        rc = rc ? rc : dev_alloc((void **)&h->sLG, sizeof(uint64_t) * nLG);
        rc = rc ? rc : dev_alloc((void **)&h->sH, sizeof(uint64_t) * nH);
        rc = rc ? rc : dev_alloc((void **)&h->sY, sizeof(uint64_t) * nY);
        rc = rc ? rc : dev_alloc((void **)&h->sflags, sizeof(unsigned) * nF);
        if (rc) return rc;
        HIP_TRY(hipMemset(h->sX, 0, sizeof(uint64_t) * nX));
        HIP_TRY(hipMemset(h->sLG, 0, sizeof(uint64_t) * nLG));
        HIP_TRY(hipMemset(h->sH, 0, sizeof(uint64_t) * nH));
        HIP_TRY(hipMemset(h->sY, 0, sizeof(uint64_t) * nY));
        HIP_TRY(hipMemset(h->sflags, 0, sizeof(unsigned) * nF));
    }
    return HOARD_OK;
}

// Phase-stamp buffer of a traced one-launch decode ([layer][256][kTracePhases]);
// *out stays null while tracing is off.
int trace_buffer(hoard_moe *h, int l0, int l1, unsigned long long **out) {
    *out = nullptr;
    if (!h->tracing) return HOARD_OK;
    const int nl = h->cfg.n_layer;
    if (h->trace_layers < (size_t)nl) {
        hipFree(h->ptrace);
        h->ptrace = nullptr;
        int rc = dev_alloc((void **)&h->ptrace, sizeof(unsigned long long) * nl * 256 * hoard::kTracePhases);
        if (rc) return rc;
        h->trace_layers = nl;
    }
    *out = h->ptrace;
    h->trace_last = l1 - l0;
    return HOARD_OK;
}

// The rows-spread one-launch decode over [l0, l1); the layer table is current.
template <class Skip>
int spread_decode(hoard_moe *h, int l0, int l1, float *x, float eps, hipStream_t s, bool *used, Skip skip) {
    const hoard_moe_cfg &c = h->cfg;
    const bool sh = c.n_ff_shexp > 0;
    const int d_type = h->layers[l0].down_type, sh_d_type = sh ? h->layers[l0].sh_down_type : d_type;
    for (int l = l0; l < l1; ++l) {
        const Layer &L = h->layers[l];
        if (L.gate_type != HOARD_TYPE_Q4_K || L.up_type != HOARD_TYPE_Q4_K || L.down_type != d_type)
            return skip("rows-spread decode takes Q4_K gate/up and one down type over the range");
        if (sh) {
            if (L.sh_gate_type != HOARD_TYPE_Q4_K || L.sh_up_type != HOARD_TYPE_Q4_K || L.sh_down_type != sh_d_type)
                return skip("rows-spread decode takes a Q4_K/Q4_K shared expert of one down type over the range");
            const uintptr_t al = reinterpret_cast<uintptr_t>(L.sh_gate) | reinterpret_cast<uintptr_t>(L.sh_up) |
                                 reinterpret_cast<uintptr_t>(L.sh_down) | reinterpret_cast<uintptr_t>(L.sh_gate_inp);
            if (al & 15) return skip("shared expert tensors are not 16-byte aligned");
        }
        if (reinterpret_cast<uintptr_t>(L.router) & 15) return skip("router is not 16-byte aligned");
    }
    hoard::SpreadArgs a = spread_shape(c);
    a.d_type = d_type;
    a.sh_d_type = sh_d_type;
    if (!hoard::spread_shape_compiled(a)) return skip("no rows-spread kernel for these down types");
    a.layers = h->d_table;
    a.l0 = l0;
    a.l1 = l1;
    a.x = x;
    a.eps = eps;
    a.renorm = c.renorm;
    a.LG = h->sLG;
    a.H = h->sH;
    a.Y = h->sY;
    a.X = h->sX;
    a.tickets = h->sflags;
    a.err = h->perr;
    a.seq = h->seqw + 32;
    a.wait_ticks = h->wait_ticks;
    if (int rc = trace_buffer(h, l0, l1, &a.trace)) return rc;
    hipError_t e;
    {
        KernelMark mark(h, HOARD_KERNEL_DECODE, s);
        e = hoard::launch_spread_decode(a, s, h->coop_launch);
    }
    if (e != hipSuccess) {
        (void)hipGetLastError();
        if (h->persistent_mode == 2) return fail(HOARD_ERR_HIP, "spread decode launch: %s", hipGetErrorString(e));
        return HOARD_OK;  // auto mode: fall back to the per-layer kernels
    }
    *used = true;
    return HOARD_OK;
}

// The per-layer kernels over [l0, l1): route, slot fetch when pooled, experts and combine.
int decode_layers(hoard_moe *h, int l0, int l1, float *x_dev, float eps, hipStream_t s) {
    for (int l = l0; l < l1; ++l) {
        int rc = 0;
        const Layer &L = h->layers[l];
        bool fused = false;
        rc = run_layer_fused(h, L, x_dev, 1, eps, x_dev, x_dev, h->sel, h->wsel, s, &fused);
        if (rc) return rc;
        if (fused) continue;
        rc = run_route(h, L, x_dev, 1, eps, h->sel, h->wsel, s);
        if (rc) return rc;
        const int32_t *ids = h->sel;
        if (h->cfg.pool_k > 0) {
            rc = pool_after_route(h, l, h->sel, h->slot_ids, s);
            if (rc) return rc;
            ids = h->slot_ids;
        }
        rc = run_ffn(h, L, h->fx, ids, h->wsel, x_dev, x_dev, s);
        if (rc) return rc;
        rc = pool_mark_use(h, l, s);
        if (rc) return rc;
    }
    return HOARD_OK;
}

bool same_types(const Layer &a, const Layer &b) {
    return a.gate_type == b.gate_type && a.up_type == b.up_type && a.down_type == b.down_type &&
           a.sh_gate_type == b.sh_gate_type && a.sh_up_type == b.sh_up_type && a.sh_down_type == b.sh_down_type;
}

// Launches the one-launch decode when it applies; *used reports whether it did.
// A cooperative launch costs about 22 us before its first layer (35.5 us for one
// layer against 13.2 us for each further one), and the per-layer launches take
// 22-28 us a layer: automatic mode takes the one-launch kernel from 3 layers on.
constexpr int kMinPersistentLayers = 3;

int persistent_decode(hoard_moe *h, int l0, int l1, float *x, float eps, hipStream_t s, bool *used) {
    *used = false;
    if (!h->persistent_shape_ok || h->persistent_mode == 0 || l0 >= l1) return HOARD_OK;
    if (h->persistent_mode == 1 && l1 - l0 < kMinPersistentLayers) return HOARD_OK;
    const hoard_moe_cfg &c = h->cfg;
    // Forced mode reports why the range cannot take the one-launch path; auto
    // mode falls back to the per-layer kernels.
    auto skip = [&](const char *why) {
        return h->persistent_mode == 2 ? fail(HOARD_ERR_UNSUPPORTED, "persistent decode: %s", why) : HOARD_OK;
    };
    // Under stream capture only the plain launch is recorded (its sequence tags
    // live in device memory, so every replay tags its words afresh); the
    // cooperative launch is not captured, and auto mode records the per-layer
    // kernels instead.
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    HIP_TRY(hipStreamIsCapturing(s, &capture));
    if (capture != hipStreamCaptureStatusNone) {
        if (h->coop_launch) return skip("a cooperative launch cannot be captured (HOARD_OPT_DECODE_LAUNCH 1 can)");
        if (h->tracing) return skip("phase tracing is not captured");
    }
    // one kernel instantiation serves the whole range: uniform types, gate = up
    const int gu_type = h->layers[l0].gate_type, d_type = h->layers[l0].down_type;
    for (int l = l0; l < l1; ++l) {
        const Layer &L = h->layers[l];
        if (L.gate_type != gu_type || L.up_type != gu_type || L.down_type != d_type)
            return skip("layer types differ within the range");
        // rows are staged into LDS at their source offset modulo 16; the kernel's
        // row reads need that offset to be 0
        const uintptr_t al = reinterpret_cast<uintptr_t>(L.gate) | reinterpret_cast<uintptr_t>(L.up) |
                             reinterpret_cast<uintptr_t>(L.down) | L.gstride | L.ustride | L.dstride;
        if (al & 15) return skip("expert tensors are not 16-byte aligned");
    }
    // auto picks the expert-per-XCD kernel where it applies, else the rows-spread one
    const bool spread = h->decode_kernel == 2 || (h->decode_kernel == 0 && !h->xcd_ok);
    if (spread ? !h->spread_ok : !h->xcd_ok) return skip("the selected decode kernel does not take this shape");
    if (spread) return spread_decode(h, l0, l1, x, eps, s, used, skip);
    if (!hoard::persistent_shape_compiled(gu_type, c.n_embd, d_type, c.n_ff))
        return skip("no kernel instantiated for these types and sizes");
    const int max_rb_gu = (int)mat_bytes(gu_type, 1, c.n_embd), max_rb_d = (int)mat_bytes(d_type, 1, c.n_ff);
    hoard::PersistentArgs a{};
    a.l0 = l0;
    a.l1 = l1;
    a.x = x;
    a.eps = eps;
    a.n_embd = c.n_embd;
    a.E = c.n_expert;
    a.k = c.n_used;
    a.n_ff = c.n_ff;
    a.renorm = c.renorm;
    a.rows_gu = c.n_ff / 32;
    a.rows_d = c.n_embd / 32;
    a.max_rb_gu = max_rb_gu;
    a.max_rb_d = max_rb_d;
    a.gu_type = gu_type;
    a.d_type = d_type;
    if (hoard::persistent_lds_bytes(a) > hoard::kPersistentMaxLds) return skip("LDS footprint too large");
    a.layers = h->d_table;
    a.X = h->pX;
    a.LG = h->pLG;
    a.H = h->pH;
    a.Y = h->pY;
    a.tickets = h->pflags;
    a.err = h->perr;
    a.seq = h->seqw;
    a.wait_ticks = h->wait_ticks;
    if (int rc = trace_buffer(h, l0, l1, &a.trace)) return rc;
    hipError_t e;
    {
        KernelMark mark(h, HOARD_KERNEL_DECODE, s);
        e = hoard::launch_persistent_decode(a, s, h->coop_launch);
    }
    if (e != hipSuccess) {
        (void)hipGetLastError();
        if (h->persistent_mode == 2) return fail(HOARD_ERR_HIP, "persistent decode launch: %s", hipGetErrorString(e));
        return HOARD_OK;  // auto mode: fall back to the per-layer kernels
    }
    *used = true;
    return HOARD_OK;
}

}  // namespace

extern "C" {

const char *hoard_last_error(void) { return g_err.c_str(); }

// The error text other translation units of the library report through
// hoard_last_error (host_error.h).
int hoard_set_error(int code, const char *msg) {
    g_err = msg ? msg : "";
    return code;
}

int hoard_moe_create(const hoard_moe_cfg *cfg, hoard_moe **out) {
    g_err.clear();
    if (!cfg || !out) return fail(HOARD_ERR_INVALID, "null argument");
    *out = nullptr;
    const hoard_moe_cfg &c = *cfg;
    if (c.n_embd <= 0 || c.n_embd % 256) return fail(HOARD_ERR_INVALID, "n_embd %d not a positive multiple of 256", c.n_embd);
    if (c.n_ff <= 0 || c.n_ff % 256) return fail(HOARD_ERR_INVALID, "n_ff %d not a positive multiple of 256", c.n_ff);
    if (c.n_ff_shexp < 0 || c.n_ff_shexp % 256) return fail(HOARD_ERR_INVALID, "n_ff_shexp %d not a multiple of 256", c.n_ff_shexp);
    if (c.n_expert <= 0 || c.n_expert > 1024) return fail(HOARD_ERR_INVALID, "n_expert %d outside 1..1024", c.n_expert);
    if (c.n_used <= 0 || c.n_used > 16 || c.n_used > c.n_expert)
        return fail(HOARD_ERR_INVALID, "n_used %d outside 1..min(16, n_expert)", c.n_used);
    if (c.n_layer <= 0) return fail(HOARD_ERR_INVALID, "n_layer %d", c.n_layer);
    if (c.max_tokens <= 0) return fail(HOARD_ERR_INVALID, "max_tokens %d", c.max_tokens);
    if (c.pool_k < 0 || (c.pool_k > 0 && (c.pool_k < c.n_used || c.pool_k > c.n_expert)))
        return fail(HOARD_ERR_INVALID, "pool_k %d outside n_used..n_expert (or 0 for all resident)", c.pool_k);
    hoard_moe *h = new (std::nothrow) hoard_moe();
    if (!h) return fail(HOARD_ERR_OOM, "handle");
    h->cfg = c;
    if (hipGetDevice(&h->device) != hipSuccess) {
        delete h;
        return fail(HOARD_ERR_HIP, "no HIP device");
    }
    h->layers.resize(c.n_layer);
    h->hstride = c.n_ff > c.n_ff_shexp ? c.n_ff : c.n_ff_shexp;
    const size_t T = (size_t)c.max_tokens;
    int rc = 0;
    rc = rc ? rc : dev_alloc((void **)&h->fx, T * c.n_embd * sizeof(float));
    rc = rc ? rc : dev_alloc((void **)&h->logits, T * c.n_expert * sizeof(float));
    rc = rc ? rc : dev_alloc((void **)&h->counters, T * sizeof(unsigned));
    rc = rc ? rc : dev_alloc((void **)&h->sel, T * c.n_used * sizeof(int32_t));
    rc = rc ? rc : dev_alloc((void **)&h->wsel, T * c.n_used * sizeof(float));
    rc = rc ? rc : dev_alloc((void **)&h->sgate, T * sizeof(float));
    rc = rc ? rc : dev_alloc((void **)&h->hbuf, (size_t)(c.n_used + 1) * h->hstride * sizeof(float));
    rc = rc ? rc : dev_alloc((void **)&h->fctr, sizeof(unsigned long long) * (hoard::kFusedCounterWords + 1));
    if (!rc && hipMemset(h->fctr, 0, sizeof(unsigned long long) * (hoard::kFusedCounterWords + 1)) != hipSuccess)
        rc = fail(HOARD_ERR_HIP, "hipMemset fused counters");
    // tags start at 0 and the first launch's epoch tag is 1: zeroed words never match
    rc = rc ? rc : dev_alloc((void **)&h->flgw, sizeof(uint64_t) * 8 * c.n_expert);
    if (!rc && hipMemset(h->flgw, 0, sizeof(uint64_t) * 8 * c.n_expert) != hipSuccess)
        rc = fail(HOARD_ERR_HIP, "hipMemset fused logits");
    // the one-launch layer's tagged h, Q8_K(h) blocks and shared gate: zeroed,
    // so no word carries a launch epoch (those start at 1) before it is written
    {
        const size_t nht = (size_t)(c.n_used + 1) * h->hstride;
        const size_t nq8 = (size_t)(c.n_used + 1) * ((h->hstride + 255) / 256) * hoard::kFusedQ8Words;
        rc = rc ? rc : dev_alloc((void **)&h->fht, sizeof(uint64_t) * nht);
        rc = rc ? rc : dev_alloc((void **)&h->fq8d, sizeof(uint32_t) * nq8);
        rc = rc ? rc : dev_alloc((void **)&h->fq8f, sizeof(uint64_t) * 8 * 128);
        rc = rc ? rc : dev_alloc((void **)&h->fsgt, sizeof(uint64_t));
        if (!rc && (hipMemset(h->fht, 0, sizeof(uint64_t) * nht) != hipSuccess ||
                    hipMemset(h->fq8f, 0, sizeof(uint64_t) * 8 * 128) != hipSuccess ||
                    hipMemset(h->fsgt, 0, sizeof(uint64_t)) != hipSuccess))
            rc = fail(HOARD_ERR_HIP, "hipMemset one-launch layer exchange words");
    }
    if (!rc && hipMemset(h->counters, 0, T * sizeof(unsigned)) != hipSuccess)
        rc = fail(HOARD_ERR_HIP, "hipMemset counters");
    if (!rc && c.pool_k > 0) {
        h->lru.reset(c.n_layer, c.n_expert, c.pool_k);
        h->pool_ids_cap = std::max(pool_ids_cap(c), c.n_used);
        h->pool_slots.assign(h->pool_ids_cap, 0);
        h->pool_miss.assign(h->pool_ids_cap, 0);
        h->pool_mids.assign(h->pool_ids_cap, 0);
        h->pool_mj.assign(h->pool_ids_cap, 0);
        if (hipHostMalloc((void **)&h->pin_sel, sizeof(int32_t) * c.n_used, hipHostMallocDefault) != hipSuccess)
            rc = fail(HOARD_ERR_OOM, "pinned selection buffer");
        rc = rc ? rc : dev_alloc((void **)&h->slot_ids, sizeof(int32_t) * c.n_used);
        for (int i = 0; !rc && i < kUpStreams - 1; ++i)
            if (hipStreamCreateWithFlags(&h->copy_x[i], hipStreamNonBlocking) != hipSuccess)
                rc = fail(HOARD_ERR_HIP, "upload stream");
    }
    if (!rc) rc = persistent_setup(h);
    rc = rc ? rc : dev_alloc((void **)&h->nab_stats, sizeof(unsigned) * (c.n_expert + 1));
    if (!rc) {
        // this device's copy of the allocation-free entry point's fixed scratch
        const hipError_t e = hoard::noalloc_setup(h->device);
        if (e != hipSuccess) rc = fail(HOARD_ERR_HIP, "fixed scratch set-up: %s", hipGetErrorString(e));
    }
    // the zeroed counters and exchange words are in place before any launch, on
    // whatever stream the caller uses (a non-blocking stream does not wait for
    // the null stream's memsets)
    if (!rc && hipDeviceSynchronize() != hipSuccess) rc = fail(HOARD_ERR_HIP, "device synchronisation after set-up");
    if (rc) {
        delete h;
        return rc;
    }
    *out = h;
    return HOARD_OK;
}

void hoard_moe_destroy(hoard_moe *h) {
    if (!h) return;
    hipSetDevice(h->device);
    hipDeviceSynchronize();
    delete h;
}

int hoard_moe_set_layer_weights(hoard_moe *h, int layer, const hoard_layer_weights *w) {
    if (!h || !w) return fail(HOARD_ERR_INVALID, "null argument");
    if (layer < 0 || layer >= h->cfg.n_layer) return fail(HOARD_ERR_INVALID, "layer %d out of range", layer);
    const hoard_moe_cfg &c = h->cfg;
    if (!w->router || (!h->store && (!w->gate || !w->up || !w->down))) return fail(HOARD_ERR_INVALID, "missing tensor");
    if (!quant_type_ok(w->gate_type) || !quant_type_ok(w->up_type) || !quant_type_ok(w->down_type))
        return fail(HOARD_ERR_UNSUPPORTED, "expert types %d/%d/%d: Q3_K (11), Q4_K (12), Q5_K (13) and Q6_K (14) are taken", w->gate_type,
                    w->up_type, w->down_type);
    const bool sh = c.n_ff_shexp > 0;
    if (sh) {
        if (!w->sh_gate || !w->sh_up || !w->sh_down || !w->sh_gate_inp)
            return fail(HOARD_ERR_INVALID, "n_ff_shexp > 0 but shared-expert tensors missing");
        if (!quant_type_ok(w->sh_gate_type) || !quant_type_ok(w->sh_up_type) || !quant_type_ok(w->sh_down_type))
            return fail(HOARD_ERR_UNSUPPORTED, "shared expert types %d/%d/%d", w->sh_gate_type, w->sh_up_type,
                        w->sh_down_type);
    }
    HIP_TRY(hipSetDevice(h->device));
    h->weights_set = true;
    Layer &L = h->layers[layer];
    hoard_moe::free_layer(L);
    L.gate_type = w->gate_type;
    L.up_type = w->up_type;
    L.down_type = w->down_type;
    L.gbytes = L.gstride = mat_bytes(L.gate_type, c.n_ff, c.n_embd);
    L.ubytes = L.ustride = mat_bytes(L.up_type, c.n_ff, c.n_embd);
    L.dbytes = L.dstride = mat_bytes(L.down_type, c.n_embd, c.n_ff);
    const size_t E = (size_t)c.n_expert;
    int rc = 0;
    const size_t rb = (size_t)c.n_expert * c.n_embd * sizeof(float);
    rc = rc ? rc : upload((void **)&L.router, w->router, rb, rb);
    if (c.pool_k == 0) {
        rc = rc ? rc : upload((void **)&L.gate, w->gate, E * L.gstride, E * L.gstride + kTailPad);
        rc = rc ? rc : upload((void **)&L.up, w->up, E * L.ustride, E * L.ustride + kTailPad);
        rc = rc ? rc : upload((void **)&L.down, w->down, E * L.dstride, E * L.dstride + kTailPad);
    } else {
        const size_t K = (size_t)c.pool_k, rec = L.gbytes + L.ubytes + L.dbytes;
        rc = rc ? rc : dev_alloc((void **)&L.slots, K * rec + kTailPad);
        if (!rc) {
            L.gate = L.slots;
            L.up = L.slots + L.gbytes;
            L.down = L.slots + L.gbytes + L.ubytes;
            L.gstride = L.ustride = L.dstride = rec;
        }
        if (h->store) {  // expert bytes come from the storage tier on each miss
            const hoard_store_layer &sl = h->store->layers[(size_t)layer];
            if (!rc && (sl.stride[0] != L.gbytes || sl.stride[1] != L.ubytes || sl.stride[2] != L.dbytes))
                rc = fail(HOARD_ERR_INVALID, "layer %d: the store's expert strides %llu/%llu/%llu are not the %zu/%zu/%zu "
                          "bytes of types %d/%d/%d", layer, (unsigned long long)sl.stride[0],
                          (unsigned long long)sl.stride[1], (unsigned long long)sl.stride[2], L.gbytes, L.ubytes,
                          L.dbytes, L.gate_type, L.up_type, L.down_type);
        } else if (!rc && hipHostMalloc((void **)&L.host_experts, E * rec, hipHostMallocDefault) != hipSuccess) {
            L.host_experts = nullptr;
            (void)hipGetLastError();
            rc = fail(HOARD_ERR_OOM, "hipHostMalloc(%zu) for the expert masters", E * rec);
        }
        if (!rc && !h->store) {
            const uint8_t *g = static_cast<const uint8_t *>(w->gate), *u = static_cast<const uint8_t *>(w->up),
                          *d = static_cast<const uint8_t *>(w->down);
            for (size_t e = 0; e < E; ++e) {
                uint8_t *r = L.host_experts + e * rec;
                std::memcpy(r, g + e * L.gbytes, L.gbytes);
                std::memcpy(r + L.gbytes, u + e * L.ubytes, L.ubytes);
                std::memcpy(r + L.gbytes + L.ubytes, d + e * L.dbytes, L.dbytes);
            }
        }
        if (!rc && hipHostMalloc((void **)&L.slot_stage, sizeof(int32_t) * h->pool_ids_cap, hipHostMallocDefault) != hipSuccess)
            rc = fail(HOARD_ERR_OOM, "pinned slot staging");
        for (int i = 0; !rc && i < kUpStreams; ++i)
            if (hipEventCreateWithFlags(&L.copied[i], hipEventDisableTiming) != hipSuccess) rc = fail(HOARD_ERR_HIP, "pool events");
        if (!rc && (
                    hipEventCreateWithFlags(&L.last_use, hipEventDisableTiming) != hipSuccess ||
                    hipEventCreateWithFlags(&L.staged, hipEventDisableTiming) != hipSuccess))
            rc = fail(HOARD_ERR_HIP, "pool events");
        if (!rc) h->lru.reset_layer(layer);  // the slots no longer hold this layer's experts
    }
    if (sh && !rc) {
        L.sh_gate_type = w->sh_gate_type;
        L.sh_up_type = w->sh_up_type;
        L.sh_down_type = w->sh_down_type;
        const size_t sg = mat_bytes(L.sh_gate_type, c.n_ff_shexp, c.n_embd);
        const size_t su = mat_bytes(L.sh_up_type, c.n_ff_shexp, c.n_embd);
        const size_t sd = mat_bytes(L.sh_down_type, c.n_embd, c.n_ff_shexp);
        rc = rc ? rc : upload((void **)&L.sh_gate, w->sh_gate, sg, sg + kTailPad);
        rc = rc ? rc : upload((void **)&L.sh_up, w->sh_up, su, su + kTailPad);
        rc = rc ? rc : upload((void **)&L.sh_down, w->sh_down, sd, sd + kTailPad);
        rc = rc ? rc : upload((void **)&L.sh_gate_inp, w->sh_gate_inp, c.n_embd * sizeof(float), c.n_embd * sizeof(float));
    }
    if (rc) {
        hoard_moe::free_layer(L);
        return rc;
    }
    L.loaded = true;
    if (h->d_table) {
        // the one-launch decode reads each layer's pointers from this table
        const hoard::DecodeLayer t{L.router,  L.gate,      L.up,      L.down,        L.gstride,
                                   L.ustride, L.dstride,   L.gate_type, L.up_type,   L.down_type,
                                   L.sh_gate, L.sh_up,     L.sh_down, L.sh_gate_inp};
        HIP_TRY(hipMemcpy(h->d_table + layer, &t, sizeof t, hipMemcpyHostToDevice));
    }
    return HOARD_OK;
}

int hoard_moe_route(hoard_moe *h, int layer, const float *fx_dev, int32_t *sel_dev, float *w_dev,
                    void *stream) {
    int rc = check_layer(h, layer);
    if (rc) return rc;
    if (!fx_dev || !sel_dev || !w_dev) return fail(HOARD_ERR_INVALID, "null device pointer");
    return run_route(h, h->layers[layer], fx_dev, 0, 0.0f, sel_dev, w_dev, (hipStream_t)stream);
}

int hoard_moe_ffn_combine(hoard_moe *h, int layer, const float *fx_dev, const int32_t *ids_dev,
                          const float *w_dev, const float *res_dev, float *out_dev, void *stream) {
    int rc = check_layer(h, layer);
    if (rc) return rc;
    if (!fx_dev || !ids_dev || !w_dev || !res_dev || !out_dev) return fail(HOARD_ERR_INVALID, "null device pointer");
    rc = run_ffn(h, h->layers[layer], fx_dev, ids_dev, w_dev, res_dev, out_dev, (hipStream_t)stream);
    if (rc) return rc;
    return pool_mark_use(h, layer, (hipStream_t)stream);
}

int hoard_moe_layer(hoard_moe *h, int layer, const float *fx_dev, const float *res_dev, float *out_dev,
                    int32_t *sel_dev, float *w_dev, void *stream) {
    int rc = check_layer(h, layer);
    if (rc) return rc;
    if (!fx_dev || !res_dev || !out_dev) return fail(HOARD_ERR_INVALID, "null device pointer");
    int32_t *sel = sel_dev ? sel_dev : h->sel;
    float *w = w_dev ? w_dev : h->wsel;
    const Layer &L = h->layers[layer];
    hipStream_t s = (hipStream_t)stream;
    bool fused = false;
    rc = run_layer_fused(h, L, fx_dev, 0, 0.0f, res_dev, out_dev, sel, w, s, &fused);
    if (rc || fused) return rc;
    rc = run_route(h, L, fx_dev, 0, 0.0f, sel, w, s);
    if (rc) return rc;
    const int32_t *ids = sel;
    if (h->cfg.pool_k > 0) {
        rc = pool_after_route(h, layer, sel, h->slot_ids, s);
        if (rc) return rc;
        ids = h->slot_ids;
    }
    rc = run_ffn(h, L, fx_dev, ids, w, res_dev, out_dev, s);
    if (rc) return rc;
    return pool_mark_use(h, layer, s);
}

int hoard_moe_decode(hoard_moe *h, int layer_begin, int layer_end, float *x_dev, float eps, void *stream) {
    if (!h || !x_dev) return fail(HOARD_ERR_INVALID, "null argument");
    if (layer_begin < 0 || layer_end > h->cfg.n_layer || layer_begin > layer_end)
        return fail(HOARD_ERR_INVALID, "layer range [%d,%d)", layer_begin, layer_end);
    hipStream_t s = (hipStream_t)stream;
    for (int l = layer_begin; l < layer_end; ++l) {
        int rc = check_layer(h, l);
        if (rc) return rc;
    }
    // Forced mode takes the range as one launch (or fails); automatic mode splits
    // it into runs of layers with the same quant types (Q4_K_M files mix Q4_K and
    // Q6_K down experts from layer to layer) and decodes each run with the
    // one-launch kernel where it applies, else layer by layer.
    if (h->persistent_mode == 2) {
        bool used = false;
        int rc0 = persistent_decode(h, layer_begin, layer_end, x_dev, eps, s, &used);
        if (rc0 || used) return rc0;
        return decode_layers(h, layer_begin, layer_end, x_dev, eps, s);
    }
    for (int r0 = layer_begin; r0 < layer_end;) {
        int r1 = r0 + 1;
        while (r1 < layer_end && same_types(h->layers[r0], h->layers[r1])) ++r1;
        bool used = false;
        int rc = persistent_decode(h, r0, r1, x_dev, eps, s, &used);
        if (!rc && !used) rc = decode_layers(h, r0, r1, x_dev, eps, s);
        if (rc) return rc;
        r0 = r1;
    }
    return HOARD_OK;
}

int hoard_moe_pool_ensure(hoard_moe *h, int layer, const int32_t *sel_host, int32_t *slot_host,
                          int32_t *slot_dev, void *stream, void *copy_stream) {
    int rc = check_layer(h, layer);
    if (rc) return rc;
    if (h->cfg.pool_k == 0) return fail(HOARD_ERR_STATE, "handle has no slot pool (pool_k == 0)");
    if (!sel_host || (!slot_host && !slot_dev)) return fail(HOARD_ERR_INVALID, "null argument");
    return pool_ensure(h, layer, sel_host, h->cfg.n_used, false, slot_host, slot_dev, (hipStream_t)stream,
                       copy_stream ? (hipStream_t)copy_stream : (hipStream_t)stream);
}

int hoard_moe_attach_store(hoard_moe *h, hoard_store *st) {
    if (!h || !st) return fail(HOARD_ERR_INVALID, "null argument");
    const hoard_moe_cfg &c = h->cfg;
    if (c.pool_k == 0) return fail(HOARD_ERR_STATE, "a store serves a slot pool: the handle has pool_k == 0");
    if (h->weights_set) return fail(HOARD_ERR_STATE, "attach the store before setting layer weights");
    if (h->store) return fail(HOARD_ERR_STATE, "a store is attached already");
    const hoard::Store &s = st->s;
    if (s.n_layer != c.n_layer || s.n_expert != c.n_expert)
        return fail(HOARD_ERR_INVALID, "store of %d layers x %d experts for a stage of %d x %d", s.n_layer, s.n_expert,
                    c.n_layer, c.n_expert);
    if (s.cap < c.n_used) return fail(HOARD_ERR_INVALID, "RAM tier of %d experts below n_used %d", s.cap, c.n_used);
    h->store = &st->s;
    return HOARD_OK;
}

}  // extern "C"

namespace {

// Scratch of the batched entry points for batches of up to T tokens: the
// byte size of every buffer and the layout of the int arrays.  The verify-sized
// path (M <= 32) keeps 32 token places per expert group; the prefill-sized one
// keeps the pairs sorted by expert.
struct BatchedLayout {
    int T, Ts, umax, umax_s, max_units;
    size_t q8x, q8h, hbuf, ybuf, n_ints, hist, counters;  // bytes (n_ints: ints)
    size_t o_slot_of, o_uexp, o_ucount, o_utok, o_uslot, o_ysrc, o_bad, o_goff, o_ptok, o_pslot, o_pexp, o_units, o_q8hd,
        o_nunits, o_sgl;
};

BatchedLayout batched_layout(const hoard_moe_cfg &c, int T) {
    BatchedLayout L{};
    // a shared expert is one more expert id, paired with every token at slot n_used
    const int sh = c.n_ff_shexp > 0 ? 1 : 0;
    const int k = c.n_used + sh, E = c.n_expert + sh;  // the slots of a pool never outnumber the experts
    const int nb = c.n_embd / 256, nbh = c.n_ff / 256;
    L.T = T;
    L.Ts = std::min(T, hoard::kBatchedMaxTokens);
    L.umax_s = std::min(E, L.Ts * k);
    L.umax = std::min(E, T * k);
    L.max_units = hoard::prefill_max_units(T, k, E);
    const size_t pairs_s = (size_t)L.umax_s * hoard::kBatchedMaxTokens, pairs = (size_t)T * k;
    L.q8x = (size_t)T * nb * hoard::kQ8LBytes;
    L.q8h = std::max(pairs_s, pairs) * nbh * hoard::kQ8LBytes;
    L.hbuf = std::max(pairs_s, pairs) * c.n_ff * sizeof(float);
    L.ybuf = pairs * c.n_embd * sizeof(float);
    size_t o = 1;  // [0]: the group count
    auto take = [&](size_t n) {  // every array starts 16-byte aligned (read in 16-byte words)
        const size_t r = (o + 3) & ~(size_t)3;
        o = r + n;
        return r;
    };
    L.o_slot_of = take(E);
    L.o_uexp = take(L.umax);
    L.o_ucount = take(L.umax);
    L.o_utok = take(pairs_s);
    L.o_uslot = take(pairs_s);
    L.o_ysrc = take(pairs);
    L.o_bad = take(T);
    L.o_goff = take(L.umax);
    L.o_ptok = take(pairs);
    L.o_pslot = take(pairs);
    L.o_pexp = take(pairs);
    L.o_units = take((size_t)4 * L.max_units);
    L.o_q8hd = take((size_t)4 * pairs);  // floats
    L.o_nunits = take(1);
    L.o_sgl = take(T);  // floats
    L.n_ints = o;
    L.hist = sizeof(unsigned) * E;
    L.counters = sizeof(unsigned) * hoard::kBatchedCounters;
    return L;
}

// Points the args' scratch at buffers laid out by L: q8x, q8h, hbuf, ybuf and
// the int arrays, histogram and counters.
void bind_batched(hoard::BatchedArgs &a, const BatchedLayout &L, uint8_t *q8x, uint8_t *q8h, float *hbuf, float *ybuf,
                  int *ints, unsigned *hist, unsigned *counters) {
    a.q8x = q8x;
    a.q8h = q8h;
    a.hbuf = hbuf;
    a.ybuf = ybuf;
    a.n_unique = ints;
    a.slot_of = ints + L.o_slot_of;
    a.uexp = ints + L.o_uexp;
    a.ucount = ints + L.o_ucount;
    a.utok = ints + L.o_utok;
    a.uslot = ints + L.o_uslot;
    a.goff = ints + L.o_goff;
    a.ptok = ints + L.o_ptok;
    a.pslot = ints + L.o_pslot;
    a.pexp = ints + L.o_pexp;
    a.units = ints + L.o_units;
    a.q8hd = reinterpret_cast<float *>(ints + L.o_q8hd);
    a.n_units = ints + L.o_nunits;
    a.max_units = hoard::prefill_max_units(a.M, a.k + a.sh, a.n_ids + a.sh);
    a.sgl = reinterpret_cast<float *>(ints + L.o_sgl);
    a.hist = hist;
    a.counters = counters;
}

// Checks common to the batched entry points, and their arguments but the
// selection and the scratch: the shapes and types the kernels are built for,
// 16-byte aligned fx, res, out and weights.
int batched_check(hoard_moe *h, int layer, int M, const float *fx_dev, const float *res_dev, float *out_dev,
                  bool pooled_ok, int max_m, hoard::BatchedArgs *out) {
    int rc = check_layer(h, layer);
    if (rc) return rc;
    const hoard_moe_cfg &c = h->cfg;
    if (!fx_dev || !res_dev || !out_dev) return fail(HOARD_ERR_INVALID, "null device pointer");
    if (M < 1 || M > c.max_tokens || M > max_m)
        return fail(HOARD_ERR_INVALID, "M %d outside 1..min(max_tokens %d, %d)", M, c.max_tokens, max_m);
    if (c.pool_k > 0 && !pooled_ok)
        return fail(HOARD_ERR_UNSUPPORTED, "batched routing needs every expert resident (pool_k 0)");
    const Layer &L = h->layers[layer];
    const bool sh = c.n_ff_shexp > 0;
    if (sh) {
        // the shared expert runs as one more expert of the routed experts' kernels
        // (a Q6_K shared down beside Q5_K routed rows, Qwen3.5's types, runs in the
        // same down launch)
        const bool q5q6 = L.down_type == HOARD_TYPE_Q5_K && L.sh_down_type == HOARD_TYPE_Q6_K;
        if (c.n_ff_shexp != c.n_ff || L.sh_gate_type != L.gate_type || L.sh_up_type != L.up_type ||
            (L.sh_down_type != L.down_type && !(q5q6 && c.n_ff == 512)))
            return fail(HOARD_ERR_UNSUPPORTED,
                        "batched path: the shared expert (n_ff %d, types %d/%d/%d) must match the routed experts'",
                        c.n_ff_shexp, L.sh_gate_type, L.sh_up_type, L.sh_down_type);
        if (c.n_used + 1 > 16) return fail(HOARD_ERR_UNSUPPORTED, "batched path: n_used %d with a shared expert", c.n_used);
        if (((uintptr_t)L.sh_gate | (uintptr_t)L.sh_up | (uintptr_t)L.sh_down) & 15)
            return fail(HOARD_ERR_UNSUPPORTED, "batched path: shared expert matrices must be 16-byte aligned");
        if (!L.sh_gate_inp) return fail(HOARD_ERR_STATE, "shared expert gate row missing");
    }
    if (L.up_type != L.gate_type || !hoard::batched_shape_compiled(L.gate_type, c.n_embd, L.down_type, c.n_ff))
        return fail(HOARD_ERR_UNSUPPORTED, "batched path: types %d/%d/%d with n_embd %d, n_ff %d not built",
                    L.gate_type, L.up_type, L.down_type, c.n_embd, c.n_ff);
    if ((((uintptr_t)fx_dev | (uintptr_t)res_dev | (uintptr_t)out_dev) & 15) != 0)
        return fail(HOARD_ERR_INVALID, "fx, res and out must be 16-byte aligned");
    // the weight tiles are copied to LDS in 16-byte units
    if (((uintptr_t)L.gate | (uintptr_t)L.up | (uintptr_t)L.down | (uintptr_t)L.gstride | (uintptr_t)L.ustride |
         (uintptr_t)L.dstride) & 15)
        return fail(HOARD_ERR_UNSUPPORTED, "batched path: expert matrices must be 16-byte aligned");
    hoard::BatchedArgs a{};
    a.M = M;
    a.n_embd = c.n_embd;
    a.n_ff = c.n_ff;
    a.E = c.n_expert;
    a.k = c.n_used;
    a.n_ids = c.pool_k > 0 ? c.pool_k : c.n_expert;
    a.gu_type = L.gate_type;
    a.d_type = L.down_type;
    a.fx = fx_dev;
    a.res = res_dev;
    a.out = out_dev;
    a.router = L.router;
    a.renorm = c.renorm;
    a.logits = h->logits;
    a.gate = L.gate;
    a.up = L.up;
    a.down = L.down;
    a.gstride = L.gstride;
    a.ustride = L.ustride;
    a.dstride = L.dstride;
    a.sh = sh ? 1 : 0;
    a.sh_d_type = sh ? L.sh_down_type : L.down_type;
    a.sh_gate = L.sh_gate;
    a.sh_up = L.sh_up;
    a.sh_down = L.sh_down;
    a.sh_gate_inp = L.sh_gate_inp;
    *out = a;
    return HOARD_OK;
}

// batched_check, and the handle's scratch, allocated on first use for
// max_tokens (at most kBatchedMaxTokensLarge) tokens.
int batched_setup(hoard_moe *h, int layer, int M, const float *fx_dev, const float *res_dev, float *out_dev,
                  bool pooled_ok, hoard::BatchedArgs *out) {
    if (int rc = batched_check(h, layer, M, fx_dev, res_dev, out_dev, pooled_ok, hoard::kBatchedMaxTokensLarge, out))
        return rc;
    const hoard_moe_cfg &c = h->cfg;
    const BatchedLayout L = batched_layout(c, std::min(c.max_tokens, hoard::kBatchedMaxTokensLarge));
    if (!h->b_q8x) {
        int rc = 0;
        rc = rc ? rc : dev_alloc((void **)&h->b_q8x, L.q8x);
        rc = rc ? rc : dev_alloc((void **)&h->b_q8h, L.q8h);
        rc = rc ? rc : dev_alloc((void **)&h->b_h, L.hbuf);
        rc = rc ? rc : dev_alloc((void **)&h->b_y, L.ybuf);
        rc = rc ? rc : dev_alloc((void **)&h->b_ints, sizeof(int) * L.n_ints);
        rc = rc ? rc : dev_alloc((void **)&h->b_hist, L.hist);
        rc = rc ? rc : dev_alloc((void **)&h->b_counters, L.counters);
        if (rc) return rc;
        HIP_TRY(hipMemset(h->b_counters, 0, L.counters));
        // the counters must read zero before the first launch, which may go to a
        // non-blocking stream that does not wait for work on the null stream
        HIP_TRY(hipDeviceSynchronize());
    }
    bind_batched(*out, L, h->b_q8x, h->b_q8h, h->b_h, h->b_y, h->b_ints, h->b_hist, h->b_counters);
    out->ysrc = out->bad = nullptr;
    h->b_layout_ysrc = h->b_ints + L.o_ysrc;
    h->b_layout_bad = h->b_ints + L.o_bad;
    return HOARD_OK;
}

}  // namespace

extern "C" {

int hoard_moe_forward_batched(hoard_moe *h, int layer, int M, const float *fx_dev, const float *res_dev,
                              float *out_dev, int32_t *sel_dev, float *w_dev, void *stream) {
    hoard::BatchedArgs a;
    if (int rc = batched_setup(h, layer, M, fx_dev, res_dev, out_dev, false, &a)) return rc;
    hipStream_t s = (hipStream_t)stream;
    a.sel = sel_dev ? sel_dev : h->sel;
    a.wsel = w_dev ? w_dev : h->wsel;
    hipError_t e;
    {
        KernelMark mark(h, HOARD_KERNEL_BATCHED, s);
        e = hoard::launch_batched(a, s);
    }
    if (e != hipSuccess) return fail(HOARD_ERR_HIP, "batched launch: %s", hipGetErrorString(e));
    h->stats.tokens += (uint64_t)M;
    h->hist_pending = true;
    h->hist_src = a.hist;
    h->nu_src = a.n_unique;
    return HOARD_OK;
}

// The batched forward with its per-call scratch in the library's fixed device
// array (noalloc.hip) instead of buffers allocated on first use: the call
// allocates nothing.  Layout: the route counters (zeroed at set-up, left zero
// by every launch), then the logits, Q8_K(fx), Q8_K(h), h, y, the int arrays
// and the histogram, each 256-byte aligned.
int hoard_moe_forward_batched_noalloc(hoard_moe *h, int layer, int M, const float *fx_dev, const float *res_dev,
                                      float *out_dev, int32_t *sel_dev, float *w_dev, void *stream) {
    hoard::BatchedArgs a;
    if (int rc = batched_check(h, layer, M, fx_dev, res_dev, out_dev, false, hoard::kNoAllocMaxTokens, &a)) return rc;
    uint8_t *base = hoard::noalloc_scratch(h->device);
    if (!base) return fail(HOARD_ERR_STATE, "no fixed scratch set up for device %d", h->device);
    const hoard_moe_cfg &c = h->cfg;
    const BatchedLayout L = batched_layout(c, M);
    size_t o = hoard::kNoAllocCounterBytes;
    auto take = [&](size_t n) {
        const size_t r = o;
        o += (n + 255) & ~(size_t)255;
        return r;
    };
    const size_t o_log = take(sizeof(float) * M * c.n_expert), o_q8x = take(L.q8x), o_q8h = take(L.q8h);
    const size_t o_h = take(L.hbuf), o_y = take(L.ybuf), o_ints = take(sizeof(int) * L.n_ints), o_hist = take(L.hist);
    if (o > hoard::noalloc_scratch_bytes())
        return fail(HOARD_ERR_INVALID, "M %d of this shape needs %zu bytes of scratch; the fixed array holds %zu", M, o,
                    hoard::noalloc_scratch_bytes());
    a.logits = reinterpret_cast<float *>(base + o_log);
    bind_batched(a, L, base + o_q8x, base + o_q8h, reinterpret_cast<float *>(base + o_h),
                 reinterpret_cast<float *>(base + o_y), reinterpret_cast<int *>(base + o_ints),
                 reinterpret_cast<unsigned *>(base + o_hist), reinterpret_cast<unsigned *>(base));
    a.ysrc = a.bad = nullptr;
    a.sel = sel_dev ? sel_dev : h->sel;
    a.wsel = w_dev ? w_dev : h->wsel;
    hipStream_t s = (hipStream_t)stream;
    hipError_t e;
    {
        KernelMark mark(h, HOARD_KERNEL_BATCHED, s);
        e = hoard::launch_batched(a, s);
    }
    if (e != hipSuccess) return fail(HOARD_ERR_HIP, "batched launch: %s", hipGetErrorString(e));
    // the histogram and group count move out of the array every call on this GPU
    // shares into the handle's own words, so hoard_moe_get_stats reports this call
    // whatever later calls of other handles leave in the array
    const int E = c.n_expert;
    HIP_TRY(hipMemcpyAsync(h->nab_stats, a.hist, sizeof(unsigned) * E, hipMemcpyDeviceToDevice, s));
    HIP_TRY(hipMemcpyAsync(h->nab_stats + E, a.n_unique, sizeof(int), hipMemcpyDeviceToDevice, s));
    h->stats.tokens += (uint64_t)M;
    h->hist_pending = true;
    h->hist_src = h->nab_stats;
    h->nu_src = reinterpret_cast<const int *>(h->nab_stats + E);
    return HOARD_OK;
}

int hoard_moe_ffn_combine_batched(hoard_moe *h, int layer, int M, const float *fx_dev, const int32_t *ids_dev,
                                  const float *w_dev, const float *res_dev, float *out_dev, void *stream) {
    if (!ids_dev || !w_dev) return fail(HOARD_ERR_INVALID, "null device pointer");
    hoard::BatchedArgs a;
    if (int rc = batched_setup(h, layer, M, fx_dev, res_dev, out_dev, true, &a)) return rc;
    hipStream_t s = (hipStream_t)stream;
    a.sel = const_cast<int32_t *>(ids_dev);
    a.wsel = const_cast<float *>(w_dev);
    a.ysrc = h->b_layout_ysrc;
    a.bad = h->b_layout_bad;
    hipError_t e;
    {
        KernelMark mark(h, HOARD_KERNEL_BATCHED, s);
        e = hoard::launch_batched_ids(a, s);
    }
    if (e != hipSuccess) return fail(HOARD_ERR_HIP, "batched launch: %s", hipGetErrorString(e));
    h->stats.tokens += (uint64_t)M;
    return pool_mark_use(h, layer, s);
}

int hoard_moe_pool_ensure_batched(hoard_moe *h, int layer, int n, const int32_t *sel_host, int32_t *slot_host,
                                  int32_t *slot_dev, void *stream, void *copy_stream) {
    int rc = check_layer(h, layer);
    if (rc) return rc;
    const hoard_moe_cfg &c = h->cfg;
    if (c.pool_k == 0) return fail(HOARD_ERR_STATE, "handle has no slot pool (pool_k == 0)");
    if (h->pool_naive) return fail(HOARD_ERR_STATE, "naive pool mode places one token's experts; not a batch");
    if (!sel_host || (!slot_host && !slot_dev)) return fail(HOARD_ERR_INVALID, "null argument");
    if (n < 1 || n > h->pool_ids_cap)
        return fail(HOARD_ERR_INVALID, "%d ids outside 1..min(max_tokens, %d) * n_used (%d)", n,
                    hoard::kBatchedMaxTokensLarge, h->pool_ids_cap);
    // every distinct expert of the batch must hold a slot at once
    std::vector<int32_t> u(sel_host, sel_host + n);
    std::sort(u.begin(), u.end());
    const int distinct = (int)(std::unique(u.begin(), u.end()) - u.begin());
    if (distinct > c.pool_k)
        return fail(HOARD_ERR_INVALID, "%d distinct experts for %d slots", distinct, c.pool_k);
    return pool_ensure(h, layer, sel_host, n, true, slot_host, slot_dev, (hipStream_t)stream,
                       copy_stream ? (hipStream_t)copy_stream : (hipStream_t)stream);
}

int hoard_moe_get_stats(hoard_moe *h, hoard_moe_stats *out) {
    if (!h || !out) return fail(HOARD_ERR_INVALID, "null argument");
    if (h->hist_pending) {
        // histogram of the last batched call (synchronises with the device)
        const int E = h->cfg.n_expert;
        std::vector<unsigned> hist(E);
        int nu = 0;
        HIP_TRY(hipSetDevice(h->device));
        HIP_TRY(hipDeviceSynchronize());
        HIP_TRY(hipMemcpy(hist.data(), h->hist_src, sizeof(unsigned) * E, hipMemcpyDeviceToHost));
        HIP_TRY(hipMemcpy(&nu, h->nu_src, sizeof(int), hipMemcpyDeviceToHost));
        for (int e = 0; e < E && e < 1024; ++e) h->stats.expert_hist[e] = hist[e];
        h->stats.last_unique = nu;
        h->hist_pending = false;
    }
    *out = h->stats;
    return HOARD_OK;
}

int hoard_moe_reset_stats(hoard_moe *h) {
    if (!h) return fail(HOARD_ERR_INVALID, "null handle");
    h->stats = hoard_moe_stats{};
    return HOARD_OK;
}

int hoard_moe_set_option(hoard_moe *h, int option, int value) {
    if (!h) return fail(HOARD_ERR_INVALID, "null handle");
    switch (option) {
    case HOARD_OPT_PERSISTENT_DECODE:
        if (value < 0 || value > 2) return fail(HOARD_ERR_INVALID, "persistent decode mode %d", value);
        if (value == 2 && !h->persistent_shape_ok)
            return fail(HOARD_ERR_UNSUPPORTED, "shape or device does not admit the persistent decode");
        h->persistent_mode = value;
        return HOARD_OK;
    case HOARD_OPT_DECODE_KERNEL:
        if (value < 0 || value > 2) return fail(HOARD_ERR_INVALID, "decode kernel %d", value);
        if ((value == 1 && !h->xcd_ok) || (value == 2 && !h->spread_ok))
            return fail(HOARD_ERR_UNSUPPORTED, "decode kernel %d does not take this shape or device", value);
        h->decode_kernel = value;
        return HOARD_OK;
    case HOARD_OPT_LAYER_KERNELS:
        if (value < 0 || value > 1) return fail(HOARD_ERR_INVALID, "layer kernels flag %d", value);
        h->layer_kernels = value != 0;
        return HOARD_OK;
    case HOARD_OPT_DECODE_LAUNCH:
        if (value < 0 || value > 1) return fail(HOARD_ERR_INVALID, "decode launch %d", value);
        h->coop_launch = value == 0;
        return HOARD_OK;
    case HOARD_OPT_LAYER_FUSED:
        if (value < 0 || value > 1) return fail(HOARD_ERR_INVALID, "fused layer flag %d", value);
        h->layer_fused = value != 0;
        return HOARD_OK;
    case HOARD_OPT_WAIT_LIMIT_US:
        if (value < 0) return fail(HOARD_ERR_INVALID, "wait limit %d us", value);
        h->wait_ticks = 100ll * value;  // the device wall clock runs at 100 MHz
        return HOARD_OK;
    case HOARD_OPT_FAIL_UPLOAD:
        if (value < 0) return fail(HOARD_ERR_INVALID, "fail-upload countdown %d", value);
        h->fail_upload = value;
        return HOARD_OK;
    case HOARD_OPT_POOL_NAIVE:
        if (value < 0 || value > 1) return fail(HOARD_ERR_INVALID, "pool naive flag %d", value);
        if (value && h->cfg.pool_k > 0) {
            // naive mode places request j in slot j; residency restarts empty
            for (int l = 0; l < h->cfg.n_layer; ++l) h->lru.reset_layer(l);
        }
        h->pool_naive = value != 0;
        return HOARD_OK;
    default:
        return fail(HOARD_ERR_INVALID, "unknown option %d", option);
    }
}

int hoard_moe_get_option(hoard_moe *h, int option, int *value) {
    if (!h || !value) return fail(HOARD_ERR_INVALID, "null argument");
    switch (option) {
    case HOARD_OPT_PERSISTENT_DECODE:
        *value = h->persistent_mode;
        return HOARD_OK;
    case HOARD_OPT_PERSISTENT_AVAILABLE:
        *value = h->persistent_shape_ok ? 1 : 0;
        return HOARD_OK;
    case HOARD_OPT_POOL_NAIVE:
        *value = h->pool_naive ? 1 : 0;
        return HOARD_OK;
    case HOARD_OPT_DECODE_KERNEL:
        *value = h->decode_kernel;
        return HOARD_OK;
    case HOARD_OPT_LAYER_KERNELS:
        *value = h->layer_kernels ? 1 : 0;
        return HOARD_OK;
    case HOARD_OPT_DECODE_LAUNCH:
        *value = h->coop_launch ? 0 : 1;
        return HOARD_OK;
    case HOARD_OPT_DECODE_KERNELS_AVAILABLE:
        *value = (h->xcd_ok ? 1 : 0) | (h->spread_ok ? 2 : 0);
        return HOARD_OK;
    case HOARD_OPT_WAIT_LIMIT_US:
        *value = (int)(h->wait_ticks / 100);
        return HOARD_OK;
    case HOARD_OPT_LAYER_FUSED:
        *value = h->layer_fused ? 1 : 0;
        return HOARD_OK;
    case HOARD_OPT_FAIL_UPLOAD:
        *value = h->fail_upload;
        return HOARD_OK;
    default:
        return fail(HOARD_ERR_INVALID, "unknown option %d", option);
    }
}

int hoard_moe_sync_check(hoard_moe *h) {
    if (!h) return fail(HOARD_ERR_INVALID, "null handle");
    HIP_TRY(hipSetDevice(h->device));
    HIP_TRY(hipDeviceSynchronize());
    if (h->fctr) {
        int err = 0;
        int *ep = reinterpret_cast<int *>(h->fctr + hoard::kFusedCounterWords);
        HIP_TRY(hipMemcpy(&err, ep, sizeof(int), hipMemcpyDeviceToHost));
        if (err) {
            HIP_TRY(hipMemset(ep, 0, sizeof(int)));
            return fail(HOARD_ERR_HIP, "one-launch layer: a cross-workgroup wait timed out (output poisoned)");
        }
    }
    if (h->perr) {
        int err = 0;
        HIP_TRY(hipMemcpy(&err, h->perr, sizeof(int), hipMemcpyDeviceToHost));
        if (err) {
            HIP_TRY(hipMemset(h->perr, 0, sizeof(int)));
            return fail(HOARD_ERR_HIP, "persistent decode: a cross-workgroup wait timed out (output poisoned)");
        }
    }
    return HOARD_OK;
}

int hoard_moe_phase_trace(hoard_moe *h, int enable) {
    if (!h) return fail(HOARD_ERR_INVALID, "null handle");
    h->tracing = enable != 0;
    return HOARD_OK;
}

int hoard_moe_phase_trace_read(hoard_moe *h, uint64_t *out, size_t max_words, int *n_layers) {
    if (!h || !out || !n_layers) return fail(HOARD_ERR_INVALID, "null argument");
    *n_layers = 0;
    if (!h->ptrace || h->trace_last <= 0) return HOARD_OK;
    const size_t words = (size_t)h->trace_last * 256 * hoard::kTracePhases;
    if (max_words < words) return fail(HOARD_ERR_INVALID, "trace needs %zu words", words);
    HIP_TRY(hipSetDevice(h->device));
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(hipMemcpy(out, h->ptrace, words * sizeof(uint64_t), hipMemcpyDeviceToHost));
    *n_layers = h->trace_last;
    return HOARD_OK;
}

int hoard_moe_fused_trace_read(hoard_moe *h, uint64_t *out, size_t max_words, size_t *n_words) {
    if (!h || !out || !n_words) return fail(HOARD_ERR_INVALID, "null argument");
    *n_words = 0;
    if (!h->ftrace || !h->ftrace_last) return HOARD_OK;
    if (max_words < h->ftrace_last) return fail(HOARD_ERR_INVALID, "trace needs %zu words", h->ftrace_last);
    HIP_TRY(hipSetDevice(h->device));
    HIP_TRY(hipDeviceSynchronize());
    HIP_TRY(hipMemcpy(out, h->ftrace, h->ftrace_last * sizeof(uint64_t), hipMemcpyDeviceToHost));
    *n_words = h->ftrace_last;
    return HOARD_OK;
}

int hoard_moe_profile(hoard_moe *h, int enable) {
    if (!h) return fail(HOARD_ERR_INVALID, "null handle");
    h->profiling = enable != 0;
    return HOARD_OK;
}

int hoard_moe_profile_read(hoard_moe *h, hoard_moe_kernel_times *out) {
    if (!h || !out) return fail(HOARD_ERR_INVALID, "null argument");
    std::memset(out, 0, sizeof *out);
    HIP_TRY(hipSetDevice(h->device));
    if (!h->marks.empty()) HIP_TRY(hipEventSynchronize(h->marks.back().b));
    for (auto &m : h->marks) {
        float ms = 0.0f;
        HIP_TRY(hipEventElapsedTime(&ms, m.a, m.b));
        out->launches[m.kind] += 1;
        out->total_ms[m.kind] += ms;
        h->event_pool.push_back(m.a);
        h->event_pool.push_back(m.b);
    }
    h->marks.clear();
    return HOARD_OK;
}

}  // extern "C"
