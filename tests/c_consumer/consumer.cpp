// A C++ engine-side consumer of the library, written against include/*.h only:
// what hoard's own loader and per-layer loop (src/run_moe_stream.cpp,
// src/run_specloop.cpp) would call, with device memory from plain HIP.
//
//   consumer host   <model.gguf>                 GGUF reader, storage tier and LRU replay, no device
//   consumer layer  <model.gguf> <in> <out>      one resident layer: in = fx|res (f32), out = y|sel|w
//   consumer verify <model.gguf> <in> <out> K    M tokens through a K-slot pool streamed from the file:
//                                                in = M x (fx|res), out = M x (y|sel|w)
//
// Every call's status is checked; a failure prints hoard_last_error() and exits 1.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "hoard_gguf.h"
#include "hoard_moe.h"
#include "hoard_store.h"

#define CHECK(call)                                                                 \
    do {                                                                            \
        const int rc_ = (call);                                                     \
        if (rc_ != HOARD_OK) {                                                      \
            std::fprintf(stderr, "%s -> %d: %s\n", #call, rc_, hoard_last_error()); \
            std::exit(1);                                                           \
        }                                                                           \
    } while (0)
#define HIP_CHECK(call)                                                             \
    do {                                                                            \
        const hipError_t e_ = (call);                                               \
        if (e_ != hipSuccess) {                                                     \
            std::fprintf(stderr, "%s failed: %s\n", #call, hipGetErrorString(e_)); \
            std::exit(1);                                                           \
        }                                                                           \
    } while (0)

static std::vector<float> read_f32(const char *path) {
    FILE *f = std::fopen(path, "rb");
    if (!f) std::exit(2);
    std::fseek(f, 0, SEEK_END);
    const long n = std::ftell(f);
    std::fseek(f, 0, SEEK_SET);
    std::vector<float> v((size_t)n / 4);
    if (std::fread(v.data(), 4, v.size(), f) != v.size()) std::exit(2);
    std::fclose(f);
    return v;
}

static void write_all(const char *path, const void *p, size_t n, bool append) {
    FILE *f = std::fopen(path, append ? "ab" : "wb");
    if (!f || std::fwrite(p, 1, n, f) != n) std::exit(2);
    std::fclose(f);
}

// Expert bytes straight from the file, as the reference's HostExperts::read does.
static std::vector<unsigned char> file_bytes(const char *path, uint64_t off, size_t n) {
    std::vector<unsigned char> b(n);
    FILE *f = std::fopen(path, "rb");
    if (!f || std::fseek(f, (long)off, SEEK_SET) || std::fread(b.data(), 1, n, f) != n) std::exit(2);
    std::fclose(f);
    return b;
}

static int host_mode(const char *path) {
    hoard_gguf *g = nullptr;
    CHECK(hoard_gguf_open(path, &g));
    hoard_moe_cfg cfg{};
    CHECK(hoard_gguf_moe_cfg(g, &cfg));
    std::vector<hoard_store_layer> ext((size_t)cfg.n_layer);
    CHECK(hoard_gguf_store_layers(g, ext.data(), cfg.n_layer));
    hoard_store_cfg sc{4, 3 * cfg.n_used, 1, 0};
    hoard_store *st = nullptr;
    CHECK(hoard_store_open(path, cfg.n_layer, cfg.n_expert, ext.data(), &sc, &st));
    int checked = 0;
    for (int l = 0; l < cfg.n_layer; ++l) {
        const int32_t ids[3] = {0, cfg.n_expert - 1, cfg.n_expert / 2};
        const void *parts[9];
        CHECK(hoard_store_fetch(st, l, 3, ids, parts, nullptr));
        for (int j = 0; j < 3; ++j)
            for (int i = 0; i < 3; ++i) {
                const auto want = file_bytes(path, ext[(size_t)l].off[i] + (uint64_t)ids[j] * ext[(size_t)l].stride[i],
                                             (size_t)ext[(size_t)l].stride[i]);
                if (std::memcmp(parts[3 * j + i], want.data(), want.size())) {
                    std::fprintf(stderr, "layer %d expert %d tensor %d differs\n", l, ids[j], i);
                    return 1;
                }
                ++checked;
            }
    }
    hoard_store_stats ss{};
    CHECK(hoard_store_get_stats(st, &ss));
    hoard_store_close(st);
    // the slot pool's bookkeeping, replayed on the host
    hoard_slot_lru *lru = nullptr;
    CHECK(hoard_slot_lru_create(1, cfg.n_expert, cfg.n_used, 2, &lru));
    const int32_t seq[4] = {3, 3, 1, 3};
    int32_t slots[4];
    uint8_t miss[4];
    CHECK(hoard_slot_lru_access(lru, 0, seq, 4, slots, miss));
    hoard_slot_lru_destroy(lru);
    std::printf("host ok arch=%s layers=%d embd=%d experts=%d/%d ff=%d shexp=%d renorm=%d eps=%g checked=%d "
                "reads=%llu misses=%d%d%d%d\n",
                hoard_gguf_arch(g), cfg.n_layer, cfg.n_embd, cfg.n_used, cfg.n_expert, cfg.n_ff, cfg.n_ff_shexp,
                cfg.renorm, (double)hoard_gguf_rms_eps(g), checked, (unsigned long long)ss.file_reads, miss[0],
                miss[1], miss[2], miss[3]);
    hoard_gguf_close(g);
    return 0;
}

static int device_mode(const char *path, const char *in, const char *out, int pool_k) {
    hoard_gguf *g = nullptr;
    CHECK(hoard_gguf_open(path, &g));
    hoard_moe_cfg cfg{};
    CHECK(hoard_gguf_moe_cfg(g, &cfg));
    const std::vector<float> x = read_f32(in);
    const int D = cfg.n_embd, k = cfg.n_used, M = (int)(x.size() / (2 * (size_t)D));
    cfg.pool_k = pool_k;
    cfg.max_tokens = M;
    hoard_moe *moe = nullptr;
    CHECK(hoard_moe_create(&cfg, &moe));
    hoard_store *st = nullptr;
    if (pool_k > 0) {  // experts stay in the file; the pool's misses read them through the store
        std::vector<hoard_store_layer> ext((size_t)cfg.n_layer);
        CHECK(hoard_gguf_store_layers(g, ext.data(), cfg.n_layer));
        hoard_store_cfg sc{8, 64, 1, 1};
        CHECK(hoard_store_open(path, cfg.n_layer, cfg.n_expert, ext.data(), &sc, &st));
        CHECK(hoard_moe_attach_store(moe, st));
    }
    for (int l = 0; l < cfg.n_layer; ++l) {
        hoard_layer_weights w{};
        CHECK(hoard_gguf_layer_weights(g, l, &w));
        CHECK(hoard_moe_set_layer_weights(moe, l, &w));
    }
    hoard_gguf_close(g);  // the stage holds its copies
    float *fx = nullptr, *res = nullptr, *y = nullptr, *wsel = nullptr;
    int32_t *sel = nullptr, *slots = nullptr;
    HIP_CHECK(hipMalloc(&fx, sizeof(float) * M * D));
    HIP_CHECK(hipMalloc(&res, sizeof(float) * M * D));
    HIP_CHECK(hipMalloc(&y, sizeof(float) * M * D));
    HIP_CHECK(hipMalloc(&sel, sizeof(int32_t) * M * k));
    HIP_CHECK(hipMalloc(&wsel, sizeof(float) * M * k));
    HIP_CHECK(hipMalloc(&slots, sizeof(int32_t) * M * k));
    for (int t = 0; t < M; ++t) {
        HIP_CHECK(hipMemcpy(fx + (size_t)t * D, x.data() + (size_t)t * 2 * D, sizeof(float) * D, hipMemcpyHostToDevice));
        HIP_CHECK(hipMemcpy(res + (size_t)t * D, x.data() + (size_t)t * 2 * D + D, sizeof(float) * D,
                            hipMemcpyHostToDevice));
    }
    hipStream_t s;
    HIP_CHECK(hipStreamCreate(&s));
    if (pool_k == 0) {
        for (int t = 0; t < M; ++t)
            CHECK(hoard_moe_layer(moe, 0, fx + (size_t)t * D, res + (size_t)t * D, y + (size_t)t * D,
                                  sel + (size_t)t * k, wsel + (size_t)t * k, s));
    } else {
        // the verify step: route every token, ensure the batch's experts id after id,
        // then the grouped products over the slots
        for (int t = 0; t < M; ++t)
            CHECK(hoard_moe_route(moe, 0, fx + (size_t)t * D, sel + (size_t)t * k, wsel + (size_t)t * k, s));
        std::vector<int32_t> sel_h((size_t)M * k), slot_h((size_t)M * k);
        HIP_CHECK(hipMemcpyAsync(sel_h.data(), sel, sizeof(int32_t) * M * k, hipMemcpyDeviceToHost, s));
        HIP_CHECK(hipStreamSynchronize(s));
        CHECK(hoard_moe_pool_ensure_batched(moe, 0, M * k, sel_h.data(), slot_h.data(), slots, s, nullptr));
        CHECK(hoard_moe_ffn_combine_batched(moe, 0, M, fx, slots, wsel, res, y, s));
    }
    HIP_CHECK(hipStreamSynchronize(s));
    std::vector<float> yh((size_t)M * D), wh((size_t)M * k);
    std::vector<int32_t> sh((size_t)M * k);
    HIP_CHECK(hipMemcpy(yh.data(), y, sizeof(float) * M * D, hipMemcpyDeviceToHost));
    HIP_CHECK(hipMemcpy(sh.data(), sel, sizeof(int32_t) * M * k, hipMemcpyDeviceToHost));
    HIP_CHECK(hipMemcpy(wh.data(), wsel, sizeof(float) * M * k, hipMemcpyDeviceToHost));
    for (int t = 0; t < M; ++t) {
        write_all(out, yh.data() + (size_t)t * D, sizeof(float) * D, t > 0);
        write_all(out, sh.data() + (size_t)t * k, sizeof(int32_t) * k, true);
        write_all(out, wh.data() + (size_t)t * k, sizeof(float) * k, true);
    }
    hoard_moe_stats stats{};
    CHECK(hoard_moe_get_stats(moe, &stats));
    hoard_moe_destroy(moe);
    if (st) hoard_store_close(st);
    std::printf("%s ok tokens=%d pool_reqs=%llu misses=%llu\n", pool_k ? "verify" : "layer", M,
                (unsigned long long)stats.reqs, (unsigned long long)stats.misses);
    return 0;
}

int main(int argc, char **argv) {
    if (argc >= 3 && !std::strcmp(argv[1], "host")) return host_mode(argv[2]);
    if (argc >= 5 && !std::strcmp(argv[1], "layer")) return device_mode(argv[2], argv[3], argv[4], 0);
    if (argc >= 6 && !std::strcmp(argv[1], "verify")) return device_mode(argv[2], argv[3], argv[4], std::atoi(argv[5]));
    std::fprintf(stderr, "usage: consumer host|layer|verify <model.gguf> [in out [K]]\n");
    return 2;
}
