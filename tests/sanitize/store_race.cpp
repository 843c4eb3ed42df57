// Reader-pool stress for the sanitizers: many fetch batches of a small
// synthetic file through the RAM tier of hoard_store (store.cpp), each
// expert's bytes compared with the file.  Built by tests/test_store_sanitizers.py
// twice, with -fsanitize=thread and with -fsanitize=address,undefined, from
// store.cpp alone: the HIP calls the store makes only for a pinned RAM tier
// are stubbed here and abort if reached (this driver uses pageable memory).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "hoard_store.h"

static std::string g_err;
extern "C" int hoard_set_error(int code, const char *msg) {
    g_err = msg ? msg : "";
    return code;
}

static hipError_t unreachable(const char *what) {
    std::fprintf(stderr, "unexpected HIP call %s\n", what);
    std::abort();
}
hipError_t hipEventSynchronize(hipEvent_t) { return unreachable("hipEventSynchronize"); }
hipError_t hipEventDestroy(hipEvent_t) { return unreachable("hipEventDestroy"); }
hipError_t hipHostFree(void *) { return unreachable("hipHostFree"); }
hipError_t hipHostMalloc(void **, size_t, unsigned int) { return unreachable("hipHostMalloc"); }
hipError_t hipGetLastError(void) { return hipSuccess; }
hipError_t hipEventCreateWithFlags(hipEvent_t *, unsigned) { return unreachable("hipEventCreateWithFlags"); }
hipError_t hipEventRecord(hipEvent_t, hipStream_t) { return unreachable("hipEventRecord"); }

int main(int argc, char **argv) {
    if (argc < 3) {
        std::fprintf(stderr, "usage: %s FILE ITERATIONS [readers]\n", argv[0]);
        return 2;
    }
    const char *path = argv[1];
    const int iters = std::atoi(argv[2]);
    const int readers = argc > 3 ? std::atoi(argv[3]) : 8;
    std::mt19937_64 rng(1);
    std::vector<unsigned char> data(4 << 20);
    for (auto &b : data) b = (unsigned char)rng();
    FILE *f = std::fopen(path, "wb");
    if (!f || std::fwrite(data.data(), 1, data.size(), f) != data.size()) return 2;
    std::fclose(f);
    // two layers of 40 experts, gate/up/down parts at their own offsets and strides
    hoard_store_layer L[2] = {{{100, 300000, 700000}, {3000, 3000, 5000}},
                              {{1500000, 2000000, 2600000}, {4100, 4100, 9000}}};
    hoard_store_cfg cfg{readers, 6, 1, 0};  // a 6-expert RAM tier: most fetches evict
    hoard_store *s = nullptr;
    if (hoard_store_open(path, 2, 40, L, &cfg, &s)) {
        std::printf("open: %s\n", g_err.c_str());
        return 1;
    }
    int bad = 0;
    for (int it = 0; it < iters; ++it) {
        const int l = (int)(rng() % 2), n = 1 + (int)(rng() % 6);
        int32_t ids[6];
        for (int j = 0; j < n; ++j) {
            int32_t v = (int32_t)(rng() % 40);
            for (int q = 0; q < j; ++q)
                if (ids[q] == v) v = (v + 1) % 40, q = -1;  // distinct ids
            ids[j] = v;
        }
        const void *parts[18];
        if (hoard_store_fetch(s, l, n, ids, parts, nullptr)) {
            std::printf("fetch: %s\n", g_err.c_str());
            return 1;
        }
        for (int j = 0; j < n; ++j)
            for (int i = 0; i < 3; ++i)
                if (std::memcmp(parts[3 * j + i], data.data() + L[l].off[i] + (size_t)ids[j] * L[l].stride[i],
                                L[l].stride[i]))
                    ++bad;
    }
    hoard_store_stats st;
    hoard_store_get_stats(s, &st);
    std::printf("bad %d requests %llu hits %llu reads %llu direct %d\n", bad, (unsigned long long)st.requests,
                (unsigned long long)st.ram_hits, (unsigned long long)st.file_reads, st.direct);
    hoard_store_close(s);
    std::remove(path);
    return bad != 0;
}
