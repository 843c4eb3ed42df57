// Storage tier internals shared by store.cpp (the C ABI) and moe.cpp (the
// slot pool's miss path): the RAM tier of expert records and the reader pool.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <condition_variable>
#include <cstdint>
#include <list>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "hoard_store.h"

namespace hoard {

// One read: the aligned byte range [aoff, aoff + asize) of the file into dst;
// the wanted bytes are dst[head, head + rsize).
struct ReadJob {
    uint8_t *dst;
    uint64_t aoff;
    uint32_t asize, head, rsize;
};

// A persistent pool of reader threads.  run() hands a batch to the readers,
// takes a share of it on the calling thread and returns once every job is
// done, with the first error (0 when all succeeded).
class ReaderPool {
public:
    ReaderPool(int fd_direct, int fd_buffered, int n_threads);
    ~ReaderPool();
    int run(const std::vector<ReadJob> &jobs);
    bool direct() const { return fd_direct_ >= 0 && !direct_refused_; }
    bool bounced() const { return bounce_; }
    int last_errno() const { return errno_; }

private:
    void worker();
    void drain();
    int read_one(const ReadJob &j);

    int fd_direct_, fd_buffered_;
    std::atomic<bool> direct_refused_{false};
    // O_DIRECT reads cannot target memory the GPU driver pinned (EFAULT): they go
    // through a per-thread aligned buffer and a copy instead
    std::atomic<bool> bounce_{false};
    std::atomic<int> errno_{0};
    std::vector<std::thread> threads_;
    std::mutex m_;
    std::condition_variable cv_work_, cv_done_;
    const std::vector<ReadJob> *batch_ = nullptr;
    size_t next_ = 0, done_ = 0;
    uint64_t gen_ = 0;
    int error_ = 0;
    bool stop_ = false;
};

// A RAM-tier entry handed out by Store::fetch.
struct StoreEntry {
    int slot;               // RAM-tier slot (for fence())
    const uint8_t *part[3]; // gate, up, down bytes of the expert
};

class Store {
public:
    ~Store();
    int open(const char *path, int n_layer, int n_expert, const hoard_store_layer *layers,
             const hoard_store_cfg &cfg);
    // RAM-tier lookup and file reads for ids[0..n) of `layer` (see hoard_store_fetch).
    int fetch(int layer, int n, const int32_t *ids, StoreEntry *out, uint8_t *hit);
    // Records on `stream` the end of a device copy out of RAM slot `slot`; the
    // slot is not refilled before that point is reached.
    int fence(int slot, hipStream_t stream);

    int n_layer = 0, n_expert = 0, cap = 0;
    std::vector<hoard_store_layer> layers;
    hoard_store_stats stats{};

private:
    uint8_t *slot_base(int slot);
    int ensure_chunk(int slot);

    int fd_direct_ = -1, fd_buffered_ = -1;
    ReaderPool *pool_ = nullptr;
    bool pinned_ = false;
    size_t region_[3] = {0, 0, 0}, slot_bytes_ = 0;
    int per_chunk_ = 1;
    std::vector<uint8_t *> chunks_;
    std::unordered_map<int64_t, int> key2slot_;
    std::vector<int64_t> slot2key_;
    std::vector<uint32_t> head_;  // [slot][3]
    std::list<int> lru_;          // front = most recent
    std::vector<std::list<int>::iterator> pos_;
    std::vector<hipEvent_t> fence_;
    std::vector<char> fenced_;
};

}  // namespace hoard

struct hoard_store {
    hoard::Store s;
};
