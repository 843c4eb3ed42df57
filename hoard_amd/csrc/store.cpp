// Storage tier: expert bytes read from the model file into a bounded RAM tier
// (include/hoard_store.h).
//
// Counterpart of the reference's DirectIO pool, RamTier and the fetch phases
// that drive them (src/run_qwen35.cpp:99-148, :596-627): phase A classifies
// each requested expert as a RAM hit or a miss and reserves the least recently
// used entry for every miss; phase B runs all the batch's reads in parallel.
// Here the readers are Linux threads issuing pread() on an O_DIRECT file
// descriptor (FILE_FLAG_NO_BUFFERING there), each read the 4 KiB-aligned
// superset of one tensor slice straight into the RAM entry; the entry keeps
// the offset of the wanted bytes within it.
#include <errno.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <chrono>
#include <cstdlib>
#include <cstring>

#include "host_error.h"
#include "store_impl.h"

using hoard::fail_fmt;

namespace hoard {

namespace {

constexpr uint64_t kAlign = 4096;          // O_DIRECT buffer, offset and length alignment
constexpr size_t kChunkBytes = 256u << 20;  // RAM-tier memory is allocated this much at a time

uint64_t round_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

// Reads up to len bytes at off; stops early only at the end of the file.
// With O_DIRECT a short read that is not a whole number of blocks ends the
// file (a further read at an unaligned offset would be refused).
ssize_t pread_all(int fd, uint8_t *p, size_t len, uint64_t off, bool direct) {
    size_t done = 0;
    while (done < len) {
        const ssize_t r = pread(fd, p + done, len - done, (off_t)(off + done));
        if (r < 0) {
            if (errno == EINTR) continue;
            return -1;
        }
        if (r == 0) break;
        done += (size_t)r;
        if (direct && (r % (ssize_t)kAlign)) break;
    }
    return (ssize_t)done;
}

}  // namespace

ReaderPool::ReaderPool(int fd_direct, int fd_buffered, int n_threads)
    : fd_direct_(fd_direct), fd_buffered_(fd_buffered) {
    for (int i = 0; i < n_threads; ++i) threads_.emplace_back([this] { worker(); });
}

ReaderPool::~ReaderPool() {
    {
        std::lock_guard<std::mutex> lk(m_);
        stop_ = true;
    }
    cv_work_.notify_all();
    for (auto &t : threads_) t.join();
}

namespace {

// A 4 KiB-aligned buffer of the calling thread, grown to at least `bytes`.
uint8_t *bounce_buffer(size_t bytes) {
    thread_local struct Buf {
        uint8_t *p = nullptr;
        size_t n = 0;
        ~Buf() { std::free(p); }
    } b;
    if (b.n < bytes) {
        std::free(b.p);
        b.p = nullptr;
        b.n = 0;
        void *q = nullptr;
        if (posix_memalign(&q, kAlign, bytes) != 0) return nullptr;
        b.p = static_cast<uint8_t *>(q);
        b.n = bytes;
    }
    return b.p;
}

}  // namespace

int ReaderPool::read_one(const ReadJob &j) {
    if (fd_direct_ >= 0 && !direct_refused_) {
        uint8_t *dst = j.dst;
        if (bounce_ && !(dst = bounce_buffer(j.asize))) return HOARD_ERR_OOM;
        ssize_t got = pread_all(fd_direct_, dst, j.asize, j.aoff, true);
        if (got < 0 && errno == EFAULT && dst == j.dst) {  // the destination is driver-pinned memory
            bounce_ = true;  // (several readers may find this at once: each retries its own read)
            if (!(dst = bounce_buffer(j.asize))) return HOARD_ERR_OOM;
            got = pread_all(fd_direct_, dst, j.asize, j.aoff, true);
        }
        if (got >= (ssize_t)(j.head + j.rsize)) {
            if (dst != j.dst) std::memcpy(j.dst + j.head, dst + j.head, j.rsize);
            return 0;
        }
        if (got >= 0) return HOARD_ERR_IO;  // the file ends before the tensor does
        if (errno != EINVAL && errno != EOPNOTSUPP) {
            errno_ = errno;
            return HOARD_ERR_IO;
        }
        direct_refused_ = true;  // this file system takes no O_DIRECT reads: go buffered
    }
    const ssize_t got = pread_all(fd_buffered_, j.dst + j.head, j.rsize, j.aoff + j.head, false);
    if (got < 0) errno_ = errno;
    return got == (ssize_t)j.rsize ? 0 : HOARD_ERR_IO;
}

void ReaderPool::drain() {
    for (;;) {
        const std::vector<ReadJob> *b;
        size_t i;
        {
            std::lock_guard<std::mutex> lk(m_);
            if (!batch_ || next_ >= batch_->size()) return;
            b = batch_;
            i = next_++;
        }
        const int rc = read_one((*b)[i]);
        std::lock_guard<std::mutex> lk(m_);
        if (rc && !error_) error_ = rc;
        if (++done_ == b->size()) cv_done_.notify_all();
    }
}

void ReaderPool::worker() {
    uint64_t seen = 0;
    for (;;) {
        {
            std::unique_lock<std::mutex> lk(m_);
            cv_work_.wait(lk, [&] { return stop_ || gen_ != seen; });
            if (stop_) return;
            seen = gen_;
        }
        drain();
    }
}

int ReaderPool::run(const std::vector<ReadJob> &jobs) {
    if (jobs.empty()) return 0;
    if (threads_.empty() || jobs.size() == 1) {
        for (const ReadJob &j : jobs)
            if (int rc = read_one(j)) return rc;
        return 0;
    }
    {
        std::lock_guard<std::mutex> lk(m_);
        batch_ = &jobs;
        next_ = done_ = 0;
        error_ = 0;
        ++gen_;
    }
    cv_work_.notify_all();
    drain();  // the calling thread is one of the readers
    std::unique_lock<std::mutex> lk(m_);
    cv_done_.wait(lk, [&] { return done_ == jobs.size(); });
    batch_ = nullptr;
    return error_;
}

Store::~Store() {
    for (size_t i = 0; i < fence_.size(); ++i)
        if (fence_[i]) {
            if (fenced_[i]) (void)hipEventSynchronize(fence_[i]);  // no copy out of the tier is left running
            (void)hipEventDestroy(fence_[i]);
        }
    for (uint8_t *c : chunks_)
        if (c) {
            if (pinned_)
                (void)hipHostFree(c);
            else
                std::free(c);
        }
    delete pool_;
    if (fd_direct_ >= 0) close(fd_direct_);
    if (fd_buffered_ >= 0) close(fd_buffered_);
}

int Store::open(const char *path, int nl, int ne, const hoard_store_layer *ls, const hoard_store_cfg &cfg) {
    if (nl <= 0 || ne <= 0 || !ls) return fail_fmt(HOARD_ERR_INVALID, "store of %d layers x %d experts", nl, ne);
    fd_buffered_ = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd_buffered_ < 0) return fail_fmt(HOARD_ERR_IO, "%s: cannot open (%s)", path, strerror(errno));
    struct stat st;
    if (fstat(fd_buffered_, &st) != 0) return fail_fmt(HOARD_ERR_IO, "%s: cannot stat", path);
    const uint64_t fsize = (uint64_t)st.st_size;
    uint64_t max_stride[3] = {0, 0, 0};
    for (int l = 0; l < nl; ++l)
        for (int i = 0; i < 3; ++i) {
            const uint64_t sb = ls[l].stride[i];
            if (sb == 0 || sb >= (1ull << 31) || ls[l].off[i] > fsize || sb * (uint64_t)ne > fsize - ls[l].off[i])
                return fail_fmt(HOARD_ERR_INVALID, "%s: layer %d tensor %d (offset %llu, %d x %llu B) is not inside the "
                                "file (%llu B)", path, l, i, (unsigned long long)ls[l].off[i], ne,
                                (unsigned long long)sb, (unsigned long long)fsize);
            if (sb > max_stride[i]) max_stride[i] = sb;
        }
    n_layer = nl;
    n_expert = ne;
    layers.assign(ls, ls + nl);
    const int64_t total = (int64_t)nl * ne;
    cap = cfg.ram_experts <= 0 || cfg.ram_experts > total ? (int)total : cfg.ram_experts;
    if (cfg.direct) fd_direct_ = ::open(path, O_RDONLY | O_CLOEXEC | O_DIRECT);  // -1: buffered reads only
    for (int i = 0; i < 3; ++i) region_[i] = (size_t)round_up(max_stride[i] + kAlign - 1, kAlign);
    slot_bytes_ = region_[0] + region_[1] + region_[2];
    per_chunk_ = (int)(kChunkBytes / slot_bytes_);
    if (per_chunk_ < 1) per_chunk_ = 1;
    if (per_chunk_ > cap) per_chunk_ = cap;
    chunks_.assign((size_t)((cap + per_chunk_ - 1) / per_chunk_), nullptr);
    pinned_ = cfg.pinned != 0;
    slot2key_.assign((size_t)cap, -1);
    head_.assign((size_t)cap * 3, 0);
    pos_.resize((size_t)cap);
    for (int s = 0; s < cap; ++s) pos_[(size_t)s] = lru_.insert(lru_.end(), s);
    fence_.assign((size_t)cap, nullptr);
    fenced_.assign((size_t)cap, 0);
    key2slot_.reserve((size_t)cap * 2);
    const int readers = cfg.readers > 0 ? cfg.readers : 8;
    pool_ = new ReaderPool(fd_direct_, fd_buffered_, readers - 1);
    stats = hoard_store_stats{};
    stats.direct = fd_direct_ >= 0;
    stats.ram_experts = cap;
    return HOARD_OK;
}

uint8_t *Store::slot_base(int slot) {
    return chunks_[(size_t)(slot / per_chunk_)] + (size_t)(slot % per_chunk_) * slot_bytes_;
}

int Store::ensure_chunk(int slot) {
    const int c = slot / per_chunk_;
    if (chunks_[(size_t)c]) return HOARD_OK;
    const int n = per_chunk_ < cap - c * per_chunk_ ? per_chunk_ : cap - c * per_chunk_;
    const size_t bytes = (size_t)n * slot_bytes_;
    void *p = nullptr;
    if (pinned_) {
        if (hipHostMalloc(&p, bytes, hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            return fail_fmt(HOARD_ERR_OOM, "hipHostMalloc(%zu) for the RAM tier", bytes);
        }
    } else if (posix_memalign(&p, kAlign, bytes) != 0) {
        return fail_fmt(HOARD_ERR_OOM, "%zu bytes for the RAM tier", bytes);
    }
    chunks_[(size_t)c] = static_cast<uint8_t *>(p);
    return HOARD_OK;
}

int Store::fetch(int layer, int n, const int32_t *ids, StoreEntry *out, uint8_t *hit) {
    if (layer < 0 || layer >= n_layer) return fail_fmt(HOARD_ERR_INVALID, "layer %d outside 0..%d", layer, n_layer - 1);
    if (n < 0 || n > cap) return fail_fmt(HOARD_ERR_INVALID, "%d experts asked of a RAM tier of %d", n, cap);
    for (int j = 0; j < n; ++j)
        if (ids[j] < 0 || ids[j] >= n_expert) return fail_fmt(HOARD_ERR_INVALID, "expert id %d out of range", ids[j]);
    const hoard_store_layer &L = layers[(size_t)layer];
    std::vector<ReadJob> jobs;
    std::vector<int> filled;
    // On any failure the entries this call reserved hold no data: unmap them and
    // put them at the back, so no later call takes them for hits.
    auto drop_filled = [&]() {
        for (int slot : filled) {
            if (slot2key_[(size_t)slot] >= 0) key2slot_.erase(slot2key_[(size_t)slot]);
            slot2key_[(size_t)slot] = -1;
            lru_.splice(lru_.end(), lru_, pos_[(size_t)slot]);
        }
    };
    for (int j = 0; j < n; ++j) {
        const int64_t key = (int64_t)layer * n_expert + ids[j];
        stats.requests += 1;
        auto it = key2slot_.find(key);
        int slot;
        if (it != key2slot_.end()) {
            slot = it->second;
            lru_.splice(lru_.begin(), lru_, pos_[(size_t)slot]);
            stats.ram_hits += 1;
            if (hit) hit[j] = 1;
        } else {
            slot = lru_.back();
            lru_.splice(lru_.begin(), lru_, pos_[(size_t)slot]);
            if (slot2key_[(size_t)slot] >= 0) key2slot_.erase(slot2key_[(size_t)slot]);
            slot2key_[(size_t)slot] = key;
            key2slot_[key] = slot;
            filled.push_back(slot);
            if (fenced_[(size_t)slot]) {  // a device copy out of this entry may still run
                if (hipEventSynchronize(fence_[(size_t)slot]) != hipSuccess) {
                    drop_filled();
                    return fail_fmt(HOARD_ERR_HIP, "waiting on a copy out of the RAM tier");
                }
                fenced_[(size_t)slot] = 0;
            }
            if (int rc = ensure_chunk(slot)) {
                drop_filled();
                return rc;
            }
            uint8_t *base = slot_base(slot);
            size_t roff = 0;
            for (int i = 0; i < 3; ++i) {
                const uint64_t off = L.off[i] + (uint64_t)ids[j] * L.stride[i];
                const uint32_t head = (uint32_t)(off & (kAlign - 1));
                const uint32_t rsize = (uint32_t)L.stride[i];
                jobs.push_back(ReadJob{base + roff, off - head, (uint32_t)round_up(head + (uint64_t)rsize, kAlign), head,
                                       rsize});
                head_[(size_t)slot * 3 + i] = head;
                roff += region_[i];
                stats.bytes_read += rsize;
            }
            stats.file_reads += 1;
            if (hit) hit[j] = 0;
        }
        uint8_t *base = slot_base(slot);
        size_t roff = 0;
        out[j].slot = slot;
        for (int i = 0; i < 3; ++i) {
            out[j].part[i] = base + roff + head_[(size_t)slot * 3 + i];
            roff += region_[i];
        }
    }
    if (!jobs.empty()) {
        const auto t0 = std::chrono::steady_clock::now();
        const int rc = pool_->run(jobs);
        stats.read_ns += (uint64_t)std::chrono::duration_cast<std::chrono::nanoseconds>(
                             std::chrono::steady_clock::now() - t0).count();
        stats.direct = pool_->direct() ? (pool_->bounced() ? 2 : 1) : 0;
        if (rc) {  // drop the entries this batch was filling
            drop_filled();
            const int en = pool_->last_errno();
            if (en) return fail_fmt(HOARD_ERR_IO, "expert read of layer %d failed: %s", layer, strerror(en));
            return fail_fmt(HOARD_ERR_IO, "expert read of layer %d failed: the file is shorter than its tensor "
                            "table says", layer);
        }
    }
    return HOARD_OK;
}

int Store::fence(int slot, hipStream_t stream) {
    if (slot < 0 || slot >= cap) return fail_fmt(HOARD_ERR_INVALID, "RAM slot %d", slot);
    hipEvent_t &ev = fence_[(size_t)slot];
    if (!ev && hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
        ev = nullptr;
        return fail_fmt(HOARD_ERR_HIP, "event for the RAM tier");
    }
    if (hipEventRecord(ev, stream) != hipSuccess) return fail_fmt(HOARD_ERR_HIP, "recording a RAM-tier fence");
    fenced_[(size_t)slot] = 1;
    return HOARD_OK;
}

}  // namespace hoard

extern "C" {

int hoard_store_open(const char *path, int n_layer, int n_expert, const hoard_store_layer *layers,
                     const hoard_store_cfg *cfg, hoard_store **out) {
    if (!path || !cfg || !out) return fail_fmt(HOARD_ERR_INVALID, "null argument");
    *out = nullptr;
    hoard_store *s = new hoard_store;
    if (int rc = s->s.open(path, n_layer, n_expert, layers, *cfg)) {
        delete s;
        return rc;
    }
    *out = s;
    return HOARD_OK;
}

void hoard_store_close(hoard_store *s) { delete s; }

int hoard_store_fetch(hoard_store *s, int layer, int n, const int32_t *ids, const void **parts, uint8_t *hit) {
    if (!s || (n > 0 && (!ids || !parts))) return fail_fmt(HOARD_ERR_INVALID, "null argument");
    std::vector<hoard::StoreEntry> e((size_t)(n > 0 ? n : 0));
    if (int rc = s->s.fetch(layer, n, ids, e.data(), hit)) return rc;
    for (int j = 0; j < n; ++j)
        for (int i = 0; i < 3; ++i) parts[3 * j + i] = e[(size_t)j].part[i];
    return HOARD_OK;
}

int hoard_store_get_stats(const hoard_store *s, hoard_store_stats *out) {
    if (!s || !out) return fail_fmt(HOARD_ERR_INVALID, "null argument");
    *out = s->s.stats;
    return HOARD_OK;
}

int hoard_store_reset_stats(hoard_store *s) {
    if (!s) return fail_fmt(HOARD_ERR_INVALID, "null argument");
    const int32_t d = s->s.stats.direct, c = s->s.stats.ram_experts;
    s->s.stats = hoard_store_stats{};
    s->s.stats.direct = d;
    s->s.stats.ram_experts = c;
    return HOARD_OK;
}

}  // extern "C"
