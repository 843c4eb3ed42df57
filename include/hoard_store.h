/* hoard_store.h -- the storage tier under the expert slot pool: expert bytes
 * streamed from the model file through a bounded RAM tier.
 *
 * The counterpart of the reference's DirectIO worker pool and RamTier
 * (src/run_qwen35.cpp:99-148, src/run_moe_stream.cpp:79-115) and of the
 * three-tier fetch that uses them (src/run_qwen35.cpp:596-638): a request for
 * expert e of layer l is a RAM-tier hit, or it evicts the least recently used
 * RAM entry (one LRU over all layers, key l * n_expert + e) and reads the
 * expert's gate, up and down bytes from the file.  The reads of one request
 * batch run in parallel, `readers` at a time, each as one read of the
 * 4 KiB-aligned superset of the bytes straight into the RAM entry (O_DIRECT,
 * bypassing the page cache, where the file system allows it; the reference's
 * FILE_FLAG_NO_BUFFERING).
 *
 * On Linux the readers are a persistent pool of threads issuing pread();
 * the RAM tier lives in pinned host memory (hipHostMalloc) when `pinned` is
 * set, so uploads into HBM slots are DMA transfers straight from it.
 *
 * Attached to a hoard_moe handle with a slot pool (hoard_moe_attach_store),
 * the store replaces the pinned copy of every expert that such a handle keeps
 * otherwise: a slot miss is served from the RAM tier or the file.
 *
 * Every call returns HOARD_OK or a negative HOARD_ERR_* with
 * hoard_last_error() set.  A store belongs to one host thread.
 */
#ifndef HOARD_STORE_H
#define HOARD_STORE_H

#include <stddef.h>
#include <stdint.h>

#include "hoard_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct hoard_store hoard_store;

/* Where one layer's experts lie in the file: the data of its gate, up and
   down expert tensors (index 0, 1, 2) starts at off[i], expert e at
   off[i] + e * stride[i] (HostExperts goff/uoff/doff and the per-expert
   strides, src/run_moe_stream.cpp:60-64, :177-179). */
typedef struct hoard_store_layer {
    uint64_t off[3];
    uint64_t stride[3];
} hoard_store_layer;

typedef struct hoard_store_cfg {
    int32_t readers;      /* reads in flight (the reference's IOQD, default 8: :310) */
    int32_t ram_experts;  /* RAM tier capacity in experts; <= 0: every expert (the
                             reference's default ram_cap, :337) */
    int32_t direct;       /* 1: O_DIRECT reads, falling back to buffered reads where
                             the file system refuses them; 0: buffered reads */
    int32_t pinned;       /* 1: RAM tier in pinned host memory (needs a HIP device);
                             0: pageable 4 KiB-aligned memory */
} hoard_store_cfg;

typedef struct hoard_store_stats {
    uint64_t requests;    /* experts asked for */
    uint64_t ram_hits;    /* served from the RAM tier (reference ram_hit) */
    uint64_t file_reads;  /* read from the file (reference nvme_fall) */
    uint64_t bytes_read;  /* expert bytes read (reference disk_bytes) */
    uint64_t read_ns;     /* wall time inside read batches (reference disk_ns) */
    int32_t direct;       /* reads bypass the page cache: 1 straight into the RAM tier,
                             2 through a per-reader buffer (O_DIRECT cannot target
                             memory pinned by the GPU driver); 0 buffered reads */
    int32_t ram_experts;  /* the capacity in use */
} hoard_store_stats;

/* Opens `path` for expert reads and sets up the RAM tier (its memory is
   allocated as entries are first used): DirectIO::init and the RamTier set-up
   (src/run_qwen35.cpp:105-113, :390-393).  layers[n_layer] as above. */
int hoard_store_open(const char *path, int n_layer, int n_expert, const hoard_store_layer *layers,
                     const hoard_store_cfg *cfg, hoard_store **out);
void hoard_store_close(hoard_store *s);

/* Makes experts ids[0..n) of `layer` resident in the RAM tier, reading the
   missing ones from the file (phases A and B of the fetch,
   src/run_qwen35.cpp:600-627), and returns the address of each one's gate, up
   and down bytes in parts[3*j + 0..2] (hit[j] = 1 when it was already held,
   optional).  n <= the RAM tier's capacity.  The addresses stay valid until a
   later call evicts the entry. */
int hoard_store_fetch(hoard_store *s, int layer, int n, const int32_t *ids, const void **parts, uint8_t *hit);

/* The counters since opening or the last reset: the reference's ram_hit,
   nvme_fall, disk_bytes and disk_ns (src/run_qwen35.cpp:398-399, :606, :624-632). */
int hoard_store_get_stats(const hoard_store *s, hoard_store_stats *out);
int hoard_store_reset_stats(hoard_store *s);

/* Serves the slot misses of a pool handle (pool_k > 0) from the store
   instead of the pinned copy of every expert: the reference's three tiers,
   VRAM slot, RAM tier, file (src/run_qwen35.cpp:596-638).  Call before the first
   hoard_moe_set_layer_weights; afterwards that call takes expert tensors
   from the store (w->gate / up / down may be NULL; their types must give the
   store's strides).  The store must stay open while the handle uses it. */
int hoard_moe_attach_store(hoard_moe *h, hoard_store *s);

#ifdef __cplusplus
}
#endif

#endif /* HOARD_STORE_H */
