// Host replay of the expert-slot LRU: the same bookkeeping the device pool
// runs, without a device, for trace studies and tests (the counterpart of the
// reference's LRU simulators, bench/profiler.py:65-91 and
// bench/routing_model.py:61-75, but with the engine's hits-first order).
#include <new>

#include "hoard_moe.h"
#include "slot_lru.h"

struct hoard_slot_lru {
    hoard::SlotLru lru;
    int mode = 0;  // 0 hits first, 1 naive, 2 one id after the other (the verify loop's ensure)
};

extern "C" {

int hoard_slot_lru_create(int n_layer, int n_expert, int k, int naive, hoard_slot_lru **out) {
    if (!out) return HOARD_ERR_INVALID;
    *out = nullptr;
    if (n_layer <= 0 || n_expert <= 0 || k <= 0 || k > n_expert || naive < 0 || naive > 2) return HOARD_ERR_INVALID;
    hoard_slot_lru *p = new (std::nothrow) hoard_slot_lru();
    if (!p) return HOARD_ERR_OOM;
    p->lru.reset(n_layer, n_expert, k);
    p->mode = naive;
    *out = p;
    return HOARD_OK;
}

int hoard_slot_lru_access(hoard_slot_lru *p, int layer, const int32_t *sel, int n, int32_t *slot_out,
                          uint8_t *miss_out) {
    if (!p || !sel || !slot_out || n <= 0 || (p->mode != 2 && n > p->lru.k())) return HOARD_ERR_INVALID;
    for (int j = 0; j < n; ++j)
        if (sel[j] < 0 || sel[j] >= p->lru.n_expert()) return HOARD_ERR_INVALID;
    if (layer < 0 || layer >= p->lru.n_layer()) return HOARD_ERR_INVALID;
    if (p->mode == 2)
        p->lru.access_sequential(layer, sel, n, slot_out, miss_out);
    else
        p->lru.access(layer, sel, n, p->mode == 1, slot_out, miss_out);
    return HOARD_OK;
}

void hoard_slot_lru_destroy(hoard_slot_lru *p) { delete p; }

}  // extern "C"
