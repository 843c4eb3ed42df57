// Per-layer expert-slot residency with LRU replacement: the bookkeeping of
// the reference's Slots pool (src/run_moe_stream.cpp:193-203, filled at
// :386-387 and :416-419), host-only so the device pool and the host replay
// share one implementation.
#pragma once

#include <cstdint>
#include <list>
#include <vector>

namespace hoard {

class SlotLru {
  public:
    SlotLru() = default;
    SlotLru(int n_layer, int n_expert, int k) { reset(n_layer, n_expert, k); }

    void reset(int n_layer, int n_expert, int k) {
        k_ = k;
        n_expert_ = n_expert;
        slot_expert_.assign(n_layer, std::vector<int>(k, -1));
        expert_slot_.assign(n_layer, std::vector<int>(n_expert, -1));
        lru_.assign(n_layer, std::list<int>());
        for (auto &l : lru_)
            for (int s = 0; s < k; ++s) l.push_back(s);  // front = most recent, as built at :246-252
    }

    // Empties one layer's slots (its weights were replaced).
    void reset_layer(int layer) {
        slot_expert_[layer].assign(k_, -1);
        expert_slot_[layer].assign(n_expert_, -1);
        lru_[layer].clear();
        for (int s = 0; s < k_; ++s) lru_[layer].push_back(s);
    }

    int k() const { return k_; }
    int n_layer() const { return (int)lru_.size(); }
    int n_expert() const { return n_expert_; }

    // One call for the n experts a token selected in `layer`.  Hits are
    // classified first (:385-387): the slot moves to the front of the LRU list.
    // Then each miss takes the least recently used slot (:418-419), evicts its
    // expert and becomes the most recent.  Naive mode (:417) places miss j in
    // slot j and keeps no residency, so every request is a miss.
    // slot_out[j] receives the slot and miss_out[j] (if non-null) 1 for a miss.
    void access(int layer, const int32_t *sel, int n, bool naive, int32_t *slot_out, uint8_t *miss_out) {
        std::vector<int> &se = slot_expert_[layer];
        std::vector<int> &es = expert_slot_[layer];
        std::list<int> &lru = lru_[layer];
        std::vector<char> hit(n, 0);
        if (!naive) {
            for (int j = 0; j < n; ++j) {
                const int s = es[sel[j]];
                if (s >= 0) {
                    lru.remove(s);
                    lru.push_front(s);
                    slot_out[j] = s;
                    hit[j] = 1;
                }
            }
        }
        for (int j = 0; j < n; ++j) {
            if (miss_out) miss_out[j] = hit[j] ? 0 : 1;
            if (hit[j]) continue;
            if (naive) {
                slot_out[j] = j;
                continue;
            }
            const int s = lru.back();
            lru.pop_back();
            const int old = se[s];
            if (old >= 0) es[old] = -1;  // map.erase(old), whichever slot it pointed to
            se[s] = sel[j];
            es[sel[j]] = s;
            lru.push_front(s);
            slot_out[j] = s;
        }
    }

    // The verify loop's ensure (src/run_specloop.cpp:59-67), one id after the
    // other with no hits-first pass: a hit moves to the front, a miss takes the
    // back slot.  A repeated id is a hit on its earlier slot.
    void access_sequential(int layer, const int32_t *sel, int n, int32_t *slot_out, uint8_t *miss_out) {
        std::vector<int> &se = slot_expert_[layer];
        std::vector<int> &es = expert_slot_[layer];
        std::list<int> &lru = lru_[layer];
        for (int j = 0; j < n; ++j) {
            int s = es[sel[j]];
            const bool hit = s >= 0;
            if (hit) {
                lru.remove(s);
            } else {
                s = lru.back();
                lru.pop_back();
                if (se[s] >= 0) es[se[s]] = -1;
                se[s] = sel[j];
                es[sel[j]] = s;
            }
            lru.push_front(s);
            slot_out[j] = s;
            if (miss_out) miss_out[j] = hit ? 0 : 1;
        }
    }

    int slot_of(int layer, int expert) const { return expert_slot_[layer][expert]; }
    int expert_in(int layer, int slot) const { return slot_expert_[layer][slot]; }

  private:
    int k_ = 0, n_expert_ = 0;
    std::vector<std::vector<int>> slot_expert_;  // [layer][slot] -> expert, -1 empty
    std::vector<std::vector<int>> expert_slot_;  // [layer][expert] -> slot, -1 absent
    std::vector<std::list<int>> lru_;            // [layer] slots, front = most recent
};

}  // namespace hoard
