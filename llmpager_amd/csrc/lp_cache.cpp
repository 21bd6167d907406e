// Aged-LFU expert-slot bookkeeping: the semantics of the reference's
// ExpertCache (crates/llmpager-core/src/cache.rs:58-241), in C++ behind the
// C ABI so the pager and the device slot table can run without the Rust core.
//
// Experts are flat ids (layer * ids_per_partition + expert); slots are drawn
// from partitions (one per layer, or one global pool).  acquire() pins the
// slot it returns; a miss claims the unpinned slot with the lowest
// (frequency, occupied) key, lowest index first; counters halve every
// decay_interval insertions in a partition.  No iteration over the hash map,
// so slot choices are deterministic.
#include <stdint.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/llmpager_hip.h"

namespace {

struct SlotState {
    bool has_id = false;
    uint32_t id = 0;
    uint32_t freq = 0;
    uint32_t pins = 0;
    bool ready = false;  // false while a miss is in flight (cache.rs:43-46)
};

struct Partition {
    uint32_t base = 0, len = 0;
    std::unordered_map<uint32_t, uint32_t> map;  // id -> global slot
    uint32_t inserts_since_decay = 0;
};

}  // namespace

struct lp_cache {
    std::vector<SlotState> slots;
    std::vector<Partition> parts;
    uint32_t ids_per_partition = 0;
    uint32_t decay_interval = 0;
    uint64_t hits = 0, misses = 0;

    size_t part_of(uint32_t id) const {  // cache.rs:120-125
        if (parts.size() == 1) return 0;
        size_t p = id / ids_per_partition;
        return p < parts.size() ? p : parts.size() - 1;
    }
};

extern "C" {

// cache.rs:78-102
lp_cache* lp_cache_partitioned(uint32_t partitions, uint32_t ids_per_partition,
                               uint32_t slots_per_partition, uint32_t decay_interval) {
    if (partitions == 0 || slots_per_partition == 0 || decay_interval == 0 || ids_per_partition == 0)
        return nullptr;
    lp_cache* c = new lp_cache();
    c->slots.resize((size_t)partitions * slots_per_partition);
    c->parts.resize(partitions);
    for (uint32_t p = 0; p < partitions; ++p) {
        c->parts[p].base = p * slots_per_partition;
        c->parts[p].len = slots_per_partition;
    }
    c->ids_per_partition = ids_per_partition;
    c->decay_interval = decay_interval;
    return c;
}

// cache.rs:71-73: ids_per_partition is u32::MAX there, so every id below
// u32::MAX falls into partition 0 (part_of, cache.rs:120-125).  The pager
// builds its per-layer cache with lp_cache_partitioned and the
// experts-per-layer fold instead (pager.rs:339-344).
lp_cache* lp_cache_new(uint16_t num_layers, uint32_t slots_per_layer, uint32_t decay_interval) {
    return lp_cache_partitioned(num_layers, 0xffffffffu, slots_per_layer, decay_interval);
}

void lp_cache_free(lp_cache* c) { delete c; }

// cache.rs:106-108
uint32_t lp_cache_fold(uint16_t layer, uint16_t expert, uint32_t experts_per_layer) {
    return (uint32_t)layer * experts_per_layer + expert;
}

uint32_t lp_cache_slots_per_partition(const lp_cache* c) { return c ? c->parts[0].len : 0; }

uint32_t lp_cache_total_slots(const lp_cache* c) { return c ? (uint32_t)c->slots.size() : 0; }

// cache.rs:132-179
int lp_cache_acquire(lp_cache* c, uint32_t id, uint32_t* slot_out, int64_t* evicted_out) {
    if (!c) return LP_E_INVALID;
    if (evicted_out) *evicted_out = -1;
    Partition& P = c->parts[c->part_of(id)];
    auto it = P.map.find(id);
    if (it != P.map.end()) {
        SlotState& s = c->slots[it->second];
        if (s.freq != 0xffffffffu) s.freq += 1;  // saturating_add
        s.pins += 1;
        c->hits += 1;
        if (slot_out) *slot_out = it->second;
        return LP_LOOKUP_HIT;
    }
    bool found = false;
    uint32_t victim = 0, vfreq = 0;
    bool vocc = false;
    for (uint32_t i = P.base; i < P.base + P.len; ++i) {
        const SlotState& s = c->slots[i];
        if (s.pins > 0) continue;
        const bool occ = s.has_id;
        if (!found || s.freq < vfreq || (s.freq == vfreq && occ < vocc)) {
            found = true;
            victim = i;
            vfreq = s.freq;
            vocc = occ;
        }
    }
    if (!found) return LP_LOOKUP_STALLED;
    SlotState& v = c->slots[victim];
    if (v.has_id) {
        P.map.erase(v.id);
        if (evicted_out) *evicted_out = v.id;
    }
    P.map[id] = victim;
    v.has_id = true;
    v.id = id;
    v.freq = 1;
    v.pins = 1;
    v.ready = false;
    c->misses += 1;
    P.inserts_since_decay += 1;
    if (P.inserts_since_decay >= c->decay_interval) {
        P.inserts_since_decay = 0;
        for (uint32_t i = P.base; i < P.base + P.len; ++i) c->slots[i].freq /= 2;
    }
    if (slot_out) *slot_out = victim;
    return LP_LOOKUP_MISS;
}

// cache.rs:184-195
int lp_cache_lookup_ready(lp_cache* c, uint32_t id, uint32_t* slot_out) {
    if (!c) return LP_E_INVALID;
    Partition& P = c->parts[c->part_of(id)];
    auto it = P.map.find(id);
    if (it == P.map.end()) return 0;
    SlotState& s = c->slots[it->second];
    if (!s.ready) return 0;
    if (s.freq != 0xffffffffu) s.freq += 1;
    s.pins += 1;
    c->hits += 1;
    if (slot_out) *slot_out = it->second;
    return 1;
}

// cache.rs:198-200
int lp_cache_publish(lp_cache* c, uint32_t slot) {
    if (!c || slot >= c->slots.size()) return LP_E_INVALID;
    c->slots[slot].ready = true;
    return LP_OK;
}

int lp_cache_is_ready(const lp_cache* c, uint32_t slot) {
    if (!c || slot >= c->slots.size()) return LP_E_INVALID;
    return c->slots[slot].ready ? 1 : 0;
}

// cache.rs:207-211 (the reference asserts; this returns an error instead)
int lp_cache_release(lp_cache* c, uint32_t slot) {
    if (!c || slot >= c->slots.size()) return LP_E_INVALID;
    if (c->slots[slot].pins == 0) return LP_E_INVALID;
    c->slots[slot].pins -= 1;
    return LP_OK;
}

// cache.rs:218-225
int lp_cache_decay_all(lp_cache* c) {
    if (!c) return LP_E_INVALID;
    for (SlotState& s : c->slots) s.freq /= 2;
    for (Partition& p : c->parts) p.inserts_since_decay = 0;
    return LP_OK;
}

// cache.rs:229-236
int lp_cache_is_wedged(const lp_cache* c, uint32_t id) {
    if (!c) return LP_E_INVALID;
    const Partition& P = c->parts[c->part_of(id)];
    for (uint32_t i = P.base; i < P.base + P.len; ++i) {
        const SlotState& s = c->slots[i];
        if (!(s.pins > 0 && s.ready)) return 0;
    }
    return 1;
}

// cache.rs:238-240
int lp_cache_stats(const lp_cache* c, uint64_t* hits, uint64_t* misses) {
    if (!c) return LP_E_INVALID;
    if (hits) *hits = c->hits;
    if (misses) *misses = c->misses;
    return LP_OK;
}

// The expert a slot holds (-1 if empty): lets the pager rebuild a layer's
// device slot table without a second map.
int64_t lp_cache_slot_id(const lp_cache* c, uint32_t slot) {
    if (!c || slot >= c->slots.size() || !c->slots[slot].has_id) return -1;
    return c->slots[slot].id;
}

}  // extern "C"
