// Expert pager: VRAM expert slots kept by the aged-LFU ExpertCache, misses
// filled from pinned host memory by hipMemcpyAsync on dedicated copy streams.
//
// The reference pager (crates/llmpager-cuda/src/pager.rs) reads a pack file
// into a pinned buffer on I/O worker threads, copies it into the slot, records
// the slot's event and only then publishes it (pager.rs:650-718); compute
// waits device-side with wait_stream (pager.rs:499-503) and releases are
// deferred until the forward pass is done with the slot (decode.rs:621-649).
// Here the blob source is pinned host memory already (the "pinned host ring";
// the disk and RAM tiers are outside the hot path), so request() issues the
// copy itself, on a copy stream, and returns at once:
//   - the compute stream waits on each returned slot's fill event;
//   - the layer's device slot table (expert -> slot) is refreshed in stream
//     order on the compute stream, so the fused layer kernels see it;
//   - release_after() hands the pins back once the compute stream has passed
//     that point (an event), so a slot is never refilled while a kernel still
//     reads the expert it held.
// All layers share one arena of layers x slots_per_layer slots, so slot-table
// values are global slot numbers: per-layer pools and the single global pool
// (pager.rs:296-318) use the same kernels unchanged.
#include <hip/hip_runtime_api.h>
#include <string.h>

#include <algorithm>
#include <deque>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/llmpager_hip.h"
#include "lp_internal.h"

namespace {

enum class Fill { Empty, InFlight, Ready };

struct Deferred {
    hipEvent_t ev;
    std::vector<uint32_t> slots;
};

}  // namespace

struct lp_pager {
    lp_ctx* ctx = nullptr;
    lp_pager_config cfg{};
    uint64_t span = 0;
    lp_cache* cache = nullptr;
    void* arena = nullptr;                 // layers * slots_per_layer * span
    int32_t* dev_tables = nullptr;         // device int32 [layers][E]
    int32_t* host_tables = nullptr;        // pinned int32 [layers][E] (the truth)
    // staging ring for in-order table refreshes on the compute stream
    int32_t* stage = nullptr;              // pinned int32 [kRing][E]
    std::vector<hipEvent_t> stage_ev;
    size_t stage_next = 0;
    std::vector<hipStream_t> copy_streams;
    size_t copy_next = 0;
    std::vector<hipEvent_t> fill_ev;       // per slot: its last fill
    std::vector<Fill> fill;
    std::deque<Deferred> deferred;         // releases waiting on the compute stream
    std::deque<Deferred> prefetched;       // prefetch pins dropped when their fill lands
    std::vector<hipEvent_t> ev_pool;
    uint64_t bytes_fetched = 0, fetches = 0, stalls = 0, ticks = 0;
    std::mutex mu;
};

namespace {

constexpr size_t kRing = 256;
constexpr uint64_t kAlign = 4096;  // pack.rs ALIGN: slot span granularity (pager.rs:263)

int fail(int code, const std::string& m) { return lpi::set_error(code, m); }

int hip_fail(hipError_t e, const char* what) {
    return fail((int)e, std::string(what) + ": " + hipGetErrorString(e));
}

#define PCHK(expr)                                        \
    do {                                                  \
        hipError_t e_ = (expr);                           \
        if (e_ != hipSuccess) return hip_fail(e_, #expr); \
    } while (0)

uint64_t slot_dev(const lp_pager* p, uint32_t slot) {
    return reinterpret_cast<uint64_t>(p->arena) + (uint64_t)slot * p->span;
}

hipEvent_t take_event(lp_pager* p) {
    if (!p->ev_pool.empty()) {
        hipEvent_t e = p->ev_pool.back();
        p->ev_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) return nullptr;
    return e;
}

// Hand back the pins of every deferred release whose event has completed
// (all of them, waiting, when `block`); the same for prefetches.
int drain(lp_pager* p, std::deque<Deferred>& q, bool block) {
    while (!q.empty()) {
        Deferred& d = q.front();
        hipError_t e = block ? hipEventSynchronize(d.ev) : hipEventQuery(d.ev);
        if (e == hipErrorNotReady) break;
        if (e != hipSuccess) return hip_fail(e, "deferred release event");
        for (uint32_t s : d.slots) lp_cache_release(p->cache, s);
        p->ev_pool.push_back(d.ev);
        q.pop_front();
    }
    return LP_OK;
}

// The copy of blob (layer, expert) into `slot` on the next copy stream; the
// slot's fill event marks its end.  Published at once: every consumer is
// ordered behind the event (stream waits, or lp_pager_wait on the host).
int fill_slot(lp_pager* p, uint16_t layer, uint16_t expert, uint32_t slot) {
    const uint8_t* src = reinterpret_cast<const uint8_t*>(p->cfg.host_blobs) +
                         ((uint64_t)layer * p->cfg.experts_per_layer + expert) * p->cfg.host_stride;
    hipStream_t cs = p->copy_streams[p->copy_next++ % p->copy_streams.size()];
    PCHK(hipMemcpyAsync(reinterpret_cast<void*>(slot_dev(p, slot)), src, p->cfg.blob_bytes,
                        hipMemcpyHostToDevice, cs));
    PCHK(hipEventRecord(p->fill_ev[slot], cs));
    p->fill[slot] = Fill::InFlight;
    lp_cache_publish(p->cache, slot);
    p->bytes_fetched += p->cfg.blob_bytes;
    p->fetches += 1;
    return LP_OK;
}

// Point the layer's host table at the new slot (and the evicted id at -1).
void table_update(lp_pager* p, uint16_t layer, uint16_t expert, uint32_t slot, int64_t evicted) {
    const uint32_t E = p->cfg.experts_per_layer;
    if (evicted >= 0) p->host_tables[(uint64_t)evicted] = -1;  // ids fold (layer, expert) exactly
    p->host_tables[(uint64_t)layer * E + expert] = (int32_t)slot;
}

}  // namespace

extern "C" {

int lp_pager_new(lp_ctx* ctx, const lp_pager_config* cfg, lp_pager** out) {
    if (!out) return fail(LP_E_INVALID, "lp_pager_new: null out");
    *out = nullptr;
    if (!ctx || !cfg) return fail(LP_E_INVALID, "lp_pager_new: null argument");
    if (cfg->layers == 0 || cfg->experts_per_layer == 0 || cfg->experts_per_layer > 65536 ||
        cfg->slots_per_layer == 0 || cfg->blob_bytes == 0 || !cfg->host_blobs ||
        cfg->host_stride < cfg->blob_bytes || cfg->copy_streams < 1 || cfg->copy_streams > 8)
        return fail(LP_E_INVALID, "lp_pager_new: bad configuration");
    if (int r = lp_bind_thread(ctx)) return r;
    lp_pager* p = new lp_pager();
    p->ctx = ctx;
    p->cfg = *cfg;
    p->span = cfg->span ? cfg->span : (cfg->blob_bytes + kAlign - 1) / kAlign * kAlign;
    if (p->span < cfg->blob_bytes || p->span % 256) {
        delete p;
        return fail(LP_E_INVALID, "lp_pager_new: span must hold a blob and be 256-byte aligned");
    }
    const uint32_t L = cfg->layers, E = cfg->experts_per_layer, S = cfg->slots_per_layer;
    const uint64_t total = (uint64_t)L * S;
    // pager.rs:331-343: per-layer pools (decay by insertions), or one pool
    // whose decay is driven by lp_pager_tick
    p->cache = cfg->global_pool ? lp_cache_partitioned(1, E, (uint32_t)total, 0xffffffffu)
                                : lp_cache_partitioned(L, E, S, cfg->decay_interval ? cfg->decay_interval : 256);
    hipError_t e = p->cache ? hipSuccess : hipErrorOutOfMemory;
    if (e == hipSuccess) e = hipMalloc(&p->arena, total * p->span);
    if (e == hipSuccess) e = hipMalloc((void**)&p->dev_tables, (size_t)L * E * 4);
    if (e == hipSuccess) e = hipMemset(p->dev_tables, 0xff, (size_t)L * E * 4);
    if (e == hipSuccess) e = hipHostMalloc((void**)&p->host_tables, (size_t)L * E * 4, hipHostMallocDefault);
    if (e == hipSuccess) e = hipHostMalloc((void**)&p->stage, kRing * E * 4, hipHostMallocDefault);
    if (e == hipSuccess) {
        memset(p->host_tables, 0xff, (size_t)L * E * 4);
        p->fill.assign(total, Fill::Empty);
        p->fill_ev.assign(total, nullptr);
        for (uint64_t s = 0; s < total && e == hipSuccess; ++s)
            e = hipEventCreateWithFlags(&p->fill_ev[s], hipEventDisableTiming);
        p->stage_ev.assign(kRing, nullptr);
        for (size_t r = 0; r < kRing && e == hipSuccess; ++r)
            e = hipEventCreateWithFlags(&p->stage_ev[r], hipEventDisableTiming);
        for (int i = 0; i < cfg->copy_streams && e == hipSuccess; ++i) {
            hipStream_t s = nullptr;
            e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
            if (e == hipSuccess) p->copy_streams.push_back(s);
        }
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        lp_pager_free(p);
        return hip_fail(e, "lp_pager_new");
    }
    *out = p;
    return LP_OK;
}

void lp_pager_free(lp_pager* p) {
    if (!p) return;
    for (hipStream_t s : p->copy_streams) (void)hipStreamSynchronize(s);
    (void)hipDeviceSynchronize();
    for (auto* q : {&p->deferred, &p->prefetched})
        for (Deferred& d : *q) (void)hipEventDestroy(d.ev);
    for (hipEvent_t ev : p->ev_pool) (void)hipEventDestroy(ev);
    for (hipEvent_t ev : p->fill_ev)
        if (ev) (void)hipEventDestroy(ev);
    for (hipEvent_t ev : p->stage_ev)
        if (ev) (void)hipEventDestroy(ev);
    for (hipStream_t s : p->copy_streams) (void)hipStreamDestroy(s);
    if (p->stage) (void)hipHostFree(p->stage);
    if (p->host_tables) (void)hipHostFree(p->host_tables);
    if (p->dev_tables) (void)hipFree(p->dev_tables);
    if (p->arena) (void)hipFree(p->arena);
    if (p->cache) lp_cache_free(p->cache);
    delete p;
}

uint64_t lp_pager_arena(const lp_pager* p) { return p ? reinterpret_cast<uint64_t>(p->arena) : 0; }

uint64_t lp_pager_span(const lp_pager* p) { return p ? p->span : 0; }

uint64_t lp_pager_slot_table(const lp_pager* p, uint32_t layer) {
    if (!p || layer >= p->cfg.layers) return 0;
    return reinterpret_cast<uint64_t>(p->dev_tables) + (uint64_t)layer * p->cfg.experts_per_layer * 4;
}

uint32_t lp_pager_slots_per_layer(const lp_pager* p) {
    return p ? lp_cache_slots_per_partition(p->cache) : 0;
}

int lp_pager_request(lp_pager* p, uint16_t layer, const uint16_t* experts, int n, lp_stream compute,
                     uint32_t* slots_out) {
    if (!p || (n > 0 && !experts) || n < 0 || layer >= p->cfg.layers)
        return fail(LP_E_INVALID, "lp_pager_request: bad arguments");
    std::lock_guard<std::mutex> g(p->mu);
    if ((uint32_t)n > lp_cache_slots_per_partition(p->cache))
        return fail(LP_E_INVALID, "lp_pager_request: more experts than the pool holds (pager.rs:405-413)");
    if (int r = lp_bind_thread(p->ctx)) return r;
    if (int r = drain(p, p->deferred, false)) return r;
    if (int r = drain(p, p->prefetched, false)) return r;
    const uint32_t E = p->cfg.experts_per_layer;
    for (int i = 0; i < n; ++i)
        if (experts[i] >= E) return fail(LP_E_INVALID, "lp_pager_request: expert id out of range");
    hipStream_t cs = (hipStream_t)compute;
    // the pins this call has taken: handed back if it fails part-way, so a
    // failed request leaves no slot pinned
    std::vector<uint32_t> pinned;
    pinned.reserve((size_t)n);
    auto unwind = [&](int code) {
        for (uint32_t s : pinned) lp_cache_release(p->cache, s);
        return code;
    };
    for (int i = 0; i < n; ++i) {
        const uint32_t id = lp_cache_fold(layer, experts[i], E);
        uint32_t slot = 0;
        int64_t evicted = -1;
        int r;
        for (;;) {
            r = lp_cache_acquire(p->cache, id, &slot, &evicted);
            if (r != LP_LOOKUP_STALLED) break;
            // every slot pinned: wait for deferred releases, then fills of
            // prefetches; with neither, nothing can free a slot (pager.rs:430-451)
            p->stalls += 1;
            if (!p->deferred.empty()) {
                if (int q = drain(p, p->deferred, true)) return unwind(q);
            } else if (!p->prefetched.empty()) {
                if (int q = drain(p, p->prefetched, true)) return unwind(q);
            } else {
                return unwind(fail(LP_E_INVALID, "expert cache deadlock: every slot of the pool is pinned "
                                                 "with no release pending (handles held across a pass)"));
            }
        }
        if (r < 0) return unwind(r);
        pinned.push_back(slot);
        if (r == LP_LOOKUP_MISS) {
            table_update(p, layer, experts[i], slot, evicted);
            if (int q = fill_slot(p, layer, experts[i], slot)) return unwind(q);
        }
        if (p->fill[slot] == Fill::InFlight) {
            hipError_t e = hipEventQuery(p->fill_ev[slot]);
            if (e == hipSuccess) {
                p->fill[slot] = Fill::Ready;
            } else if (e == hipErrorNotReady) {
                e = hipStreamWaitEvent(cs, p->fill_ev[slot], 0);  // pager.rs:499-503
                if (e != hipSuccess) return unwind(hip_fail(e, "hipStreamWaitEvent"));
            } else {
                return unwind(hip_fail(e, "fill event"));
            }
        }
        if (slots_out) slots_out[i] = slot;
    }
    // the layer's slot table, refreshed in stream order on the compute stream
    const size_t r = p->stage_next++ % kRing;
    hipError_t e = hipEventSynchronize(p->stage_ev[r]);  // its previous copy has been consumed
    if (e != hipSuccess) return unwind(hip_fail(e, "slot-table staging event"));
    int32_t* st = p->stage + r * E;
    memcpy(st, p->host_tables + (size_t)layer * E, (size_t)E * 4);
    e = hipMemcpyAsync(reinterpret_cast<void*>(lp_pager_slot_table(p, layer)), st, (size_t)E * 4,
                       hipMemcpyHostToDevice, cs);
    if (e != hipSuccess) return unwind(hip_fail(e, "slot-table copy"));
    e = hipEventRecord(p->stage_ev[r], cs);
    if (e != hipSuccess) return unwind(hip_fail(e, "slot-table event"));
    return LP_OK;
}

int lp_pager_release(lp_pager* p, const uint32_t* slots, int n) {
    if (!p || n < 0 || (n > 0 && !slots)) return fail(LP_E_INVALID, "lp_pager_release: bad arguments");
    std::lock_guard<std::mutex> g(p->mu);
    for (int i = 0; i < n; ++i)
        if (int r = lp_cache_release(p->cache, slots[i])) return fail(r, "lp_pager_release: slot not pinned");
    return LP_OK;
}

int lp_pager_release_after(lp_pager* p, const uint32_t* slots, int n, lp_stream compute) {
    if (!p || n < 0 || (n > 0 && !slots)) return fail(LP_E_INVALID, "lp_pager_release_after: bad arguments");
    std::lock_guard<std::mutex> g(p->mu);
    if (n == 0) return LP_OK;
    hipEvent_t ev = take_event(p);
    if (!ev) return fail(LP_E_DEVICE, "lp_pager_release_after: no event");
    PCHK(hipEventRecord(ev, (hipStream_t)compute));
    p->deferred.push_back(Deferred{ev, std::vector<uint32_t>(slots, slots + n)});
    return LP_OK;
}

int lp_pager_prefetch(lp_pager* p, uint16_t layer, const uint16_t* experts, int n) {
    if (!p || n < 0 || (n > 0 && !experts) || layer >= p->cfg.layers)
        return fail(LP_E_INVALID, "lp_pager_prefetch: bad arguments");
    std::lock_guard<std::mutex> g(p->mu);
    if (int r = lp_bind_thread(p->ctx)) return r;
    const uint32_t E = p->cfg.experts_per_layer;
    std::vector<uint32_t> pinned;
    for (int i = 0; i < n; ++i) {
        if (experts[i] >= E) return fail(LP_E_INVALID, "lp_pager_prefetch: expert id out of range");
        uint32_t slot = 0;
        int64_t evicted = -1;
        const int r = lp_cache_acquire(p->cache, lp_cache_fold(layer, experts[i], E), &slot, &evicted);
        if (r == LP_LOOKUP_HIT) {
            lp_cache_release(p->cache, slot);  // pager.rs:469
        } else if (r == LP_LOOKUP_MISS) {
            table_update(p, layer, experts[i], slot, evicted);
            if (int q = fill_slot(p, layer, experts[i], slot)) return q;
            pinned.push_back(slot);
        }  // stalled: skipped (pager.rs:484)
    }
    if (pinned.empty()) return LP_OK;
    // the pins drop once the fills have landed (pager.rs:711-713,
    // release_after_fill): an event behind every fill of this call
    hipEvent_t ev = take_event(p);
    if (!ev) return fail(LP_E_DEVICE, "lp_pager_prefetch: no event");
    for (uint32_t s : pinned) PCHK(hipStreamWaitEvent(p->copy_streams[0], p->fill_ev[s], 0));
    PCHK(hipEventRecord(ev, p->copy_streams[0]));
    p->prefetched.push_back(Deferred{ev, pinned});
    return LP_OK;
}

int lp_pager_wait(lp_pager* p, uint32_t slot) {
    if (!p || slot >= p->fill.size()) return fail(LP_E_INVALID, "lp_pager_wait: bad slot");
    hipEvent_t ev;
    {
        std::lock_guard<std::mutex> g(p->mu);
        if (p->fill[slot] != Fill::InFlight) return LP_OK;
        ev = p->fill_ev[slot];
    }
    PCHK(hipEventSynchronize(ev));  // pager.rs:489-496
    std::lock_guard<std::mutex> g(p->mu);
    p->fill[slot] = Fill::Ready;
    return LP_OK;
}

int lp_pager_tick(lp_pager* p) {
    if (!p) return fail(LP_E_INVALID, "lp_pager_tick: null pager");
    std::lock_guard<std::mutex> g(p->mu);
    if (!p->cfg.global_pool) return LP_OK;  // pager.rs:524-533
    const uint32_t every = p->cfg.pool_decay_tokens ? p->cfg.pool_decay_tokens : 4;
    if (++p->ticks % every == 0) lp_cache_decay_all(p->cache);
    return LP_OK;
}

int lp_pager_sync(lp_pager* p) {
    if (!p) return fail(LP_E_INVALID, "lp_pager_sync: null pager");
    std::lock_guard<std::mutex> g(p->mu);
    for (hipStream_t s : p->copy_streams) PCHK(hipStreamSynchronize(s));
    if (int r = drain(p, p->deferred, true)) return r;
    return drain(p, p->prefetched, true);
}

int lp_pager_get_metrics(lp_pager* p, lp_pager_metrics* out) {
    if (!p || !out) return fail(LP_E_INVALID, "lp_pager_get_metrics: bad arguments");
    std::lock_guard<std::mutex> g(p->mu);
    uint64_t h = 0, m = 0;
    lp_cache_stats(p->cache, &h, &m);
    out->hits = h;
    out->misses = m;
    out->bytes_fetched = p->bytes_fetched;
    out->fetches = p->fetches;
    out->stalls = p->stalls;
    return LP_OK;
}

}  // extern "C"
