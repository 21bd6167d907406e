// Expert pager: VRAM expert slots kept by the aged-LFU ExpertCache, misses
// filled by hipMemcpyAsync on dedicated copy streams (pager.rs).
//
// Fill sources (lp_pager_config.source):
//   LP_PAGER_SRC_PINNED  the blobs already sit in pinned host memory: request()
//                        issues each copy itself, round-robin over the copy
//                        streams, and returns at once;
//   LP_PAGER_SRC_HOST    the blobs sit in pageable host memory (a RAM tier, a
//                        mapped file): I/O workers copy each into a pinned
//                        staging ring and DMA it from there;
//   LP_PAGER_SRC_PACK    a .llmpk pack file (lp_pager_open): I/O workers pread
//                        the blob (O_DIRECT optional) into the staging ring,
//                        through an optional RAM tier, then DMA it.
// The workers follow pager.rs:650-718: read into a pinned buffer, copy to the
// slot on the worker's stream, record the slot's event, publish.  A ring
// buffer is reused once its copy has completed (its own event), so the ring
// is a few span-sized buffers per worker whatever the pack's size.
//
// Compute never waits on the host for a copy to finish: the compute stream
// waits on each slot's fill event.  It does wait on the host until a missed
// expert's copy has been *enqueued* (its read done), as wait_stream does
// (pager.rs:497-503).  The layer's device slot table (expert -> slot) is
// refreshed in stream order on the compute stream, so the fused layer kernels
// see it; deferred releases hand pins back once the compute stream has
// passed a point (an event), so a slot is never refilled while a kernel
// still reads the expert it held.  All layers share one arena of
// layers x slots_per_layer slots, so slot-table values are global slot
// numbers: per-layer pools and the single global pool (pager.rs:296-318) use
// the same kernels unchanged.
#include <hip/hip_runtime_api.h>
#include <string.h>
#include <sys/mman.h>

#include <algorithm>
#include <chrono>
#include <condition_variable>
#include <deque>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/llmpager_hip.h"
#include "lp_internal.h"

namespace {

// Pending: a worker has the job (read not yet enqueued as a copy);
// InFlight: the copy is enqueued and the slot's event recorded.
enum class Fill { Empty, Pending, InFlight, Ready };

struct Deferred {
    hipEvent_t ev;
    std::vector<uint32_t> slots;
};

struct Job {
    uint16_t layer, expert;
    uint32_t slot;
    bool release_after_fill;  // a prefetch: the pin drops when the fill lands
};

// The host-RAM tier in front of a pack (pager.rs:69-164): one anonymous
// mapping of span-sized slabs, bookkept by a single-pool ExpertCache whose
// ids fold (layer, expert).
struct RamTier {
    lp_cache* cache = nullptr;
    uint8_t* base = nullptr;
    size_t bytes = 0;
    uint64_t span = 0;
    uint32_t experts = 0;
    uint64_t hits = 0;
    std::mutex mu;
};

}  // namespace

struct lp_pager {
    lp_ctx* ctx = nullptr;
    lp_pager_config cfg{};
    int device = 0;
    uint64_t span = 0;
    lp_cache* cache = nullptr;
    void* arena = nullptr;                 // layers * slots_per_layer * span
    int32_t* dev_tables = nullptr;         // device int32 [layers][E]
    int32_t* host_tables = nullptr;        // pinned int32 [layers][E] (the truth)
    // staging ring for in-order table refreshes on the compute stream
    int32_t* stage = nullptr;              // pinned int32 [kRing][E]
    std::vector<hipEvent_t> stage_ev;
    size_t stage_next = 0;
    std::vector<hipStream_t> copy_streams; // pinned source
    size_t copy_next = 0;
    std::vector<hipEvent_t> fill_ev;       // per slot: its last fill
    std::vector<Fill> fill;
    std::deque<Deferred> deferred;         // releases waiting on the compute stream
    std::deque<Deferred> prefetched;       // prefetch pins dropped when their fill lands
    std::vector<hipEvent_t> ev_pool;
    uint64_t bytes_fetched = 0, fetches = 0, stalls = 0, ticks = 0;
    std::mutex mu;
    // I/O workers (host and pack sources)
    lp_pack* pack = nullptr;
    std::vector<std::thread> workers;
    std::deque<Job> jobs;
    std::condition_variable jobs_cv, fill_cv;
    bool stop = false;
    int worker_err = LP_OK;
    std::string worker_msg;
    int pending_prefetch = 0;              // prefetch jobs not yet enqueued
    RamTier* ram = nullptr;
    std::vector<uint64_t> fetch_counts;    // per (layer, expert): fills, the profile prewarm uses
    uint64_t lat_buckets[7] = {};          // worker fetch time: <1, <2, <5, <10, <20, <50, >=50 ms
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

bool uses_workers(const lp_pager* p) { return p->cfg.source != LP_PAGER_SRC_PINNED; }

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
// (all of them, waiting, when `block`); the same for prefetches.  Caller
// holds p->mu.
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

// Pinned source: the copy of blob (layer, expert) into `slot` on the next copy
// stream; the slot's fill event marks its end.  Published at once: every
// consumer is ordered behind the event (stream waits, or lp_pager_wait).
int fill_slot_pinned(lp_pager* p, uint16_t layer, uint16_t expert, uint32_t slot) {
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
    p->fetch_counts[(size_t)layer * p->cfg.experts_per_layer + expert] += 1;
    return LP_OK;
}

// A miss: queue the fill (worker sources) or issue it (pinned source).
// Caller holds p->mu.
int schedule_fill(lp_pager* p, uint16_t layer, uint16_t expert, uint32_t slot, bool prefetch) {
    if (!uses_workers(p)) return fill_slot_pinned(p, layer, expert, slot);
    p->fill[slot] = Fill::Pending;
    lp_cache_publish(p->cache, slot);  // consumers wait on the fill state, then the event
    p->jobs.push_back(Job{layer, expert, slot, prefetch});
    if (prefetch) p->pending_prefetch += 1;
    p->jobs_cv.notify_one();
    return LP_OK;
}

// Point the layer's host table at the new slot (and the evicted id at -1).
void table_update(lp_pager* p, uint16_t layer, uint16_t expert, uint32_t slot, int64_t evicted) {
    const uint32_t E = p->cfg.experts_per_layer;
    if (evicted >= 0) p->host_tables[(uint64_t)evicted] = -1;  // ids fold (layer, expert) exactly
    p->host_tables[(uint64_t)layer * E + expert] = (int32_t)slot;
}

// RAM tier: copy the expert into dst on a hit (pager.rs:121-134).
bool ram_get(RamTier* r, uint16_t layer, uint16_t expert, void* dst) {
    const uint32_t key = (uint32_t)layer * r->experts + expert;
    uint32_t slot = 0;
    {
        std::lock_guard<std::mutex> g(r->mu);
        if (!lp_cache_lookup_ready(r->cache, key, &slot)) return false;
    }
    memcpy(dst, r->base + (size_t)slot * r->span, r->span);
    std::lock_guard<std::mutex> g(r->mu);
    lp_cache_release(r->cache, slot);
    r->hits += 1;
    return true;
}

// RAM tier: write-allocate after a disk read, best effort (pager.rs:137-157).
void ram_put(RamTier* r, uint16_t layer, uint16_t expert, const void* src) {
    const uint32_t key = (uint32_t)layer * r->experts + expert;
    uint32_t slot = 0;
    int64_t evicted = -1;
    {
        std::lock_guard<std::mutex> g(r->mu);
        const int rc = lp_cache_acquire(r->cache, key, &slot, &evicted);
        if (rc == LP_LOOKUP_HIT) {
            lp_cache_release(r->cache, slot);
            return;
        }
        if (rc != LP_LOOKUP_MISS) return;
    }
    memcpy(r->base + (size_t)slot * r->span, src, r->span);
    std::lock_guard<std::mutex> g(r->mu);
    lp_cache_publish(r->cache, slot);
    lp_cache_release(r->cache, slot);
}

// A blob's staging is split over cfg.stage_threads threads in 1 MiB pieces:
// a decode step misses only one or two experts per layer, and one thread's
// memcpy (or pread) of a 10 MB blob is what the layer would wait for.
constexpr uint64_t kStagePiece = 1ull << 20;

int stage_threads(const lp_pager* p) { return p->cfg.stage_threads ? (int)p->cfg.stage_threads : 4; }

void stage_copy(const lp_pager* p, void* dst, const void* src, uint64_t n) {
    const int64_t pieces = (int64_t)((n + kStagePiece - 1) / kStagePiece);
#pragma omp parallel for num_threads(stage_threads(p)) schedule(static) if (pieces > 1)
    for (int64_t i = 0; i < pieces; ++i) {
        const uint64_t o = (uint64_t)i * kStagePiece;
        memcpy(static_cast<uint8_t*>(dst) + o, static_cast<const uint8_t*>(src) + o, std::min(kStagePiece, n - o));
    }
}

// The blob's aligned span read from the pack in pieces (each 4096-aligned,
// as O_DIRECT wants).
bool stage_pack_read(lp_pager* p, uint16_t layer, uint16_t expert, void* dst) {
    uint64_t off = 0, n = 0;
    if (lp_pack_entry(p->pack, layer, expert, &off, &n) != LP_OK) return false;
    const uint64_t span = (n + kAlign - 1) / kAlign * kAlign;
    if (span > p->span) return false;
    const int64_t pieces = (int64_t)((span + kStagePiece - 1) / kStagePiece);
    int bad = 0;
#pragma omp parallel for num_threads(stage_threads(p)) schedule(static) reduction(+ : bad) if (pieces > 1)
    for (int64_t i = 0; i < pieces; ++i) {
        const uint64_t o = (uint64_t)i * kStagePiece;
        if (lp_pack_read_range(p->pack, off + o, static_cast<uint8_t*>(dst) + o, std::min(kStagePiece, span - o)))
            bad += 1;
    }
    return bad == 0;
}

// One I/O worker (pager.rs:650-718): its own copy stream and staging ring.
void worker_main(lp_pager* p, int wid) {
    hipStream_t stream = nullptr;
    std::vector<void*> ring;
    std::vector<hipEvent_t> ring_ev;
    std::string err;
    auto note_error = [&](const std::string& m) {
        std::lock_guard<std::mutex> g(p->mu);
        if (p->worker_err == LP_OK) {
            p->worker_err = LP_E_DEVICE;
            p->worker_msg = m;
        }
        p->fill_cv.notify_all();
    };
    if (hipSetDevice(p->device) != hipSuccess || hipStreamCreateWithFlags(&stream, hipStreamNonBlocking) != hipSuccess) {
        note_error("pager worker: no stream");
        return;
    }
    const uint32_t nring = p->cfg.ring_slots ? p->cfg.ring_slots : 2;
    for (uint32_t i = 0; i < nring; ++i) {
        void* b = nullptr;
        hipEvent_t e = nullptr;
        if (hipHostMalloc(&b, p->span, hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
            note_error("pager worker: cannot allocate its pinned staging ring");
            if (b) (void)hipHostFree(b);
            for (void* q : ring) (void)hipHostFree(q);
            for (hipEvent_t q : ring_ev) (void)hipEventDestroy(q);
            (void)hipStreamDestroy(stream);
            return;
        }
        ring.push_back(b);
        ring_ev.push_back(e);
    }
    size_t next = 0;
    for (;;) {
        Job job;
        {
            std::unique_lock<std::mutex> g(p->mu);
            p->jobs_cv.wait(g, [&] { return p->stop || !p->jobs.empty(); });
            if (p->jobs.empty()) break;  // stopping with nothing left
            job = p->jobs.front();
            p->jobs.pop_front();
        }
        const auto t0 = std::chrono::steady_clock::now();
        const size_t r = next++ % nring;
        bool ok = hipEventSynchronize(ring_ev[r]) == hipSuccess;  // its previous copy has landed
        if (ok) {
            if (p->cfg.source == LP_PAGER_SRC_HOST) {
                const uint8_t* src = reinterpret_cast<const uint8_t*>(p->cfg.host_blobs) +
                                     ((uint64_t)job.layer * p->cfg.experts_per_layer + job.expert) * p->cfg.host_stride;
                stage_copy(p, ring[r], src, p->cfg.blob_bytes);
            } else if (!(p->ram && ram_get(p->ram, job.layer, job.expert, ring[r]))) {
                ok = stage_pack_read(p, job.layer, job.expert, ring[r]);
                if (ok && p->ram) ram_put(p->ram, job.layer, job.expert, ring[r]);
            }
        }
        hipEvent_t done = nullptr;
        if (ok) {
            std::lock_guard<std::mutex> g(p->mu);
            if (job.release_after_fill) done = take_event(p);
        }
        ok = ok && hipMemcpyAsync(reinterpret_cast<void*>(slot_dev(p, job.slot)), ring[r], p->cfg.blob_bytes,
                                  hipMemcpyHostToDevice, stream) == hipSuccess &&
             hipEventRecord(p->fill_ev[job.slot], stream) == hipSuccess &&
             hipEventRecord(ring_ev[r], stream) == hipSuccess &&
             (!done || hipEventRecord(done, stream) == hipSuccess);
        {
            std::lock_guard<std::mutex> g(p->mu);
            if (ok) {
                p->fill[job.slot] = Fill::InFlight;
                p->bytes_fetched += p->cfg.blob_bytes;
                p->fetches += 1;
                p->fetch_counts[(size_t)job.layer * p->cfg.experts_per_layer + job.expert] += 1;
                if (done) p->prefetched.push_back(Deferred{done, {job.slot}});
                // pager.rs:677-686: the read-and-enqueue time of the fetch
                const double ms =
                    std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
                const double edges[6] = {1, 2, 5, 10, 20, 50};
                int bk = 0;
                while (bk < 6 && ms >= edges[bk]) ++bk;
                p->lat_buckets[bk] += 1;
            } else {
                if (p->worker_err == LP_OK) {
                    p->worker_err = LP_E_DEVICE;
                    p->worker_msg = "pager worker: reading or copying expert (" + std::to_string(job.layer) + ", " +
                                    std::to_string(job.expert) + ") failed";
                }
                p->fill[job.slot] = Fill::Empty;
                if (done) p->ev_pool.push_back(done);
                if (job.release_after_fill) lp_cache_release(p->cache, job.slot);
            }
            if (job.release_after_fill) p->pending_prefetch -= 1;
        }
        p->fill_cv.notify_all();
    }
    (void)hipStreamSynchronize(stream);
    for (void* b : ring) (void)hipHostFree(b);
    for (hipEvent_t e : ring_ev) (void)hipEventDestroy(e);
    (void)hipStreamDestroy(stream);
}

// Wait (host) until the slot's copy is enqueued; caller holds the lock.
int wait_enqueued(lp_pager* p, std::unique_lock<std::mutex>& g, uint32_t slot) {
    p->fill_cv.wait(g, [&] { return p->fill[slot] != Fill::Pending || p->worker_err != LP_OK; });
    if (p->fill[slot] == Fill::Pending || p->fill[slot] == Fill::Empty)
        return fail(p->worker_err != LP_OK ? p->worker_err : LP_E_DEVICE,
                    p->worker_msg.empty() ? "pager: fill failed" : p->worker_msg);
    return LP_OK;
}

// Make `cs` wait for the slot's fill (pager.rs:499-503); caller holds the lock.
int stream_wait_slot(lp_pager* p, std::unique_lock<std::mutex>& g, uint32_t slot, hipStream_t cs) {
    if (int r = wait_enqueued(p, g, slot)) return r;
    if (p->fill[slot] == Fill::InFlight) {
        hipError_t e = hipEventQuery(p->fill_ev[slot]);
        if (e == hipSuccess) {
            p->fill[slot] = Fill::Ready;
        } else if (e == hipErrorNotReady) {
            e = hipStreamWaitEvent(cs, p->fill_ev[slot], 0);
            if (e != hipSuccess) return hip_fail(e, "hipStreamWaitEvent");
        } else {
            return hip_fail(e, "fill event");
        }
    }
    return LP_OK;
}

// Pin the n experts of `layer` (misses scheduled); slots_out gets the slots.
// On failure every pin this call took is handed back.  Caller holds the lock.
int acquire_all(lp_pager* p, std::unique_lock<std::mutex>& g, uint16_t layer, const uint16_t* experts, int n,
                uint32_t* slots_out) {
    const uint32_t E = p->cfg.experts_per_layer;
    for (int i = 0; i < n; ++i)
        if (experts[i] >= E) return fail(LP_E_INVALID, "lp_pager_request: expert id out of range");
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
            } else if (p->pending_prefetch > 0 && p->worker_err == LP_OK) {
                p->fill_cv.wait(g);  // a prefetch's copy is being enqueued
            } else {
                return unwind(fail(LP_E_INVALID, "expert cache deadlock: every slot of the pool is pinned "
                                                 "with no release pending (handles held across a pass)"));
            }
        }
        if (r < 0) return unwind(r);
        pinned.push_back(slot);
        if (r == LP_LOOKUP_MISS) {
            table_update(p, layer, experts[i], slot, evicted);
            if (int q = schedule_fill(p, layer, experts[i], slot, false)) return unwind(q);
        }
        slots_out[i] = slot;
    }
    return LP_OK;
}

// The layer's slot table, refreshed in stream order on `cs`; caller holds the lock.
int refresh_table(lp_pager* p, uint16_t layer, hipStream_t cs) {
    const uint32_t E = p->cfg.experts_per_layer;
    const size_t r = p->stage_next++ % kRing;
    PCHK(hipEventSynchronize(p->stage_ev[r]));  // its previous copy has been consumed
    int32_t* st = p->stage + r * E;
    memcpy(st, p->host_tables + (size_t)layer * E, (size_t)E * 4);
    PCHK(hipMemcpyAsync(reinterpret_cast<void*>(lp_pager_slot_table(p, layer)), st, (size_t)E * 4,
                        hipMemcpyHostToDevice, cs));
    PCHK(hipEventRecord(p->stage_ev[r], cs));
    return LP_OK;
}

int pager_init(lp_ctx* ctx, const lp_pager_config* cfg, lp_pack* pack, lp_pager** out) {
    if (int r = lp_bind_thread(ctx)) {
        lp_pack_close(pack);
        return r;
    }
    lp_pager* p = new lp_pager();
    p->ctx = ctx;
    p->cfg = *cfg;
    p->pack = pack;
    p->device = lpi::ctx_device(ctx);
    p->span = cfg->span ? cfg->span : (cfg->blob_bytes + kAlign - 1) / kAlign * kAlign;
    if (p->span < cfg->blob_bytes || p->span % 256 || (pack && p->span % kAlign)) {
        lp_pager_free(p);
        return fail(LP_E_INVALID, "lp_pager_new: span must hold a blob and be 256-byte (pack: 4096-byte) aligned");
    }
    const uint32_t L = cfg->layers, E = cfg->experts_per_layer;
    if (cfg->reserve_bytes > 0) {
        // The arena is a cache, the first thing to give up for a co-tenant
        // of the card (PagerConfig::reserve_bytes, pager.rs:46-50): keep at
        // most as many slots per layer as leave reserve_bytes of device
        // memory free once the arena and the slot tables are allocated.
        size_t free_b = 0, total_b = 0;
        const hipError_t me = hipMemGetInfo(&free_b, &total_b);
        if (me != hipSuccess) {
            lp_pager_free(p);
            return hip_fail(me, "lp_pager: hipMemGetInfo");
        }
        const uint64_t tables = (uint64_t)L * E * 4, layer_slot = (uint64_t)L * p->span;
        const uint64_t room = (uint64_t)free_b > cfg->reserve_bytes + tables
                                  ? (uint64_t)free_b - cfg->reserve_bytes - tables : 0;
        const uint64_t fit = room / layer_slot;
        if (fit == 0) {
            lp_pager_free(p);
            return fail(LP_E_UNSUPPORTED, "lp_pager: " + std::to_string(free_b) + " bytes of device memory free; "
                                          "keeping " + std::to_string(cfg->reserve_bytes) + " free leaves no room "
                                          "for one slot per layer (" + std::to_string(layer_slot) + " bytes)");
        }
        if (fit < p->cfg.slots_per_layer) p->cfg.slots_per_layer = (uint32_t)fit;
    }
    const uint32_t S = p->cfg.slots_per_layer;
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
        p->fetch_counts.assign((size_t)L * E, 0);
        memset(p->host_tables, 0xff, (size_t)L * E * 4);
        p->fill.assign(total, Fill::Empty);
        p->fill_ev.assign(total, nullptr);
        for (uint64_t s = 0; s < total && e == hipSuccess; ++s)
            e = hipEventCreateWithFlags(&p->fill_ev[s], hipEventDisableTiming);
        p->stage_ev.assign(kRing, nullptr);
        for (size_t r = 0; r < kRing && e == hipSuccess; ++r)
            e = hipEventCreateWithFlags(&p->stage_ev[r], hipEventDisableTiming);
        if (!uses_workers(p)) {
            for (int i = 0; i < cfg->copy_streams && e == hipSuccess; ++i) {
                hipStream_t s = nullptr;
                e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
                if (e == hipSuccess) p->copy_streams.push_back(s);
            }
        }
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        lp_pager_free(p);
        return hip_fail(e, "lp_pager_new");
    }
    if (pack && cfg->ram_bytes >= p->span) {
        // pager.rs:69-113: slabs of one span, keys folded into the cache's ids
        RamTier* r = new RamTier();
        r->span = p->span;
        r->experts = E;
        const uint64_t slots = cfg->ram_bytes / p->span;
        r->bytes = (size_t)(slots * p->span);
        void* m = mmap(nullptr, r->bytes, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
        r->cache = m != MAP_FAILED ? lp_cache_new(1, (uint32_t)slots, (uint32_t)std::max<uint64_t>(slots, 64) * 4)
                                   : nullptr;
        if (m == MAP_FAILED || !r->cache) {
            if (m != MAP_FAILED) munmap(m, r->bytes);
            delete r;
            lp_pager_free(p);
            return fail(LP_E_INVALID, "lp_pager_new: cannot map the RAM tier");
        }
        r->base = static_cast<uint8_t*>(m);
        p->ram = r;
    }
    if (uses_workers(p)) {
        const uint32_t nw = cfg->io_threads ? cfg->io_threads : 4;
        for (uint32_t i = 0; i < nw; ++i) p->workers.emplace_back(worker_main, p, (int)i);
    }
    *out = p;
    return LP_OK;
}

}  // namespace

extern "C" {

int lp_pager_new(lp_ctx* ctx, const lp_pager_config* cfg, lp_pager** out) {
    if (!out) return fail(LP_E_INVALID, "lp_pager_new: null out");
    *out = nullptr;
    if (!ctx || !cfg) return fail(LP_E_INVALID, "lp_pager_new: null argument");
    if (cfg->source != LP_PAGER_SRC_PINNED && cfg->source != LP_PAGER_SRC_HOST)
        return fail(LP_E_INVALID, "lp_pager_new: source must be pinned or host memory (packs: lp_pager_open)");
    if (cfg->layers == 0 || cfg->experts_per_layer == 0 || cfg->experts_per_layer > 65536 ||
        cfg->slots_per_layer == 0 || cfg->blob_bytes == 0 || !cfg->host_blobs ||
        cfg->host_stride < cfg->blob_bytes || (cfg->source == LP_PAGER_SRC_PINNED &&
                                               (cfg->copy_streams < 1 || cfg->copy_streams > 8)) ||
        cfg->io_threads > 64 || cfg->ring_slots > 64)
        return fail(LP_E_INVALID, "lp_pager_new: bad configuration");
    return pager_init(ctx, cfg, nullptr, out);
}

int lp_pager_open(lp_ctx* ctx, const char* pack_path, const lp_pager_config* cfg, lp_pager** out) {
    if (!out) return fail(LP_E_INVALID, "lp_pager_open: null out");
    *out = nullptr;
    if (!ctx || !cfg || !pack_path) return fail(LP_E_INVALID, "lp_pager_open: null argument");
    lp_pack* pack = nullptr;
    if (int r = lp_pack_open(pack_path, cfg->direct, &pack)) return r;
    lp_pager_config c = *cfg;
    uint32_t L = 0, E = 0;
    uint64_t maxb = 0;
    lp_pack_info(pack, &L, &E, &maxb);
    // pager.rs:263-265: the pack defines layers, experts and the slot span
    if ((c.layers && c.layers != L) || (c.experts_per_layer && c.experts_per_layer != E)) {
        lp_pack_close(pack);
        return fail(LP_E_INVALID, "lp_pager_open: layers / experts differ from the pack's");
    }
    c.layers = L;
    c.experts_per_layer = E;
    c.blob_bytes = maxb;
    c.span = (maxb + kAlign - 1) / kAlign * kAlign;
    c.source = LP_PAGER_SRC_PACK;
    c.host_blobs = nullptr;
    if (c.slots_per_layer == 0 || c.io_threads > 64 || c.ring_slots > 64 || maxb == 0) {
        lp_pack_close(pack);
        return fail(LP_E_INVALID, "lp_pager_open: bad configuration");
    }
    return pager_init(ctx, &c, pack, out);
}

void lp_pager_free(lp_pager* p) {
    if (!p) return;
    {
        std::lock_guard<std::mutex> g(p->mu);
        p->stop = true;
    }
    p->jobs_cv.notify_all();
    for (std::thread& t : p->workers) t.join();
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
    if (p->ram) {
        munmap(p->ram->base, p->ram->bytes);
        lp_cache_free(p->ram->cache);
        delete p->ram;
    }
    lp_pack_close(p->pack);
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
    std::unique_lock<std::mutex> g(p->mu);
    if ((uint32_t)n > lp_cache_slots_per_partition(p->cache))
        return fail(LP_E_INVALID, "lp_pager_request: more experts than the pool holds (pager.rs:405-413)");
    if (int r = lp_bind_thread(p->ctx)) return r;
    if (int r = drain(p, p->deferred, false)) return r;
    if (int r = drain(p, p->prefetched, false)) return r;
    std::vector<uint32_t> slots((size_t)n);
    if (int r = acquire_all(p, g, layer, experts, n, slots.data())) return r;
    hipStream_t cs = (hipStream_t)compute;
    int rc = LP_OK;
    for (int i = 0; i < n && rc == LP_OK; ++i) rc = stream_wait_slot(p, g, slots[(size_t)i], cs);
    if (rc == LP_OK) rc = refresh_table(p, layer, cs);
    if (rc != LP_OK) {
        for (uint32_t s : slots) lp_cache_release(p->cache, s);
        return rc;
    }
    if (slots_out) memcpy(slots_out, slots.data(), (size_t)n * 4);
    return LP_OK;
}

int lp_pager_request_handles(lp_pager* p, uint16_t layer, const uint16_t* experts, int n,
                             lp_expert_handle* out) {
    if (!p || (n > 0 && (!experts || !out)) || n < 0 || layer >= p->cfg.layers)
        return fail(LP_E_INVALID, "lp_pager_request_handles: bad arguments");
    std::unique_lock<std::mutex> g(p->mu);
    if ((uint32_t)n > lp_cache_slots_per_partition(p->cache))
        return fail(LP_E_INVALID, "lp_pager_request_handles: more experts than the pool holds (pager.rs:405-413)");
    if (int r = lp_bind_thread(p->ctx)) return r;
    if (int r = drain(p, p->deferred, false)) return r;
    if (int r = drain(p, p->prefetched, false)) return r;
    std::vector<uint32_t> slots((size_t)n);
    if (int r = acquire_all(p, g, layer, experts, n, slots.data())) return r;
    for (int i = 0; i < n; ++i) {
        out[i].layer = layer;
        out[i].expert = experts[i];
        out[i].slot = slots[(size_t)i];
        out[i].dev = slot_dev(p, slots[(size_t)i]);
        // a pack's blobs differ in size: the handle carries this one's
        // (pager.rs:595-603 takes it from the pack index)
        uint64_t nb = p->cfg.blob_bytes;
        if (p->pack) lp_pack_entry(p->pack, layer, experts[i], nullptr, &nb);
        out[i].len = nb;
    }
    return LP_OK;
}

int lp_pager_wait_stream(lp_pager* p, const lp_expert_handle* h, lp_stream s) {
    if (!p || !h || h->slot >= p->fill.size()) return fail(LP_E_INVALID, "lp_pager_wait_stream: bad handle");
    std::unique_lock<std::mutex> g(p->mu);
    if (int r = lp_bind_thread(p->ctx)) return r;
    return stream_wait_slot(p, g, h->slot, (hipStream_t)s);
}

int lp_pager_refresh_table(lp_pager* p, uint16_t layer, lp_stream s) {
    if (!p || layer >= p->cfg.layers) return fail(LP_E_INVALID, "lp_pager_refresh_table: bad layer");
    std::lock_guard<std::mutex> g(p->mu);
    if (int r = lp_bind_thread(p->ctx)) return r;
    return refresh_table(p, layer, (hipStream_t)s);
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
    for (int i = 0; i < n; ++i)
        if (experts[i] >= E) return fail(LP_E_INVALID, "lp_pager_prefetch: expert id out of range");
    std::vector<uint32_t> pinned;
    for (int i = 0; i < n; ++i) {
        uint32_t slot = 0;
        int64_t evicted = -1;
        const int r = lp_cache_acquire(p->cache, lp_cache_fold(layer, experts[i], E), &slot, &evicted);
        if (r == LP_LOOKUP_HIT) {
            lp_cache_release(p->cache, slot);  // pager.rs:469
        } else if (r == LP_LOOKUP_MISS) {
            table_update(p, layer, experts[i], slot, evicted);
            if (int q = schedule_fill(p, layer, experts[i], slot, true)) {
                lp_cache_release(p->cache, slot);
                return q;
            }
            if (!uses_workers(p)) pinned.push_back(slot);
        }  // stalled: skipped (pager.rs:484)
    }
    if (pinned.empty()) return LP_OK;
    // pinned source: the pins drop once the fills have landed (pager.rs:711-713,
    // release_after_fill): an event behind every fill of this call (the
    // workers do the same per fill for the other sources)
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
        std::unique_lock<std::mutex> g(p->mu);
        if (p->fill[slot] == Fill::Pending)
            if (int r = wait_enqueued(p, g, slot)) return r;
        if (p->fill[slot] != Fill::InFlight) return LP_OK;
        ev = p->fill_ev[slot];
    }
    PCHK(hipEventSynchronize(ev));  // pager.rs:489-496
    std::lock_guard<std::mutex> g(p->mu);
    if (p->fill[slot] == Fill::InFlight) p->fill[slot] = Fill::Ready;
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
    std::unique_lock<std::mutex> g(p->mu);
    // every queued job enqueued, then every copy done
    p->fill_cv.wait(g, [&] { return (p->jobs.empty() && p->pending_prefetch == 0) || p->worker_err != LP_OK; });
    for (size_t s = 0; s < p->fill.size(); ++s)
        if (p->fill[s] == Fill::Pending)
            if (int r = wait_enqueued(p, g, (uint32_t)s)) return r;
    for (hipStream_t s : p->copy_streams) PCHK(hipStreamSynchronize(s));
    for (size_t s = 0; s < p->fill.size(); ++s)
        if (p->fill[s] == Fill::InFlight) {
            PCHK(hipEventSynchronize(p->fill_ev[s]));
            p->fill[s] = Fill::Ready;
        }
    if (int r = drain(p, p->deferred, true)) return r;
    if (int r = drain(p, p->prefetched, true)) return r;
    if (p->worker_err != LP_OK) return fail(p->worker_err, p->worker_msg);
    return LP_OK;
}

int lp_pager_expert_stats(lp_pager* p, uint64_t* counts, uint64_t n) {
    if (!p || (!counts && n)) return fail(LP_E_INVALID, "lp_pager_expert_stats: bad arguments");
    std::lock_guard<std::mutex> g(p->mu);
    const uint64_t m = std::min<uint64_t>(n, p->fetch_counts.size());
    for (uint64_t i = 0; i < m; ++i) counts[i] = p->fetch_counts[i];
    return (int)std::min<uint64_t>(p->fetch_counts.size(), 0x7fffffff);
}

int lp_pager_prewarm(lp_pager* p, const uint64_t* counts, uint64_t n) {
    if (!p || (!counts && n)) return fail(LP_E_INVALID, "lp_pager_prewarm: bad arguments");
    if (!p->ram || !p->pack) return 0;  // pager.rs:540-543: no RAM tier, nothing to warm
    const uint64_t total = std::min<uint64_t>(n, (uint64_t)p->cfg.layers * p->cfg.experts_per_layer);
    const uint64_t capacity = p->ram->bytes / p->ram->span;
    // the most-fetched experts that fit, read in pack order (pager.rs:544-567)
    std::vector<std::pair<uint64_t, uint64_t>> ranked;
    for (uint64_t i = 0; i < total; ++i)
        if (counts[i] > 0) ranked.emplace_back(counts[i], i);
    std::stable_sort(ranked.begin(), ranked.end(), [](const auto& a, const auto& b) { return a.first > b.first; });
    if (ranked.size() > capacity) ranked.resize(capacity);
    std::vector<uint64_t> idx;
    for (const auto& r : ranked) idx.push_back(r.second);
    std::sort(idx.begin(), idx.end());
    void* buf = nullptr;
    if (posix_memalign(&buf, kAlign, p->span) != 0) return fail(LP_E_INVALID, "lp_pager_prewarm: out of memory");
    int loaded = 0;
    for (uint64_t i : idx) {
        const uint16_t layer = (uint16_t)(i / p->cfg.experts_per_layer), expert = (uint16_t)(i % p->cfg.experts_per_layer);
        if (lp_pack_read_blob(p->pack, layer, expert, buf, p->span) < 0) {
            free(buf);
            return fail(LP_E_INVALID, "lp_pager_prewarm: pack read failed");
        }
        ram_put(p->ram, layer, expert, buf);
        ++loaded;
    }
    free(buf);
    return loaded;
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
    out->ram_hits = 0;
    for (int i = 0; i < 7; ++i) out->latency_ms_buckets[i] = p->lat_buckets[i];
    if (p->ram) {
        std::lock_guard<std::mutex> rg(p->ram->mu);
        out->ram_hits = p->ram->hits;
    }
    return LP_OK;
}

}  // extern "C"
