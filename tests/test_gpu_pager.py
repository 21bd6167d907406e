"""The expert pager (pager.rs) on the GPU: fills are byte-exact copies of the
host blobs, cache decisions are the ExpertCache's (cache.rs), and a paged
layer stack computes what the all-resident oracle computes."""
import ctypes as C

import numpy as np
import pytest

import llmpager_amd as lp
import _oracle as O
from _gpu import align, rel_l2

pytestmark = pytest.mark.gpu

H, I, E, K, G = 128, 64, 8, 2, 32


class HostPack:
    """Every (layer, expert) blob, span-strided, as the pager's fill source:
    pinned host memory ("pinned"), pageable host memory staged through the
    pager's pinned ring ("host"), or a .llmpk pack file read by its I/O
    workers ("pack")."""

    def __init__(self, cuda, layers: int, seed: int, source: str = "pinned", tmp=None):
        self.cuda, self.layers, self.source = cuda, layers, source
        self.blob = lp.blob_bytes(H, I, G)
        self.span = align(self.blob)
        n = layers * E * self.span
        self.pin = cuda.alloc_pinned(n) if source == "pinned" else None
        self.view = (np.ctypeslib.as_array((C.c_uint8 * n).from_address(self.pin)) if self.pin
                     else np.zeros(n, np.uint8))
        for l in range(layers):
            lp.synth_blobs(E, self.span, H, I, G, seed, l, out=self.view[l * E * self.span:(l + 1) * E * self.span])
        self.path = None
        if source == "pack":
            self.path = str(tmp / f"pack{seed}.llmpk")
            w = lp.PackWriter(self.path, layers, E)
            for l in range(layers):
                for e in range(E):
                    w.add_blob(self.blob_of(l, e))
            w.finish()

    def blob_of(self, l: int, e: int) -> np.ndarray:
        o = (l * E + e) * self.span
        return self.view[o:o + self.blob]

    def pager_config(self, slots: int, streams: int = 2, glob: int = 0, decay: int = 256,
                     ram_bytes: int = 0) -> lp.PagerConfig:
        src = {"pinned": lp.PAGER_SRC_PINNED, "host": lp.PAGER_SRC_HOST, "pack": lp.PAGER_SRC_PACK}[self.source]
        return lp.PagerConfig(layers=self.layers, experts_per_layer=E, slots_per_layer=slots,
                              decay_interval=decay, blob_bytes=self.blob, span=0,
                              host_blobs=self.pin or self.view.ctypes.data, host_stride=self.span,
                              copy_streams=streams, global_pool=glob, source=src, io_threads=3, ring_slots=2,
                              ram_bytes=ram_bytes)

    def pager(self, slots: int, streams: int = 2, glob: int = 0, decay: int = 256, ram_bytes: int = 0) -> lp.Pager:
        cfg = self.pager_config(slots, streams, glob, decay, ram_bytes)
        if self.source == "pack":
            cfg.host_blobs, cfg.blob_bytes, cfg.host_stride = None, 0, 0
            return lp.Pager(self.cuda, cfg, pack_path=self.path)
        return lp.Pager(self.cuda, cfg)

    def free(self):
        if self.pin:
            self.cuda.free_pinned(self.pin)


SOURCES = ["pinned", "host", "pack"]


def _cache_model(layers: int, slots: int, glob: bool):
    # the pager's cache: per-layer pools decaying every 256 insertions, or one
    # pool that only decays on ticks (pager.rs:331-343)
    L = lp.lib()
    L.lp_cache_partitioned.restype = C.c_void_p
    L.lp_cache_partitioned.argtypes = [C.c_uint32] * 4
    if glob:
        return L.lp_cache_partitioned(1, E, slots * layers, 0xffffffff)
    return L.lp_cache_partitioned(layers, E, slots, 256)


@pytest.mark.parametrize("source", SOURCES)
def test_pager_fills_are_byte_exact(cuda, source, tmp_path):
    pk = HostPack(cuda, 2, seed=3, source=source, tmp=tmp_path)
    pg = pk.pager(slots=3)
    s = cuda.stream()
    slots = pg.request(1, [3, 5, 1], s)
    cuda.sync_stream(s)
    for e, sl in zip((3, 5, 1), slots):
        got = cuda.download(pg.arena + int(sl) * pg.span, (pk.blob,), np.uint8)
        assert np.array_equal(got, pk.blob_of(1, e)), (e, sl)
    table = cuda.download(pg.slot_table(1), (E,), np.int32)
    assert [table[e] for e in (3, 5, 1)] == list(slots)
    assert (np.delete(table, [3, 5, 1]) == -1).all()
    assert pg.metrics()["misses"] == 3
    pg.release_after(slots, s)
    pg.sync()
    pg.close()
    cuda.destroy_stream(s)
    pk.free()


@pytest.mark.parametrize("source", SOURCES)
def test_pager_prefetch_then_hit(cuda, source, tmp_path):
    pk = HostPack(cuda, 1, seed=4, source=source, tmp=tmp_path)
    pg = pk.pager(slots=4)
    pg.prefetch(0, [6, 2])
    s = cuda.stream()
    slots = pg.request(0, [2, 6, 7], s)   # two hits (prefetched), one miss
    cuda.sync_stream(s)
    m = pg.metrics()
    assert (m["hits"], m["misses"]) == (2, 3)
    for e, sl in zip((2, 6, 7), slots):
        assert np.array_equal(cuda.download(pg.arena + int(sl) * pg.span, (pk.blob,), np.uint8),
                              pk.blob_of(0, e))
    pg.release(slots)
    pg.sync()
    pg.close()
    cuda.destroy_stream(s)
    pk.free()


@pytest.mark.parametrize("source", SOURCES)
def test_pager_deadlock_is_an_error(cuda, source, tmp_path):
    # every slot pinned and nothing pending: the reference bails out rather than
    # hang (pager.rs:430-451); so does the C ABI
    pk = HostPack(cuda, 1, seed=5, source=source, tmp=tmp_path)
    pg = pk.pager(slots=2)
    s = cuda.stream()
    pg.request(0, [0, 1], s)
    with pytest.raises(RuntimeError, match="deadlock"):
        pg.request(0, [2], s)
    with pytest.raises(RuntimeError):
        pg.request(0, [0, 1, 2], s)     # more than the pool holds (pager.rs:405-413)
    cuda.sync_stream(s)
    pg.close()
    cuda.destroy_stream(s)
    pk.free()


@pytest.mark.parametrize("source", SOURCES)
@pytest.mark.parametrize("glob", [0, 1])
def test_paged_stack_matches_the_oracle(cuda, glob, source, tmp_path):
    # Two layers, 4 of 8 expert slots per layer (8 in one pool when glob): each
    # decode step routes on the device, reads the picks back, asks the pager for
    # them (misses copied on the copy streams), re-resolves the expert table and
    # runs the experts -- the reference's order (decode.rs:305-337) with the
    # routing on the GPU.  Hits and misses must be those of the ExpertCache fed
    # the same requests, and h must match the oracle with every expert resident.
    layers, slots, steps = 2, 4, 10
    pk = HostPack(cuda, layers, seed=6, source=source, tmp=tmp_path)
    pg = pk.pager(slots=slots, glob=glob)
    model = _cache_model(layers, slots, bool(glob))
    Lc = lp.lib()
    Lc.lp_cache_acquire.argtypes = [C.c_void_p, C.c_uint32, C.POINTER(C.c_uint32), C.POINTER(C.c_int64)]
    Lc.lp_cache_release.argtypes = [C.c_void_p, C.c_uint32]
    Lc.lp_cache_stats.argtypes = [C.c_void_p, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]
    Lc.lp_cache_free.argtypes = [C.c_void_p]
    Lc.lp_cache_decay_all.argtypes = [C.c_void_p]
    s = cuda.stream()
    routers = [lp.synth_bf16(E * H, 0.2, 6, 1000 + l) for l in range(layers)]
    d_routers = [cuda.upload(r) for r in routers]
    go, uo, do = lp.blob_offsets(H, I, G)
    descs = [lp.LayerDesc(hidden=H, inter=I, experts=E, top_k=K, group=G, gating=lp.GATING_SOFTMAX,
                          renorm=1, routed_scaling=1.0, router_w=d_routers[l], slot_table=pg.slot_table(l),
                          arena_base=pg.arena, slot_span=pg.span, gate_off=go, up_off=uo, down_off=do)
             for l in range(layers)]
    moe = [lp.MoeLayer(cuda, d) for d in descs]
    lay = lp.ws_layout(descs[0], 1)
    ws = cuda.alloc_device(lay.total)
    h0 = lp.synth_f32_bf16(steps * H, 1.0, 6, 2).reshape(steps, H)
    dh = cuda.upload(h0)
    for t in range(steps):
        ht = dh + t * H * 4
        for l in range(layers):
            moe[l].route(ht, 1, ws, s)
            cuda.sync_stream(s)
            ids = cuda.download(ws + lay.ids, (K,), np.int32)
            cnt = int(cuda.download(ws + lay.cnt, (1,), np.int32)[0])
            picks = sorted(set(int(e) for e in ids[:cnt]))
            got = pg.request(l, picks, s)
            ref_slots = []
            for e in picks:
                sl, ev = C.c_uint32(), C.c_int64()
                Lc.lp_cache_acquire(model, l * E + e, C.byref(sl), C.byref(ev))
                ref_slots.append(sl.value)
            assert list(got) == ref_slots, (t, l)
            moe[l].resolve(1, ws, s)
            moe[l].experts(ht, ht, 1, ws, s)
            pg.release_after(got, s)
            for sl in ref_slots:
                Lc.lp_cache_release(model, sl)
        pg.tick()
        if glob and (t + 1) % 4 == 0:   # pool_decay_tokens defaults to 4
            Lc.lp_cache_decay_all(model)
    cuda.sync_stream(s)
    got_h = cuda.download(dh, (steps, H), np.float32)
    hits, misses = C.c_uint64(), C.c_uint64()
    Lc.lp_cache_stats(model, C.byref(hits), C.byref(misses))
    m = pg.metrics()
    assert (m["hits"], m["misses"]) == (hits.value, misses.value)
    assert m["misses"] > slots and m["hits"] > 0        # evictions happened, and hits
    # the oracle with every expert resident
    want = h0.copy()
    for t in range(steps):
        for l in range(layers):
            desc = dict(hidden=H, inter=I, experts=E, top_k=K, group=G, gating=0, renorm=True,
                        routed_scaling=1.0, min_weight=0.0, router_w=routers[l], router_bias=None,
                        offsets=(go, uo, do))
            x = want[t:t + 1].copy()
            want[t:t + 1] = O.moe_layer(desc, [pk.blob_of(l, e) for e in range(E)], x, want[t:t + 1].copy())[0]
    assert rel_l2(got_h - h0, want - h0) <= 1e-3
    Lc.lp_cache_free(model)
    pg.sync()
    pg.close()
    for p in d_routers + [ws, dh]:
        cuda.free_device(p)
    cuda.destroy_stream(s)
    pk.free()


def test_pager_handles_and_ram_tier(cuda, tmp_path):
    # Pager::request -> ExpertHandle, wait_stream, then the layer's slot table
    # refreshed for the fused kernels (pager.rs:402-503), over a pack with a
    # RAM tier: a second round of the same experts after they were evicted
    # from VRAM is served from host RAM, byte-exact.
    pk = HostPack(cuda, 1, seed=9, source="pack", tmp=tmp_path)
    pg = pk.pager(slots=3, ram_bytes=8 * pk.span)
    s = cuda.stream()
    for rnd in range(2):
        for group in ([0, 1, 2], [3, 4, 5]):
            hs = pg.request_handles(0, group)
            assert [h.expert for h in hs] == group and all(h.len == pk.blob for h in hs)
            assert all(h.dev == pg.arena + h.slot * pg.span for h in hs)
            for h in hs:
                pg.wait_stream(h, s)
            pg.refresh_table(0, s)
            cuda.sync_stream(s)
            table = cuda.download(pg.slot_table(0), (E,), np.int32)
            for h in hs:
                assert table[h.expert] == h.slot
                assert np.array_equal(cuda.download(h.dev, (pk.blob,), np.uint8), pk.blob_of(0, h.expert))
            pg.release([h.slot for h in hs])
    m = pg.metrics()
    assert m["misses"] == 12 and m["ram_hits"] == 6   # the second round came from the RAM tier
    # the fetch latency histogram (pager.rs:677-686) counts every worker fetch once
    assert len(m["latency_ms_buckets"]) == 7 and sum(m["latency_ms_buckets"]) == m["fetches"] == 12
    pg.sync()
    pg.close()
    cuda.destroy_stream(s)


def test_pager_expert_stats_and_prewarm(cuda, tmp_path):
    # Pager::expert_stats / prewarm (pager.rs:532-567): the fill profile of one
    # pager warms the RAM tier of a fresh one, whose misses then come from RAM
    pk = HostPack(cuda, 1, seed=10, source="pack", tmp=tmp_path)
    pg = pk.pager(slots=2)
    s = cuda.stream()
    for group in ([0, 1], [2, 3], [0, 1]):
        pg.release(pg.request(0, group, s))
    stats = pg.expert_stats()
    assert stats.tolist() == [2, 2, 1, 1, 0, 0, 0, 0]
    pg.sync()
    pg.close()
    pg2 = pk.pager(slots=2, ram_bytes=3 * pk.span)
    assert pg2.prewarm(stats) == 3                     # the three most fetched that fit
    got = pg2.request(0, [0, 1], s)
    cuda.sync_stream(s)
    assert pg2.metrics()["ram_hits"] == 2
    for e, sl in zip((0, 1), got):
        assert np.array_equal(cuda.download(pg2.arena + int(sl) * pg2.span, (pk.blob,), np.uint8), pk.blob_of(0, e))
    pg2.release(got)
    pg2.sync()
    pg2.close()
    cuda.destroy_stream(s)


def test_pager_reserve_clamps_slots(cuda):
    # PagerConfig::reserve_bytes (pager.rs:46-50): device memory to leave
    # free.  The slot count drops until the arena and the slot tables leave
    # that much; a reserve that leaves no room for one slot per layer is an
    # error.  Memory is measured just before the pager allocates, so the
    # reserve is set to leave room for about 3 slots per layer.
    pk = HostPack(cuda, 2, seed=12, source="pinned")
    try:
        per_slot = 2 * pk.span
        free, _ = cuda.mem_info()
        cfg_slots = 6
        pg = pk.pager(slots=cfg_slots)
        assert pg.slots_per_layer == cfg_slots      # no reserve: as configured
        pg.close()
        cfg = lp.PagerConfig.from_buffer_copy(pk.pager_config(slots=cfg_slots))
        free, _ = cuda.mem_info()
        cfg.reserve_bytes = free - 3 * per_slot - 2 * E * 4 - 4096
        pg = lp.Pager(cuda, cfg)
        assert 1 <= pg.slots_per_layer <= 3, pg.slots_per_layer
        free_after, _ = cuda.mem_info()
        assert free_after >= cfg.reserve_bytes - (8 << 20)   # within allocation granularity
        # the clamped pager still works: fill and read back one expert
        s = cuda.stream()
        sl = pg.request(0, [5], s)
        cuda.sync_stream(s)
        assert np.array_equal(cuda.download(pg.arena + int(sl[0]) * pg.span, (pk.blob,), np.uint8),
                              pk.blob_of(0, 5))
        pg.release(sl)
        pg.sync()
        pg.close()
        cuda.destroy_stream(s)
        free, _ = cuda.mem_info()
        cfg.reserve_bytes = free + (1 << 30)
        with pytest.raises(lp.LpError, match="no room"):
            lp.Pager(cuda, cfg)
    finally:
        pk.free()


def test_pack_handles_carry_each_blobs_length(cuda, tmp_path):
    # ExpertHandle.len is the expert's own blob length from the pack index
    # (pager.rs:595-603), not the largest blob's: blobs of mixed sizes
    path = str(tmp_path / "mixed.llmpk")
    blob = lp.synth_blob(H, I, G, 3, 0, 0)
    w = lp.PackWriter(path, 1, E)
    lens = [blob.size + 100 * e for e in range(E)]
    for e in range(E):
        w.add_blob(np.concatenate([blob, np.full(lens[e] - blob.size, e, np.uint8)]))
    w.finish()
    cfg = lp.PagerConfig(slots_per_layer=4, decay_interval=256, io_threads=2, ring_slots=2)
    pg = lp.Pager(cuda, cfg, pack_path=path)
    s = cuda.stream()
    for group in ([0, 7, 3], [5, 1]):
        hs = pg.request_handles(0, group)
        assert [h.len for h in hs] == [lens[e] for e in group]
        for h in hs:
            pg.wait_stream(h, s)
        cuda.sync_stream(s)
        for h in hs:
            got = cuda.download(h.dev, (h.len,), np.uint8)
            assert np.array_equal(got[:blob.size], blob) and np.all(got[blob.size:] == h.expert)
        pg.release([h.slot for h in hs])
    pg.sync()
    pg.close()
    cuda.destroy_stream(s)
