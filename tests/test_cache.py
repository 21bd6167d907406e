"""The reference's ExpertCache tests (crates/llmpager-core/src/cache.rs:247-416),
ported one for one onto the C++ restatement behind the C ABI."""
import ctypes as C

import pytest

import llmpager_amd as lp

HIT, MISS, STALLED = 0, 1, 2


class Cache:
    def __init__(self, ptr):
        assert ptr
        self.p = ptr
        L = lp.lib()
        self.L = L

    @classmethod
    def new(cls, layers, slots, decay):
        return cls(lp.lib().lp_cache_new(layers, slots, decay))

    @classmethod
    def partitioned(cls, parts, ids_per, slots, decay):
        return cls(lp.lib().lp_cache_partitioned(parts, ids_per, slots, decay))

    def acquire(self, id_):
        slot, ev = C.c_uint32(), C.c_int64()
        r = self.L.lp_cache_acquire(self.p, id_, C.byref(slot), C.byref(ev))
        if r == HIT:
            return ("hit", slot.value)
        if r == MISS:
            return ("miss", slot.value, None if ev.value < 0 else ev.value)
        assert r == STALLED
        return ("stalled",)

    def lookup_ready(self, id_):
        slot = C.c_uint32()
        return slot.value if self.L.lp_cache_lookup_ready(self.p, id_, C.byref(slot)) == 1 else None

    def publish(self, s):
        assert self.L.lp_cache_publish(self.p, s) == 0

    def release(self, s):
        assert self.L.lp_cache_release(self.p, s) == 0

    def is_ready(self, s):
        return self.L.lp_cache_is_ready(self.p, s) == 1

    def decay_all(self):
        self.L.lp_cache_decay_all(self.p)

    def is_wedged(self, id_):
        return self.L.lp_cache_is_wedged(self.p, id_) == 1

    def stats(self):
        h, m = C.c_uint64(), C.c_uint64()
        self.L.lp_cache_stats(self.p, C.byref(h), C.byref(m))
        return h.value, m.value

    def __del__(self):
        if getattr(self, "p", None):
            self.L.lp_cache_free(self.p)


@pytest.fixture(autouse=True, scope="module")
def _sigs():
    L = lp.lib()
    vp = C.c_void_p
    L.lp_cache_new.restype = vp
    L.lp_cache_new.argtypes = [C.c_uint16, C.c_uint32, C.c_uint32]
    L.lp_cache_partitioned.restype = vp
    L.lp_cache_partitioned.argtypes = [C.c_uint32] * 4
    L.lp_cache_free.argtypes = [vp]
    L.lp_cache_fold.restype = C.c_uint32
    L.lp_cache_fold.argtypes = [C.c_uint16, C.c_uint16, C.c_uint32]
    L.lp_cache_acquire.argtypes = [vp, C.c_uint32, C.POINTER(C.c_uint32), C.POINTER(C.c_int64)]
    L.lp_cache_lookup_ready.argtypes = [vp, C.c_uint32, C.POINTER(C.c_uint32)]
    for n in ("lp_cache_publish", "lp_cache_release", "lp_cache_is_ready", "lp_cache_is_wedged"):
        getattr(L, n).argtypes = [vp, C.c_uint32]
    L.lp_cache_decay_all.argtypes = [vp]
    L.lp_cache_stats.argtypes = [vp, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]
    yield


def fold(layer, expert, epl):
    return lp.lib().lp_cache_fold(layer, expert, epl)


def test_hit_after_miss():
    c = Cache.new(1, 4, 1000)
    r = c.acquire(7)
    assert r[0] == "miss" and r[2] is None
    slot = r[1]
    c.publish(slot)
    c.release(slot)
    assert c.acquire(7) == ("hit", slot)
    assert c.is_ready(slot)
    assert c.stats() == (1, 1)


def test_evicts_lowest_freq_unpinned():
    c = Cache.new(1, 2, 1000)
    for e in (0, 1):
        r = c.acquire(e)
        assert r[0] == "miss"
        c.publish(r[1])
        c.release(r[1])
    for _ in range(3):
        r = c.acquire(1)
        assert r[0] == "hit"
        c.release(r[1])
    r = c.acquire(2)
    assert r[0] == "miss" and r[2] == 0


def test_pinned_slots_are_not_victims():
    c = Cache.new(1, 1, 1000)
    r = c.acquire(0)
    assert r[0] == "miss"
    assert c.acquire(1) == ("stalled",)
    c.release(r[1])
    r = c.acquire(1)
    assert r[0] == "miss" and r[2] == 0


def test_decay_halves_frequencies():
    c = Cache.new(1, 2, 2)
    r = c.acquire(0)
    c.release(r[1])
    for _ in range(7):
        r = c.acquire(0)
        assert r[0] == "hit"
        c.release(r[1])
    r = c.acquire(1)
    c.release(r[1])
    r = c.acquire(2)
    c.release(r[1])
    r = c.acquire(3)
    assert r[0] == "miss" and r[2] != 0


def test_lookup_ready_never_inserts():
    c = Cache.new(1, 2, 1000)
    assert c.lookup_ready(3) is None
    r = c.acquire(3)
    assert c.lookup_ready(3) is None
    c.publish(r[1])
    c.release(r[1])
    got = c.lookup_ready(3)
    assert got == r[1]
    c.release(got)


def test_layers_are_independent():
    c = Cache.partitioned(2, 128, 1, 1000)
    a, b = fold(0, 5, 128), fold(1, 5, 128)
    s0 = c.acquire(a)[1]
    s1 = c.acquire(b)[1]
    assert s0 != s1
    c.release(s0)
    c.release(s1)
    assert c.acquire(a)[0] == "hit"
    assert c.acquire(b)[0] == "hit"


def test_fold_round_trips_layer_and_expert():
    assert fold(0, 0, 128) == 0
    assert fold(0, 127, 128) == 127
    assert fold(1, 0, 128) == 128
    assert fold(47, 127, 128) == 47 * 128 + 127


def test_one_partition_lets_a_hot_layer_take_more_slots():
    c = Cache.partitioned(1, 128, 4, 1000)
    for _ in range(3):
        for e in range(3):
            r = c.acquire(fold(0, e, 128))
            assert r[0] != "stalled"
            if r[0] == "miss":
                c.publish(r[1])
            c.release(r[1])
    id1 = fold(1, 0, 128)
    r = c.acquire(id1)
    assert r[0] == "miss"
    c.publish(r[1])
    c.release(r[1])
    for e in range(3):
        assert c.acquire(fold(0, e, 128))[0] == "hit"
    assert c.acquire(id1)[0] == "hit"


def test_decay_all_halves_every_partition():
    c = Cache.partitioned(2, 128, 2, 1_000_000)
    for layer, expert in ((0, 1), (1, 1)):
        id_ = fold(layer, expert, 128)
        r = c.acquire(id_)
        assert r[0] == "miss"
        c.publish(r[1])
        c.release(r[1])
        for _ in range(7):
            r = c.acquire(id_)
            assert r[0] == "hit"
            c.release(r[1])
    c.decay_all()
    for layer in (0, 1):
        r = c.acquire(fold(layer, 9, 128))
        assert r[0] == "miss"
        c.release(r[1])
        assert c.acquire(fold(layer, 1, 128))[0] == "hit"


def test_wedged_only_when_everything_is_pinned_and_ready():
    c = Cache.new(1, 2, 1000)
    assert not c.is_wedged(0)
    a = c.acquire(0)[1]
    b = c.acquire(1)[1]
    assert not c.is_wedged(0)
    c.publish(a)
    c.publish(b)
    assert c.is_wedged(0)
    c.release(a)
    assert not c.is_wedged(0)


def test_release_without_acquire_is_an_error():
    # the reference asserts (cache.rs:209); the C ABI reports LP_E_INVALID
    c = Cache.new(1, 2, 1000)
    assert lp.lib().lp_cache_release(c.p, 0) != 0


def test_new_puts_every_id_in_partition_zero():
    # cache.rs:71-73 passes u32::MAX as ids_per_partition: part_of sends every
    # id below it to partition 0, so new(2, 1, ..) behaves as one pool of 1 slot
    c = Cache.new(2, 1, 1000)
    r = c.acquire(fold(0, 1, 128))
    assert c.acquire(fold(1, 1, 128)) == ("stalled",)
    c.release(r[1])
