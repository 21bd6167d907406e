"""The .llmpk pack (crates/llmpager-core/src/pack.rs) written and read through
the C ABI: the reference's own pack tests restated (round trip with
varying, non-aligned sizes; an incomplete pack is rejected; an O_DIRECT read
where the filesystem supports it), plus the on-disk header and index layout
(pack.rs:1-16) checked byte by byte."""
import json
import struct

import numpy as np
import pytest

import llmpager_amd as lp


def blob_for(layer, expert, nbytes):
    # pack.rs:329-333
    return ((layer * 31 + expert * 7 + np.arange(nbytes)) % 256).astype(np.uint8)


def test_round_trip(tmp_path):
    path = str(tmp_path / "t.llmpk")
    w = lp.PackWriter(path, 3, 4, model="synthetic", dtype="q4_gs64")
    sizes = {}
    for l in range(3):
        for e in range(4):
            sizes[l, e] = 1000 + l * 500 + e * 13   # varying, non-aligned sizes exercise padding
            w.add_blob(blob_for(l, e, sizes[l, e]))
    w.finish()
    r = lp.Pack(path)
    assert (r.layers, r.experts, r.max_blob) == (3, 4, max(sizes.values()))
    for (l, e), n in sizes.items():
        off, nb = r.entry(l, e)
        assert nb == n and off % 4096 == 0
        assert np.array_equal(r.read_blob(l, e), blob_for(l, e, n))
    r.close()
    raw = open(path, "rb").read()
    assert raw[:8] == b"LLMPK1\0\0"
    ver, jl = struct.unpack("<II", raw[8:16])
    meta = json.loads(raw[16:16 + jl])
    assert ver == 1 and meta == {"model": "synthetic", "num_layers": 3, "experts_per_layer": 4, "dtype": "q4_gs64"}
    idx = np.frombuffer(raw[4096:4096 + 12 * 16], np.uint64).reshape(12, 2)
    assert idx[0, 0] == 8192 and all(idx[i + 1, 0] == idx[i, 0] + (idx[i, 1] + 4095) // 4096 * 4096 for i in range(11))
    assert len(raw) == idx[-1, 0] + (idx[-1, 1] + 4095) // 4096 * 4096


def test_incomplete_pack_rejected(tmp_path):
    w = lp.PackWriter(str(tmp_path / "t.llmpk"), 1, 2, model="x", dtype="raw")
    w.add_blob(np.array([1, 2, 3], np.uint8))
    with pytest.raises(lp.LpError):
        w.finish()


def test_o_direct_read(tmp_path):
    path = str(tmp_path / "t.llmpk")
    w = lp.PackWriter(path, 1, 1, model="x", dtype="raw")
    want = blob_for(0, 0, 8192)
    w.add_blob(want)
    w.finish()
    try:
        r = lp.Pack(path, direct=True)
    except lp.LpError:
        pytest.skip("this filesystem refuses O_DIRECT (pack.rs:392-397 skips the same way)")
    assert np.array_equal(r.read_blob(0, 0), want)
    r.close()


def test_not_a_pack(tmp_path):
    path = tmp_path / "x.llmpk"
    path.write_bytes(b"\0" * 8192)
    with pytest.raises(lp.LpError):
        lp.Pack(str(path))
