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


def _raw_pack(path, meta_json: bytes, index=None, blobs_end=12288):
    """A hand-made pack: header with the given metadata text, then the index
    entries given (offset, nbytes), then zeros up to blobs_end."""
    head = bytearray(4096)
    head[:8] = b"LLMPK1\0\0"
    head[8:16] = struct.pack("<II", 1, len(meta_json))
    head[16:16 + len(meta_json)] = meta_json
    body = bytearray(max(blobs_end - 4096, 0))
    for i, (off, nb) in enumerate(index or []):
        body[16 * i:16 * i + 16] = struct.pack("<QQ", off, nb)
    path.write_bytes(bytes(head) + bytes(body))
    return str(path)


def _meta(layers, experts):
    return ('{"model":"m","num_layers":%s,"experts_per_layer":%s,"dtype":"q4g32-gud"}' % (layers, experts)).encode()


def test_malformed_metadata_is_an_error_not_an_abort(tmp_path):
    """PackMeta (pack.rs:29-48) holds both counts as u16: text that is not an
    unsigned integer, or a value past 65535, is refused with an error (the
    C ABI never throws through its callers)."""
    ok = _raw_pack(tmp_path / "ok.llmpk", _meta(1, 1), [(8192, 100)])
    lp.Pack(ok).close()
    for layers, experts in (('"x"', 1), ("true", 1), ("-1", 1), ("1.5", 1), ("1e3", 1), (1, "null"),
                            (70000, 1), (1, 65536), ("99999999999999999999999", 1), (0, 1), (1, 0)):
        p = _raw_pack(tmp_path / "bad.llmpk", _meta(layers, experts), [(8192, 100)])
        with pytest.raises(lp.LpError):
            lp.Pack(p)


def test_oversized_counts_and_bad_index_rejected(tmp_path):
    """Counts that fit u16 but whose index the file cannot hold, and index
    entries outside the file or off the 4096 grid, are refused at open."""
    # 65535 x 65535 entries (64 GiB of index) in a 12 KiB file
    p = _raw_pack(tmp_path / "big.llmpk", _meta(65535, 65535))
    with pytest.raises(lp.LpError, match="shorter than its index"):
        lp.Pack(p)
    for entry in ((4096, 10),          # inside the index
                  (8192 + 512, 10),    # not 4096-aligned
                  (8192, 8192),        # runs past the end of the file
                  (1 << 62, 10),       # far outside
                  (8192, 1 << 63)):    # absurd length
        p = _raw_pack(tmp_path / "idx.llmpk", _meta(1, 1), [entry])
        with pytest.raises(lp.LpError, match="index entry 0"):
            lp.Pack(p)
