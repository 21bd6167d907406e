"""The layer-stack driver (lp_moe_stack_forward; decode.rs:277-343 restricted
to the MoE block, batched as decode.rs:431-532) and its HIP-graph capture.

Both run the same kernels on the same inputs as a host loop of
lp_moe_forward calls, so the residual must come out bit-identical; the
per-layer oracle parity of that loop is test_gpu_fp32_paths.py's
test_stack_config1_inplace.  Graph replays are checked one by one against
the eager result, with eager work and synchronisations between them."""
import numpy as np
import pytest

import llmpager_amd as lp
from _gpu import DeviceLayer

pytestmark = pytest.mark.gpu

H = 2048


@pytest.fixture(scope="module")
def layers(cuda):
    Ls = [DeviceLayer(cuda, H=H, I=768, E=128, k=8, group=32, seed=91, layer=l) for l in range(4)]
    yield Ls
    for L in Ls:
        L.free()


def _fp32(n, seed):
    return np.random.default_rng(seed).standard_normal(n).astype(np.float32)


@pytest.mark.parametrize("T", [1, 8, 32])
def test_stack_matches_layer_loop(cuda, layers, T):
    h0 = _fp32(T * H, 900 + T).reshape(T, H)
    st = lp.MoeStack(cuda, [L.desc for L in layers])
    ws = cuda.alloc_device(st.ws_bytes(T))
    d_loop, d_stack = cuda.upload(h0), cuda.upload(h0)
    for L in layers:
        L.layer.forward(d_loop, d_loop, T, ws)
    st.forward(d_stack, T, ws)
    want = cuda.download(d_loop, (T, H), np.float32)
    got = cuda.download(d_stack, (T, H), np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert not np.array_equal(want, h0)
    for p in (ws, d_loop, d_stack):
        cuda.free_device(p)


@pytest.mark.parametrize("T", [1, 32])
def test_stack_graph_replays(cuda, layers, T):
    h0 = _fp32(T * H, 950 + T).reshape(T, H)
    st = lp.MoeStack(cuda, [L.desc for L in layers])
    s = cuda.stream()
    ws = cuda.alloc_device(st.ws_bytes(T))
    ws_e = cuda.alloc_device(st.ws_bytes(T))
    saved, dh, de = cuda.upload(h0), cuda.upload(h0), cuda.upload(h0)
    cuda.sync()
    st.forward(de, T, ws_e)
    want = cuda.download(de, (T, H), np.float32)
    g = st.capture(dh, T, ws, s)
    for rep in range(3):
        cuda.dtod_async(dh, saved, h0.nbytes, s)
        g.launch(s)
        cuda.sync_stream(s)
        got = cuda.download(dh, (T, H), np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), rep
        # eager work between replays
        cuda.dtod_async(de, saved, h0.nbytes, None)
        st.forward(de, T, ws_e)
        cuda.sync()
    g.close()
    cuda.sync()
    for p in (ws, ws_e, saved, dh, de):
        cuda.free_device(p)
    cuda.destroy_stream(s)


def test_stack_rejects_a_bad_layer_before_launching(cuda, layers):
    T = 1
    h0 = _fp32(T * H, 7).reshape(T, H)
    descs = [L.desc for L in layers]
    bad = lp.LayerDesc.from_buffer_copy(descs[2])
    bad.top_k = 99
    st = lp.MoeStack(cuda, [descs[0], descs[1], bad])
    ws = cuda.alloc_device(lp.ws_layout(descs[0], T).total)
    dh = cuda.upload(h0)
    with pytest.raises(lp.LpError) as ei:
        st.forward(dh, T, ws)
    assert "layer 2" in str(ei.value)
    assert np.array_equal(cuda.download(dh, (T, H), np.float32), h0)
    for p in (ws, dh):
        cuda.free_device(p)


def test_graph_keeps_its_counters_after_its_stream_is_gone(cuda, layers):
    # A graph holds its own routing arrival counters for its whole life: its
    # capture stream destroyed, a stream created afterwards (which would have
    # taken the freed counters) routes while the graph replays on a third
    # stream, with no ordering between the two; both stay bit-exact with the
    # eager result.
    T = 8
    h0 = _fp32(T * H, 990).reshape(T, H)
    st = lp.MoeStack(cuda, [L.desc for L in layers])
    s = cuda.stream()
    ws_g, ws_e = cuda.alloc_device(st.ws_bytes(T)), cuda.alloc_device(st.ws_bytes(T))
    dg, de, saved = cuda.upload(h0), cuda.upload(h0), cuda.upload(h0)
    cuda.sync()
    st.forward(de, T, ws_e)
    cuda.sync()
    want = cuda.download(de, (T, H), np.float32)
    g = st.capture(dg, T, ws_g, s)
    cuda.destroy_stream(s)
    s2, s3 = cuda.stream(), cuda.stream()
    for rep in range(4):
        cuda.dtod_async(dg, saved, h0.nbytes, s3)
        cuda.dtod_async(de, saved, h0.nbytes, s2)
        cuda.sync()
        g.launch(s3)
        st.forward(de, T, ws_e, s2)
        cuda.sync()
        got_g = cuda.download(dg, (T, H), np.float32)
        got_e = cuda.download(de, (T, H), np.float32)
        assert np.array_equal(got_g.view(np.uint32), want.view(np.uint32)), rep
        assert np.array_equal(got_e.view(np.uint32), want.view(np.uint32)), rep
    g.close()
    for p in (ws_g, ws_e, dg, de, saved):
        cuda.free_device(p)
    cuda.destroy_stream(s2)
    cuda.destroy_stream(s3)


def test_stack_rejects_a_short_workspace(cuda, layers):
    T = 8
    h0 = _fp32(T * H, 991).reshape(T, H)
    st = lp.MoeStack(cuda, [L.desc for L in layers])
    ws = cuda.alloc_device(st.ws_bytes(T) - 256)
    dh = cuda.upload(h0)
    s = cuda.stream()
    with pytest.raises(lp.LpError, match="workspace"):
        st.forward(dh, T, ws)
    with pytest.raises(lp.LpError, match="workspace"):
        st.capture(dh, T, ws, s)
    cuda.sync()
    assert np.array_equal(cuda.download(dh, (T, H), np.float32), h0)
    for p in (ws, dh):
        cuda.free_device(p)
    cuda.destroy_stream(s)
