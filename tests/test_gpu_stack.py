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
