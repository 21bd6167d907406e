"""Every form of the decode kernels against the oracle, with fp32 activations.

The balanced gate/up comes as four kernels (16- or 8-step tiles; scales
through LDS windows for group 32, or read per lane for groups 64 and 128,
the reference's own q4g64 among them), the balanced down as two (6 steps, up
to 8), and a one-token batch takes down and combine in one launch
(`lp_moe_down_comb`, up to 8 steps, `_comb16` for 9..16, `_comb_rs` with
per-lane scales: groups 64 and 128, or scale rows not 16-byte aligned; it
also takes a shared MLP's down on its idle waves).  Each case names
the kernels it must reach; the per-kernel launch counts of the profiling
mode show that it did.  Layer outputs within rel-L2 1e-3 on the delta
h' - h, routing bit-exact given the device's logits (decode.rs:303-342)."""
import numpy as np
import pytest

import llmpager_amd as lp
import _oracle as O
from _gpu import DeviceLayer, rel_l2

pytestmark = pytest.mark.gpu


def fp32_normal(n: int, seed: int) -> np.ndarray:
    return np.random.default_rng(seed).standard_normal(n).astype(np.float32)


FORMS = [
    # H, I, group, T, kernels that must run
    (2048, 768, 64, 1, ("lp_moe_gateup_bal_rs", "lp_moe_down_comb_rs")),
    (2048, 1408, 32, 1, ("lp_moe_gateup_bal", "lp_moe_down_comb_rs")),
    (2048, 768, 64, 32, ("lp_moe_gateup_bal_rs", "lp_moe_down")),
    (2048, 768, 128, 8, ("lp_moe_gateup_bal_rs",)),
    (1024, 512, 32, 1, ("lp_moe_gateup_bal8", "lp_moe_down_comb")),
    (1024, 512, 32, 32, ("lp_moe_gateup_bal8", "lp_moe_down_bal")),
    (1024, 512, 64, 32, ("lp_moe_gateup_bal_rs8",)),
    (2048, 1536, 32, 1, ("lp_moe_gateup_bal", "lp_moe_down_comb16")),
    (2048, 1024, 32, 32, ("lp_moe_gateup_bal", "lp_moe_down_bal")),
    (2048, 768, 32, 32, ("lp_moe_gateup_bal", "lp_moe_down_bal6")),
]


# One token with a shared MLP (config 5's layout): its gate/up rides on the
# routed experts' balanced launch, and top-6 leaves two of the one-token
# down + combine's waves idle, which take its down (its group the routed
# one's) — one gate/up launch, no lp_moe_down_wide; with another group the
# shared MLP runs on its own.
SHARED5 = dict(E=64, k=6, gating=lp.GATING_SIGMOID, renorm=True, routed_scaling=2.5, min_weight=0.0,
               router_std=0.05)


@pytest.mark.parametrize("H,I,group,T,kernels,extra", [f + ({},) for f in FORMS] + [
    (2048, 1408, 32, 1, {"lp_moe_gateup_bal_sh": 1, "lp_moe_gateup_bal": 0, "lp_moe_down_comb_rs": 1,
                         "lp_moe_down_wide": 0}, dict(SHARED5, shared=(2816, 32))),
    (2048, 1408, 32, 16, {"lp_moe_gateup_bal_sh": 1, "lp_moe_gateup_bal": 0}, dict(SHARED5, shared=(2816, 32))),
    (2048, 1408, 32, 1, {"lp_moe_down_comb_rs": 1, "lp_moe_down_wide": 1}, dict(SHARED5, shared=(2816, 64))),
    (2048, 768, 64, 1, {"lp_moe_down_comb_rs": 1, "lp_moe_down_wide": 0}, dict(SHARED5, shared=(1536, 64))),
])
def test_decode_kernel_forms(cuda, H, I, group, T, kernels, extra):
    extra = dict(extra)
    E, k = extra.pop("E", 64), extra.pop("k", 8)
    bias = None
    if extra.get("gating") == lp.GATING_SIGMOID:
        bias = np.random.default_rng(T).standard_normal(E).astype(np.float32) * 0.05
    L = DeviceLayer(cuda, H=H, I=I, E=E, k=k, group=group, seed=H + I + group + T, bias=bias, **extra)
    x = fp32_normal(T * H, 7 * T + group).reshape(T, H)
    h = fp32_normal(T * H, 11 * T + group).reshape(T, H)
    lay = lp.ws_layout(L.desc, T)
    ws = cuda.alloc_device(lay.total)
    dx, dh = cuda.upload(x), cuda.upload(h)
    cuda.profile_reset()
    cuda.profile(True)
    L.layer.forward(dx, dh, T, ws)
    cuda.sync()
    counts = {kn: cuda.profile_read(kn)[1] for kn in kernels}
    cuda.profile(False)
    got = cuda.download(dh, (T, H), np.float32)
    logits = cuda.download(ws + lay.logits, (T, E), np.float32)
    ids = cuda.download(ws + lay.ids, (T, k), np.int32)
    wts = cuda.download(ws + lay.wts, (T, k), np.float32)
    cnt = cuda.download(ws + lay.cnt, (T,), np.int32)
    assert L.layer.status(ws, T)[1] == 0
    for p in (ws, dx, dh):
        cuda.free_device(p)
    want_n = kernels if isinstance(kernels, dict) else dict.fromkeys(kernels, 1)
    assert counts == want_n, counts
    want, wlog, wids, ww, wcnt = O.moe_layer(L.oracle_desc(), L.oracle_blobs(), x, h, threads=8,
                                             shared_blob=L.shared)
    L.free()
    assert np.array_equal(logits.view(np.uint32), wlog.view(np.uint32))
    assert np.array_equal(cnt, wcnt)
    for t in range(T):
        c = cnt[t]
        assert np.array_equal(ids[t, :c], wids[t, :c]), t
        assert np.array_equal(wts[t, :c].view(np.uint32), ww[t, :c].view(np.uint32)), t
    assert rel_l2(got - h, want - h) <= 1e-3
