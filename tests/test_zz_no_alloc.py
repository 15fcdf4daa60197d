"""obs_moe_decode_static, the decode entry point that allocates nothing: its
intermediates live in a file-scope device array per GPU. Called through the C
ABI (ctypes, no torch types) and compared with obs_moe_decode, which runs the
same kernels on context-allocated workspaces: outputs, ids and weights must be
identical bit for bit, on two calls in a row, the second with a smaller input
(a smaller model shape, which takes the 4-launch path), then once more at the
first shape (the fused path's exchange area keeps the earlier calls' epochs).
"""
import ctypes as C

import numpy as np
import pytest

import obsidian_hip as oh
from obsidian_hip import synth

pytestmark = pytest.mark.gpu


def _case(exe, seed, E, H, I, k, with_norm):
    t = synth.moe_layer(seed, E, H, I, 64)
    rng = np.random.default_rng(seed + 1)
    if with_norm:
        t["norm_w"] = synth.bf16_normal(rng, H, 0.5)
    layer = oh.MoeLayer.upload(exe, t)
    cfg = oh.MoeConfig(E, k, H, I, 64, True, rms_eps=1e-6)
    x = exe.upload(synth.bf16_normal(rng, H))
    res = exe.upload(synth.bf16_normal(rng, H, 4.0))
    return cfg, layer, x, res


def _run(exe, fn, cfg, layer, x, res):
    H, k = cfg.hidden, cfg.top_k
    y = exe.alloc(H, np.uint16)
    ids = exe.alloc(k, np.int32)
    w = exe.alloc(k, np.float32)
    c, l = cfg.to_c(), layer.to_c()
    rc = fn(exe.ctx, C.byref(c), C.byref(l), C.c_void_p(x.ptr), C.c_void_p(res.ptr), C.c_void_p(y.ptr),
            C.c_void_p(ids.ptr), C.c_void_p(w.ptr))
    assert rc == oh.OBS_OK, exe.last_error()
    exe.device_status()
    return y.download(), ids.download(), w.download()


def test_static_decode_equals_allocating_decode(exe):
    L = oh.lib()
    big = _case(exe, 3, 128, 2048, 768, 8, True)   # Qwen3-30B-A3B shape: the one-launch path
    small = _case(exe, 4, 64, 1024, 512, 4, False)  # smaller input: the 4-launch path
    for case in (big, small, big):
        ref = _run(exe, L.obs_moe_decode, *case)
        got = _run(exe, L.obs_moe_decode_static, *case)
        for a, b in zip(got, ref):
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
        assert np.all(ref[1] >= 0)


def test_static_decode_rejects_bad_shapes(exe):
    cfg, layer, x, res = _case(exe, 5, 16, 1024, 256, 4, False)
    bad = oh.MoeConfig(16, 4, 1024, 4096, 64, True)  # inter beyond what any decode path takes
    with pytest.raises(oh.ObsError) as ei:
        exe.moe_decode_static(bad, layer, x, exe.alloc(1024, np.uint16))
    assert ei.value.code == oh.OBS_E_SHAPE


def test_static_decode_captured_in_a_fresh_context():
    """No warm-up call: in a new context the first obs_moe_decode_static is
    recorded into a graph (nothing to allocate), and each replay, with eager
    calls between them, equals the eager result bit for bit."""
    with oh.ObsidianExecutor(0) as exe2:
        cfg, layer, x, res = _case(exe2, 6, 128, 2048, 768, 8, False)
        H, k = cfg.hidden, cfg.top_k
        y = exe2.alloc(H, np.uint16)
        ids = exe2.alloc(k, np.int32)
        w = exe2.alloc(k, np.float32)
        exe2.sync()
        exe2.capture_begin()
        exe2.moe_decode_static(cfg, layer, x, y, residual=res, ids_out=ids, w_out=w)
        g = exe2.capture_end()
        try:
            ref = _run(exe2, oh.lib().obs_moe_decode, cfg, layer, x, res)
            for _ in range(3):
                y.upload(np.zeros(H, np.uint16))
                exe2.graph_launch(g)
                exe2.device_status()
                got = (y.download(), ids.download(), w.download())
                for a, b in zip(got, ref):
                    assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
                _run(exe2, oh.lib().obs_moe_decode_static, cfg, layer, x, res)  # eager work between replays
        finally:
            exe2.graph_destroy(g)
