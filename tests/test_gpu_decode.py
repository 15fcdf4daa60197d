"""GPU parity of the decode MoE half (forward.rs:421-441; the 30B-A3B decode layer shapes):
router ids/weights bit-exact with the oracle, layer output within 1e-2
relative of the oracle's fp64 evaluation on the same routing."""
import numpy as np
import pytest

import oracle as O
import obsidian_hip as oh
from obsidian_hip import synth

pytestmark = pytest.mark.gpu

REL_TOL = 1e-2  # north-star tolerance for layer outputs (bf16)


@pytest.fixture(scope="module")
def qwen_layer(exe):
    """One full Qwen3-30B-A3B-shaped MoE layer: 128 experts, H 2048, I 768."""
    t = synth.moe_layer(11, 128, 2048, 768, 64)
    return t, oh.MoeLayer.upload(exe, t), O.Layer(t, 128, 2048, 768, 64)


def _check_close(y_gpu_bits, y64):
    y = synth.bf16_bits_to_f32(y_gpu_bits).astype(np.float64)
    rel = np.linalg.norm(y - y64) / np.linalg.norm(y64)
    assert rel <= REL_TOL, rel
    floor = REL_TOL * np.sqrt(np.mean(y64 ** 2))
    assert np.all(np.abs(y - y64) <= REL_TOL * np.abs(y64) + floor)
    return rel


@pytest.fixture(params=[oh.OBS_DECODE_FUSED, oh.OBS_DECODE_MULTI], ids=["fused", "multi"])
def path(exe, request):
    exe.set_decode_path(request.param)
    yield request.param
    exe.set_decode_path(oh.OBS_DECODE_AUTO)
    exe.device_status()


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_moe_decode_config2(exe, qwen_layer, path, seed):
    t, layer, L = qwen_layer
    cfg = oh.MoeConfig(128, 8, 2048, 768, 64, True)
    rng = np.random.default_rng(1000 + seed)
    x = synth.bf16_normal(rng, 2048)
    dx = exe.upload(x)
    y = exe.alloc(2048, np.uint16)
    ids = exe.alloc(8, np.int32)
    w = exe.alloc(8, np.float32)
    exe.moe_decode(cfg, layer, dx, y, ids_out=ids, w_out=w)
    exe.device_status()
    gi, gw = ids.download(), w.download()
    _, ri, rw = O.router(L, x, 8, True)
    assert np.array_equal(gi, ri[0])
    assert np.array_equal(gw.view(np.uint32), rw[0].view(np.uint32))
    y64, _, _ = O.moe_decode(L, x, 8, True, ids=gi[None], w=gw[None])
    rel = _check_close(y.download(), y64[0])
    print(f"seed {seed}: ids {list(gi)} rel err {rel:.2e}")


@pytest.mark.parametrize("seed", [0, 1])
def test_moe_decode_with_post_attention_norm(exe, qwen_layer, path, seed):
    """forward.rs:419-440: x1n = rmsnorm(x1) feeds the router and experts and
    the combine accumulates into x1. With the layer's norm weight set, the
    layer equals the oracle on O.rmsnorm(x1): ids and weights bit-exact (the
    norm is bit-exact), output within 1e-2 of fp64 with x1 as residual."""
    t, _, L = qwen_layer
    rng = np.random.default_rng(2000 + seed)
    norm_w = synth.bf16_normal(rng, 2048, 0.5)
    layer = oh.MoeLayer.upload(exe, dict(t, norm_w=norm_w))
    cfg = oh.MoeConfig(128, 8, 2048, 768, 64, True, rms_eps=1e-6)
    x1 = synth.bf16_normal(rng, 2048, 3.0)
    dx = exe.upload(x1)
    y = exe.alloc(2048, np.uint16)
    ids = exe.alloc(8, np.int32)
    w = exe.alloc(8, np.float32)
    exe.moe_decode(cfg, layer, dx, y, residual=dx, ids_out=ids, w_out=w)
    exe.device_status()
    x1n = O.rmsnorm(x1, norm_w, 1e-6)
    _, ri, rw = O.router(L, x1n, 8, True)
    gi, gw = ids.download(), w.download()
    assert np.array_equal(gi, ri[0])
    assert np.array_equal(gw.view(np.uint32), rw[0].view(np.uint32))
    y64, _, _ = O.moe_decode(L, x1n, 8, True, ids=gi[None], w=gw[None])
    rel = _check_close(y.download(), y64[0] + synth.bf16_bits_to_f32(x1).astype(np.float64))
    print(f"norm seed {seed}: rel err {rel:.2e}")


def test_moe_decode_fused_matches_multi_and_repeats(exe, qwen_layer):
    """Many back-to-back fused launches (device-side epoch advances every
    launch) agree with the 4-launch path to bf16 rounding."""
    t, layer, L = qwen_layer
    cfg = oh.MoeConfig(128, 8, 2048, 768, 64, True)
    rng = np.random.default_rng(1050)
    xs = [synth.bf16_normal(rng, 2048) for _ in range(12)]
    dxs = [exe.upload(x) for x in xs]
    outs = {}
    for p in (oh.OBS_DECODE_FUSED, oh.OBS_DECODE_MULTI):
        exe.set_decode_path(p)
        ys = [exe.alloc(2048, np.uint16) for _ in xs]
        idb = [exe.alloc(8, np.int32) for _ in xs]
        for dx, y, i in zip(dxs, ys, idb):
            exe.moe_decode(cfg, layer, dx, y, ids_out=i)
        exe.device_status()
        outs[p] = ([synth.bf16_bits_to_f32(y.download()) for y in ys], [i.download() for i in idb])
    exe.set_decode_path(oh.OBS_DECODE_AUTO)
    for n in range(len(xs)):
        assert np.array_equal(outs[1][1][n], outs[2][1][n])
        a, b = outs[1][0][n].astype(np.float64), outs[2][0][n].astype(np.float64)
        assert np.linalg.norm(a - b) / np.linalg.norm(b) < 4e-3


def test_moe_decode_fused_graph_replay(exe, qwen_layer):
    """Captured once, replayed many times with new inputs written in between:
    every replay must see its own epoch and produce the right layer output."""
    t, layer, L = qwen_layer
    cfg = oh.MoeConfig(128, 8, 2048, 768, 64, True)
    exe.set_decode_path(oh.OBS_DECODE_FUSED)
    rng = np.random.default_rng(1060)
    dx = exe.alloc(2048, np.uint16)
    y = exe.alloc(2048, np.uint16)
    ids = exe.alloc(8, np.int32)
    w = exe.alloc(8, np.float32)
    dx.upload(synth.bf16_normal(rng, 2048))
    exe.moe_decode(cfg, layer, dx, y, ids_out=ids, w_out=w)  # workspace exists before capture
    exe.sync()
    exe.capture_begin()
    exe.moe_decode(cfg, layer, dx, y, ids_out=ids, w_out=w)
    g = exe.capture_end()
    try:
        for rep in range(6):
            x = synth.bf16_normal(rng, 2048)
            dx.upload(x)
            for _ in range(rep % 3 + 1):
                exe.graph_launch(g)
            exe.device_status()
            gi, gw = ids.download(), w.download()
            _, ri, rw = O.router(L, x, 8, True)
            assert np.array_equal(gi, ri[0])
            y64, _, _ = O.moe_decode(L, x, 8, True, ids=gi[None], w=gw[None])
            _check_close(y.download(), y64[0])
    finally:
        exe.graph_destroy(g)
        exe.set_decode_path(oh.OBS_DECODE_AUTO)


def test_moe_decode_residual_and_one_hot(exe, qwen_layer, path):
    t, layer, L = qwen_layer
    cfg = oh.MoeConfig(128, 8, 2048, 768, 64, True)
    rng = np.random.default_rng(1100)
    x = synth.bf16_normal(rng, 2048)
    res = synth.bf16_normal(rng, 2048, 100.0)
    dx = exe.upload(x)
    y0 = exe.alloc(2048, np.uint16)
    y1 = exe.alloc(2048, np.uint16)
    ids = exe.alloc(8, np.int32)
    w = exe.alloc(8, np.float32)
    exe.moe_decode(cfg, layer, dx, y0, ids_out=ids, w_out=w)
    exe.moe_decode(cfg, layer, dx, y1, residual=exe.upload(res), ids_out=ids, w_out=w)
    gi, gw = ids.download(), w.download()
    y64, _, _ = O.moe_decode(L, x, 8, True, ids=gi[None], w=gw[None])
    _check_close(y1.download(), y64[0] + synth.bf16_bits_to_f32(res).astype(np.float64))


def test_moe_decode_top1_equals_single_expert(exe, qwen_layer):
    """k = 1, norm_topk: the weight is exactly 1, output = the argmax expert."""
    t, layer, L = qwen_layer
    cfg = oh.MoeConfig(128, 1, 2048, 768, 64, True)
    rng = np.random.default_rng(1200)
    x = synth.bf16_normal(rng, 2048)
    y = exe.alloc(2048, np.uint16)
    ids = exe.alloc(1, np.int32)
    w = exe.alloc(1, np.float32)
    exe.moe_decode(cfg, layer, exe.upload(x), y, ids_out=ids, w_out=w)
    assert w.download()[0] == 1.0
    y64, _, _ = O.moe_decode(L, x, 1, True, ids=ids.download()[None], w=np.ones((1, 1), np.float32))
    _check_close(y.download(), y64[0])


def test_moe_decode_small_shapes(exe):
    """Other supported shapes: 16 experts, H 1024, I 256, top-4 without renorm."""
    E, H, I = 16, 1024, 256
    t = synth.moe_layer(12, E, H, I, 64)
    layer = oh.MoeLayer.upload(exe, t)
    L = O.Layer(t, E, H, I, 64)
    cfg = oh.MoeConfig(E, 4, H, I, 64, False)
    rng = np.random.default_rng(1300)
    x = synth.bf16_normal(rng, H)
    y = exe.alloc(H, np.uint16)
    ids = exe.alloc(4, np.int32)
    w = exe.alloc(4, np.float32)
    exe.moe_decode(cfg, layer, exe.upload(x), y, ids_out=ids, w_out=w)
    _, ri, rw = O.router(L, x, 4, False)
    assert np.array_equal(ids.download(), ri[0]) and np.array_equal(w.download(), rw[0])
    y64, _, _ = O.moe_decode(L, x, 4, False, ids=ri, w=rw)
    _check_close(y.download(), y64[0])


def test_moe_decode_rejects_bad_config(exe, qwen_layer):
    _, layer, _ = qwen_layer
    y = exe.alloc(2048, np.uint16)
    x = exe.alloc(2048, np.uint16)
    for cfg in (oh.MoeConfig(128, 9, 2048, 768, 64), oh.MoeConfig(128, 8, 2048, 768, 32),
                oh.MoeConfig(300, 8, 2048, 768, 64), oh.MoeConfig(128, 8, 3000, 768, 64)):
        with pytest.raises(oh.ObsError) as ei:
            exe.moe_decode(cfg, layer, x, y)
        assert ei.value.code == oh.OBS_E_SHAPE
    # the fused path refuses shapes it is not built for
    exe.set_decode_path(oh.OBS_DECODE_FUSED)
    try:
        with pytest.raises(oh.ObsError) as ei:
            exe.moe_decode(oh.MoeConfig(128, 4, 2048, 768, 64), layer, x, y)
        assert ei.value.code == oh.OBS_E_SHAPE
    finally:
        exe.set_decode_path(oh.OBS_DECODE_AUTO)
