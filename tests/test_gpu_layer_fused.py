"""GPU parity of the one-launch decode layer (obs_layer_decode: forward_layer,
forward.rs:398-443, at the Qwen3-30B-A3B shape): the attention half and the
MoE half with its post-attention norm in one launch must give what the two
launches give, obs_attn_decode (x -> x1) followed by obs_moe_decode (x1 -> y,
x1 the residual), bit for bit: x1, y, the expert ids, the routing weights and
the key/value caches. Checked at several positions of a 4,096-position
cache, over consecutive launches (the launch's epoch advances), over graph
replays with new inputs written between them, and with the output written
over the input (the decoder's in-place step). The two launches themselves are
pinned against the oracle by test_gpu_attention_fused.py and
test_gpu_decode.py."""
import numpy as np
import pytest

import obsidian_hip as oh
from obsidian_hip import synth

pytestmark = pytest.mark.gpu

H, NH, NKV, HD, ML = 2048, 32, 4, 128, 4096
EPS, THETA = 1e-6, 1e7
E, K, I, G = 128, 8, 768, 64


@pytest.fixture(scope="module")
def layer(exe):
    rng = np.random.default_rng(3030)
    t = {}
    for name, (r, c) in (("q", (NH * HD, H)), ("k", (NKV * HD, H)), ("v", (NKV * HD, H)), ("o", (H, NH * HD))):
        t[name + "_w"], t[name + "_s"], t[name + "_b"] = synth.centered_quant(rng, r, c, 64)
    t["in_norm"] = synth.norm_weight(rng, H)
    t["q_norm"] = synth.norm_weight(rng, HD)
    t["k_norm"] = synth.norm_weight(rng, HD)
    attn = {k: exe.upload(v) for k, v in t.items()}
    m = synth.moe_layer(31, E, H, I, G)
    m["norm_w"] = synth.norm_weight(rng, H)
    moe = oh.MoeLayer.upload(exe, m)
    cfg = oh.MoeConfig(E, K, H, I, G, True, rms_eps=EPS)
    kc = synth.bf16_normal(rng, (NKV, ML, HD))
    vt = np.ascontiguousarray(synth.bf16_normal(rng, (NKV, ML, HD)).transpose(0, 2, 1))
    return attn, moe, cfg, kc, vt


class _Run:
    """One path's buffers: its own copies of the caches, x1, y, ids, weights."""

    def __init__(self, exe, kc, vt):
        self.kc, self.vc = exe.upload(kc), exe.upload(vt)
        self.x1 = exe.alloc(H, np.uint16)
        self.y = exe.alloc(H, np.uint16)
        self.ids = exe.alloc(K, np.int32)
        self.w = exe.alloc(K, np.float32)

    def two_launches(self, exe, attn, moe, cfg, x, state, y=None):
        exe.attn_decode(attn, x, self.kc, self.vc, ML, EPS, THETA, state, self.x1)
        exe.moe_decode(cfg, moe, self.x1, self.y if y is None else y, residual=self.x1, ids_out=self.ids,
                       w_out=self.w)

    def one_launch(self, exe, attn, moe, cfg, x, state, y=None):
        exe.layer_decode(attn, cfg, moe, x, self.kc, self.vc, ML, EPS, THETA, state, self.x1,
                         self.y if y is None else y, ids_out=self.ids, w_out=self.w)

    def result(self):
        return [b.download() for b in (self.x1, self.y, self.ids, self.w, self.kc, self.vc)]


def _same(a, b, what):
    names = ("x1", "y", "ids", "weights", "key cache", "value cache")
    for n, u, v in zip(names, a, b):
        assert np.array_equal(u.view(np.uint8), v.view(np.uint8)), f"{what}: {n} differs"


@pytest.mark.parametrize("pos", [0, 7, 1000, 4000, 4095])
def test_layer_decode_equals_the_two_launches(exe, layer, pos):
    attn, moe, cfg, kc, vt = layer
    rng = np.random.default_rng(3100 + pos)
    x = exe.upload(synth.bf16_normal(rng, H, 0.5))
    state = exe.upload(np.array([pos, 0], np.int32))
    a, b = _Run(exe, kc, vt), _Run(exe, kc, vt)
    a.two_launches(exe, attn, moe, cfg, x, state)
    b.one_launch(exe, attn, moe, cfg, x, state)
    exe.device_status()
    ra, rb = a.result(), b.result()
    _same(ra, rb, f"pos {pos}")
    assert np.all(np.isfinite(synth.bf16_bits_to_f32(rb[1])))
    assert len(set(rb[2].tolist())) == K


def test_layer_decode_consecutive_in_place(exe, layer):
    """Eight layers' worth of launches in a row at consecutive positions, each
    writing its output over its input as the decoder's step does (x <- y):
    every launch equals the two launches run on their own buffers."""
    attn, moe, cfg, kc, vt = layer
    rng = np.random.default_rng(3200)
    x0 = synth.bf16_normal(rng, H, 0.5)
    xa, xb = exe.upload(x0), exe.upload(x0)
    a, b = _Run(exe, kc, vt), _Run(exe, kc, vt)
    for step, pos in enumerate(range(3000, 3008)):
        state = exe.upload(np.array([pos, 0], np.int32))
        a.two_launches(exe, attn, moe, cfg, xa, state, y=xa)
        b.one_launch(exe, attn, moe, cfg, xb, state, y=xb)
        exe.device_status()
        assert np.array_equal(xa.download(), xb.download()), f"step {step}"
        _same(a.result()[2:], b.result()[2:], f"step {step}")


def test_layer_decode_graph_replay(exe, layer):
    """Captured once, replayed with new inputs written between replays (1-3
    replays each, the program's own work in between): every replay equals the
    two launches on the same input and position."""
    attn, moe, cfg, kc, vt = layer
    rng = np.random.default_rng(3300)
    x = exe.alloc(H, np.uint16)
    state = exe.alloc(2, np.int32)
    a, b = _Run(exe, kc, vt), _Run(exe, kc, vt)
    x.upload(synth.bf16_normal(rng, H, 0.5))
    state.upload(np.array([10, 0], np.int32))
    b.one_launch(exe, attn, moe, cfg, x, state)  # the workspace exists before the capture
    a.two_launches(exe, attn, moe, cfg, x, state)
    exe.sync()
    exe.capture_begin()
    b.one_launch(exe, attn, moe, cfg, x, state)
    g = exe.capture_end()
    try:
        for rep in range(6):
            pos = 2000 + 17 * rep
            x.upload(synth.bf16_normal(rng, H, 0.5))
            state.upload(np.array([pos, 0], np.int32))
            for _ in range(rep % 3 + 1):
                exe.graph_launch(g)
                a.two_launches(exe, attn, moe, cfg, x, state)
            exe.device_status()
            _same(a.result(), b.result(), f"replay {rep}")
    finally:
        exe.graph_destroy(g)


def test_layer_decode_rejects_what_it_cannot_run(exe, layer):
    """A MoE layer without the post-attention norm, a shape outside the fused
    decode's, misaligned caches and a context set to the 4-launch path are
    refused before any launch."""
    attn, moe, cfg, kc, vt = layer
    r = _Run(exe, kc, vt)
    x = exe.upload(synth.bf16_normal(np.random.default_rng(3400), H, 0.5))
    state = exe.upload(np.array([5, 0], np.int32))
    no_norm = oh.MoeLayer({k: v for k, v in moe.ptrs.items() if k != "norm_w"})
    cases = [(oh.MoeConfig(E, 4, H, I, G, True), moe, r.kc, oh.OBS_E_SHAPE),
             (cfg, no_norm, r.kc, oh.OBS_E_SHAPE),
             (cfg, moe, r.kc.ptr + 8, oh.OBS_E_ALIGN)]
    for c, m, kcp, code in cases:
        with pytest.raises(oh.ObsError) as ei:
            exe.layer_decode(attn, c, m, x, kcp, r.vc, ML, EPS, THETA, state, r.x1, r.y)
        assert ei.value.code == code
    exe.set_decode_path(oh.OBS_DECODE_MULTI)
    try:
        with pytest.raises(oh.ObsError) as ei:
            exe.layer_decode(attn, cfg, moe, x, r.kc, r.vc, ML, EPS, THETA, state, r.x1, r.y)
        assert ei.value.code == oh.OBS_E_UNSUPPORTED
    finally:
        exe.set_decode_path(oh.OBS_DECODE_AUTO)
    assert np.array_equal(r.kc.download(), kc) and np.array_equal(r.vc.download(), vt)
