"""GPU parity of the one-launch attention half of a decode layer
(obs_attn_decode; forward.rs:403-418) at the Qwen3-30B-A3B attention shape
with a 4,096-position cache: against the oracle's attention half, and against
the separate launches it replaces (obs_q4_gemv + obs_attn_prep +
obs_sdpa_decode + obs_q4_gemv), over consecutive launches (the exchange epoch
advances per launch).

Bars: x1 within 1e-2 of the fp64 oracle (2-norm, and elementwise with a floor
of 1e-2 rms); the appended key and value bit-exact with the separate
launches (the same mat-vec and norm/RoPE sequences) and every other cache
entry untouched; x1 within 1e-2 of the separate launches (the attention
splits are reduced in another order)."""
import numpy as np
import pytest

import oracle as O
from obsidian_hip import synth

pytestmark = pytest.mark.gpu

H, NH, NKV, HD, ML = 2048, 32, 4, 128, 4096
EPS, THETA = 1e-6, 1e7
OCFG = {"hidden": H, "n_heads": NH, "n_kv": NKV, "head_dim": HD, "eps": EPS, "theta": THETA}


def _f(b):
    return synth.bf16_bits_to_f32(b).astype(np.float64)


def _close(got, want, tol=1e-2):
    rel = float(np.linalg.norm(got - want) / np.linalg.norm(want))
    assert rel <= tol, rel
    floor = tol * np.sqrt(np.mean(want ** 2))
    assert np.all(np.abs(got - want) <= tol * np.abs(want) + floor), float(np.max(np.abs(got - want)))
    return rel


@pytest.fixture(scope="module")
def layer(exe):
    rng = np.random.default_rng(2024)
    t = {}
    for name, (r, c) in (("q", (NH * HD, H)), ("k", (NKV * HD, H)), ("v", (NKV * HD, H)), ("o", (H, NH * HD))):
        t[name + "_w"], t[name + "_s"], t[name + "_b"] = synth.centered_quant(rng, r, c, 64)
    t["in_norm"] = synth.norm_weight(rng, H)
    t["q_norm"] = synth.norm_weight(rng, HD)
    t["k_norm"] = synth.norm_weight(rng, HD)
    d = {k: exe.upload(v) for k, v in t.items()}
    kc = synth.bf16_normal(rng, (NKV, ML, HD))
    vc = synth.bf16_normal(rng, (NKV, ML, HD))
    return t, d, kc, vc


def _separate(exe, d, x, kc, vc, state):
    """The separate launches obs_attn_decode replaces, on copies of the caches."""
    q = exe.alloc(NH * HD, np.uint16)
    k = exe.alloc(NKV * HD, np.uint16)
    v = exe.alloc(NKV * HD, np.uint16)
    attn = exe.alloc(NH * HD, np.uint16)
    x1 = exe.alloc(H, np.uint16)
    exe.q4_gemv(x, H, [(d["q_w"], d["q_s"], d["q_b"], NH * HD, None, q, None),
                       (d["k_w"], d["k_s"], d["k_b"], NKV * HD, None, k, None),
                       (d["v_w"], d["v_s"], d["v_b"], NKV * HD, None, v, None)], norm_w=d["in_norm"], eps=EPS)
    exe.attn_prep(q, k, v, d["q_norm"], d["k_norm"], kc, vc, NH, NKV, HD, ML, EPS, THETA, state)
    ws = exe.alloc(exe.sdpa_workspace(NH, NKV, HD, ML), np.uint8)
    exe.sdpa_decode(q, kc, vc, attn, NH, NKV, HD, ML, state, ws)
    exe.q4_gemv(attn, NH * HD, [(d["o_w"], d["o_s"], d["o_b"], H, None, x1, x)])
    return x1


# positions 0..7 put the new token in each of the four value words a lane
# splices (and keep the context short enough that a wrong splice shows)
@pytest.mark.parametrize("pos", [0, 1, 2, 4, 6, 7, 33, 1000, 4063, 4095])
def test_attn_decode_vs_oracle_and_separate_launches(exe, layer, pos):
    t, d, kc0, vc0 = layer
    rng = np.random.default_rng(2100 + pos)
    x = synth.bf16_normal(rng, H, 0.5)
    dx = exe.upload(x)
    state = exe.upload(np.array([pos, 0], np.int32))
    vt0 = np.ascontiguousarray(vc0.transpose(0, 2, 1))
    kc_f, vc_f = exe.upload(kc0), exe.upload(vt0)
    x1 = exe.alloc(H, np.uint16)
    exe.attn_decode(d, dx, kc_f, vc_f, ML, EPS, THETA, state, x1)
    kc_s, vc_s = exe.upload(kc0), exe.upload(vt0)
    x1_s = _separate(exe, d, dx, kc_s, vc_s, state)
    gk, gv = kc_f.download(), vc_f.download()
    # the appended entries equal the separate launches' bit for bit; nothing else moved
    assert np.array_equal(gk, kc_s.download()) and np.array_equal(gv, vc_s.download())
    keep = np.ones(ML, bool)
    keep[pos] = False
    assert np.array_equal(gk[:, keep], kc0[:, keep]) and np.array_equal(gv[:, :, keep], vt0[:, :, keep])
    got = _f(x1.download())
    rel_s = _close(got, _f(x1_s.download()))
    kc_o, vc_o = kc0.copy(), vc0.copy()
    want = O.attention_half(t, x, kc_o, vc_o, pos, OCFG)
    rel_o = _close(got, _f(want))
    print(f"pos {pos}: rel vs oracle {rel_o:.2e}, vs separate launches {rel_s:.2e}")


def test_attn_decode_consecutive_launches(exe, layer):
    """Five launches in a row at consecutive positions on one cache (each
    launch's exchange slots carry a new epoch): every step equals the separate
    launches run on their own cache copy."""
    t, d, kc0, vc0 = layer
    rng = np.random.default_rng(2200)
    vt0 = np.ascontiguousarray(vc0.transpose(0, 2, 1))
    kc_f, vc_f = exe.upload(kc0), exe.upload(vt0)
    kc_s, vc_s = exe.upload(kc0), exe.upload(vt0)
    x1 = exe.alloc(H, np.uint16)
    for pos in range(2000, 2005):
        dx = exe.upload(synth.bf16_normal(rng, H, 0.5))
        state = exe.upload(np.array([pos, 0], np.int32))
        exe.attn_decode(d, dx, kc_f, vc_f, ML, EPS, THETA, state, x1)
        x1_s = _separate(exe, d, dx, kc_s, vc_s, state)
        _close(_f(x1.download()), _f(x1_s.download()))
    assert np.array_equal(kc_f.download(), kc_s.download()) and np.array_equal(vc_f.download(), vc_s.download())
    exe.device_status()  # raises if a cross-workgroup wait timed out


def test_attn_decode_rejects_misaligned_caches(exe, layer):
    """Each lane reads its 8 value positions as one 16-byte load, so a value
    cache (or key cache, or x) off a 16-byte boundary is refused before any
    launch, and nothing is written."""
    import obsidian_hip as oh
    t, d, kc0, vc0 = layer
    vt0 = np.ascontiguousarray(vc0.transpose(0, 2, 1))
    kc, vc = exe.upload(kc0), exe.upload(vt0)
    x = exe.upload(synth.bf16_normal(np.random.default_rng(2300), H, 0.5))
    state = exe.upload(np.array([100, 0], np.int32))
    x1 = exe.alloc(H, np.uint16)
    for args in ((x, kc, vc.ptr + 8), (x, kc.ptr + 8, vc), (x.ptr + 8, kc, vc)):
        with pytest.raises(oh.ObsError) as ei:
            exe.attn_decode(d, args[0], args[1], args[2], ML, EPS, THETA, state, x1)
        assert ei.value.code == oh.OBS_E_ALIGN
    assert np.array_equal(kc.download(), kc0) and np.array_equal(vc.download(), vt0)
