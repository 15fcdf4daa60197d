"""GPU parity of the reference's routing rule in every routing path.

The reference stores each router logit as a half (dequant_matvec_8bit.metal:30),
runs the softmax and the top-k on those halves with ties to the lower id, and
stores the weights as halves (moe_routing_topk.metal:24-56). The paths checked
here: the standalone router (obs_q8_gate_logits + obs_route_topk), the fused
one-launch decode, the four-launch decode and the prefill's computed routing.

Bars: logits, ids and weights bit-exact with the oracle (its router follows the
kernels' documented logit reduction order and ORC_ROUTE_REF), on inputs built
to force f16 ties: duplicated router rows (equal logits) and rows one 8-bit step
apart in a column whose activation is small (fp32 logits that differ by less
than one f16 step, larger at the higher id, so the two rules order them
differently).
"""
import numpy as np
import pytest

import oracle as O
import obsidian_hip as oh
from obsidian_hip import synth

pytestmark = pytest.mark.gpu

E, H, I, K = 128, 2048, 768, 8
DUP = [(a, a + 64) for a in range(0, 12)]          # row a + 64 copies row a
NEAR = [(a, a + 64) for a in range(16, 28)]        # row a + 64 = row a, one step more in column 0


def _tie_layer(seed: int, router_scale: float):
    t = synth.moe_layer(seed, E, H, I, 64)
    s = synth.bf16_bits_to_f32(t["router_s"]) * np.float32(router_scale)
    b = synth.bf16_bits_to_f32(t["router_b"]) * np.float32(router_scale)
    t["router_s"], t["router_b"] = synth.f32_to_bf16_bits(s), synth.f32_to_bf16_bits(b)
    rw = t["router_w"].copy()
    lo8 = ~np.uint32(0xFF)
    for a, c in DUP + NEAR:
        rw[c] = rw[a]
        t["router_s"][c] = t["router_s"][a]
        t["router_b"][c] = t["router_b"][a]
    for a, c in NEAR:
        rw[a, 0] = (rw[a, 0] & lo8) | np.uint32(100)
        rw[c, 0] = (rw[c, 0] & lo8) | np.uint32(101)
    t["router_w"] = rw
    return t


def _inputs(seed: int, T: int):
    x = synth.bf16_normal(np.random.default_rng(seed), (T, H))
    x[:, 0] = 0x3B80  # 2^-8: the NEAR rows' logits differ by about s * 2^-8
    return x


def _tie_pairs_seen(ids: np.ndarray) -> int:
    """(token, pair) cases where both rows of a forced pair were chosen."""
    n = 0
    for row in ids:
        r = set(int(v) for v in row)
        n += sum(1 for a, c in DUP + NEAR if a in r and c in r)
    return n


@pytest.fixture(scope="module", params=[1.0, 1.0 / 32.0], ids=["sd100", "sd4"])
def tie_model(request, exe):
    t = _tie_layer(77, request.param)
    return t, oh.MoeLayer.upload(exe, t), O.Layer(t, E, H, I, 64)


@pytest.mark.parametrize("scale", [1.0, 1.0 / 32.0], ids=["sd100", "sd4"])
def test_router_3000_tokens_both_rules(exe, scale):
    """obs_q8_gate_logits + obs_route_topk on 3,000 tokens: logits bit-exact;
    ids and weights bit-exact under the reference rule and under the fp32 rule;
    the two rules differ on some tokens (so the rounding is exercised)."""
    w8, s8, b8 = synth.quant_tensor(np.random.default_rng(6), E, H, 8, 64)
    s8 = synth.f32_to_bf16_bits(synth.bf16_bits_to_f32(s8) * np.float32(scale))
    b8 = synth.f32_to_bf16_bits(synth.bf16_bits_to_f32(b8) * np.float32(scale))
    T = 3000
    x = synth.bf16_normal(np.random.default_rng(7), (T, H))
    dlg = exe.alloc((T, E), np.float32)
    exe.q8_gate_logits(exe.upload(w8), exe.upload(s8), exe.upload(b8), exe.upload(x), dlg, T, H, E)
    lg = dlg.download()
    xf = synth.bf16_bits_to_f32(x)
    ref_lg = np.stack([O.qmatvec("lanes", 8, w8, s8, b8, xf[i], H, E) for i in range(0, T, 97)])
    assert np.array_equal(lg[::97].view(np.uint32), ref_lg.view(np.uint32))
    got = {}
    for rule in (O.ROUTE_REF, O.ROUTE_F32):
        ids = exe.alloc((T, K), np.int32)
        w = exe.alloc((T, K), np.float32)
        exe.route_topk(dlg, ids, w, T, E, K, True, rule=rule)
        gi, gw = ids.download(), w.download()
        ri, rw = O.route_topk(lg, K, True, O.SUM_WAVE, rule=rule)
        assert np.array_equal(gi, ri), rule
        assert np.array_equal(gw.view(np.uint32), rw.view(np.uint32)), rule
        got[rule] = gi
    # the reference's serial softmax sum gives the same ids under its rule
    si, _ = O.route_topk(lg, K, True, O.SUM_SERIAL)
    assert np.array_equal(got[O.ROUTE_REF], si)
    assert np.any(got[O.ROUTE_REF] != got[O.ROUTE_F32])


@pytest.mark.parametrize("path", [oh.OBS_DECODE_FUSED, oh.OBS_DECODE_MULTI], ids=["fused", "multi"])
def test_decode_routing_forced_ties(exe, tie_model, path):
    """obs_moe_decode (one launch, and four launches) on inputs with forced f16
    ties: ids and weights bit-exact with the oracle's reference rule."""
    t, layer, L = tie_model
    T = 64
    x = _inputs(90, T)
    _, ri, rw = O.router(L, x, K, True)
    _, fi, _ = O.router(L, x, K, True, rule=O.ROUTE_F32)
    assert _tie_pairs_seen(ri) > 0
    cfg = oh.MoeConfig(E, K, H, I, 64, True)
    exe.set_decode_path(path)
    try:
        dx = exe.upload(x)
        y = exe.alloc((H,), np.uint16)
        ids = exe.alloc((T, K), np.int32)
        w = exe.alloc((T, K), np.float32)
        for i in range(T):
            exe.moe_decode(cfg, layer, dx.ptr + 2 * H * i, y, ids_out=ids.ptr + 4 * K * i, w_out=w.ptr + 4 * K * i)
        exe.device_status()
        gi, gw = ids.download(), w.download()
    finally:
        exe.set_decode_path(oh.OBS_DECODE_AUTO)
    assert np.array_equal(gi, ri)
    assert np.array_equal(gw.view(np.uint32), rw.view(np.uint32))
    if not np.array_equal(ri, fi):  # where the rules differ, the kernel followed the reference's
        assert not np.array_equal(gi, fi)


def test_prefill_computed_routing_forced_ties(exe, tie_model):
    """obs_moe_prefill with computed routing at T = 512: the routing it leaves
    in the workspace is bit-exact with the oracle's reference rule, and the
    output is within 1e-2 of the fp64 oracle evaluated with that routing."""
    t, layer, L = tie_model
    T = 512
    X = _inputs(91, T)
    cfg = oh.MoeConfig(E, K, H, I, 64, True)
    ws_bytes = exe.moe_prefill_workspace(cfg, T)
    ws = exe.alloc(ws_bytes, np.uint8)
    Y = exe.alloc((T, H), np.uint16)
    exe.moe_prefill(cfg, layer, exe.upload(X), Y, T, ws=ws)
    gi, gw = exe.prefill_routing(cfg, T, ws)
    _, ri, rw = O.router(L, X, K, True)
    assert _tie_pairs_seen(ri) > 0
    assert np.array_equal(gi, ri)
    assert np.array_equal(gw.view(np.uint32), rw.view(np.uint32))
    y = synth.bf16_bits_to_f32(Y.download()).astype(np.float64)
    sel = slice(0, 64)
    ref = O.moe_prefill(L, X[sel], ri[sel], rw[sel], O.MODE_F64)
    rel = float(np.linalg.norm(y[sel] - ref) / np.linalg.norm(ref))
    assert rel < 1e-2, rel


@pytest.mark.parametrize("T", [1, 7, 64, 65, 512, 1100, 3000])
def test_one_launch_router_matches_the_two_calls(exe, T):
    """obs_route (up to 8 tokens one launch whose last workgroup routes, else
    the two launches) against obs_q8_gate_logits + obs_route_topk and the
    oracle: logits, ids and weights bit-exact, under both rules, on a router
    with forced f16 ties; two calls in a row (the launch leaves its counter at
    zero for the next)."""
    t = _tie_layer(78, 1.0)
    w8, s8, b8 = (exe.upload(t[k]) for k in ("router_w", "router_s", "router_b"))
    x = _inputs(92 + T, T)
    dx = exe.upload(x)
    lg2 = exe.alloc((T, E), np.float32)
    exe.q8_gate_logits(w8, s8, b8, dx, lg2, T, H, E)
    ref_lg = lg2.download()
    sel = list(range(0, T, max(1, T // 40)))
    xf = synth.bf16_bits_to_f32(x)
    want_lg = np.stack([O.qmatvec("lanes", 8, t["router_w"], t["router_s"], t["router_b"], xf[i], H, E) for i in sel])
    assert np.array_equal(ref_lg[sel].view(np.uint32), want_lg.view(np.uint32))
    for rule in (O.ROUTE_REF, O.ROUTE_F32):
        ids2, w2 = exe.alloc((T, K), np.int32), exe.alloc((T, K), np.float32)
        exe.route_topk(lg2, ids2, w2, T, E, K, True, rule=rule)
        ri, rw = O.route_topk(ref_lg, K, True, O.SUM_WAVE, rule=rule)
        assert np.array_equal(ids2.download(), ri)
        for rep in range(2):
            lg1 = exe.alloc((T, E), np.float32)
            ids1, w1 = exe.alloc((T, K), np.int32), exe.alloc((T, K), np.float32)
            exe.route(w8, s8, b8, dx, lg1, ids1, w1, T, H, E, K, True, rule=rule)
            exe.device_status()
            assert np.array_equal(lg1.download().view(np.uint32), ref_lg.view(np.uint32)), (rule, rep)
            assert np.array_equal(ids1.download(), ri), (rule, rep)
            assert np.array_equal(w1.download().view(np.uint32), rw.view(np.uint32)), (rule, rep)


def test_one_launch_router_rejects_bad_arguments(exe):
    x = exe.alloc(64, np.uint16)
    with pytest.raises(oh.ObsError, match="k must be"):
        exe.route(x, x, x, x, x, x, x, 1, H, E, 0, True)
    with pytest.raises(oh.ObsError, match="OBS_E_SHAPE"):
        exe.route(x, x, x, x, x, x, x, 1, 1000, E, K, True)
