"""The dispatch facts the one-launch kernels build on, probed at obs_create,
and the paths they gate; the one-launch prefill FFN's bounded-wait report.

No reference counterpart: the reference's executor setup (executor.rs:39-58)
probes nothing, and its Metal dispatches never observe GPU errors. The
outputs of the separate-launch paths are compared with the one-launch
paths' on the same inputs (the items' arithmetic is the same, so the prefill
results are bit-identical; the 4-launch decode is checked against its forced
selection bit for bit and the oracle elsewhere).
"""
import numpy as np
import pytest

import obsidian_hip as oh
from obsidian_hip import synth

pytestmark = pytest.mark.gpu

E, H, I, K = 128, 2048, 768, 8


@pytest.fixture(scope="module")
def table():
    return synth.moe_layer(41, E, H, I, 64)


def _kernels(exe, fn):
    exe.profile_clear()
    exe.profile_enable(True)
    fn()
    exe.profile_enable(False)
    exe.profile_accumulate()
    st = exe.profile_stats()
    exe.profile_clear()
    return st


def test_probe_finds_the_mi355x_dispatch(exe):
    n, xcd_map, in_order = exe.dispatch_info()
    print(f"CUs {n}, each group b % 8 on one XCD: {xcd_map}, in-order dispatch per XCD: {in_order}")
    assert n >= 256 and xcd_map and in_order
    assert exe.paths() == oh.OBS_PATH_FUSED_DECODE | oh.OBS_PATH_FUSED_ATTN | oh.OBS_PATH_FFN_ONE_LAUNCH


def test_decode_without_the_xcd_map_takes_four_launches(table):
    rng = np.random.default_rng(3)
    x = synth.bf16_normal(rng, H)
    cfg = oh.MoeConfig(E, K, H, I, 64, True)
    with oh.ObsidianExecutor(0) as exe:
        layer = oh.MoeLayer.upload(exe, table)
        dx, y = exe.upload(x), exe.alloc(H, np.uint16)
        st = _kernels(exe, lambda: exe.moe_decode(cfg, layer, dx, y))
        assert "decode_fused" in st
        exe.set_decode_path(oh.OBS_DECODE_MULTI)
        exe.moe_decode(cfg, layer, dx, y)
        y_multi = y.download()
        exe.set_decode_path(oh.OBS_DECODE_AUTO)
        exe.set_dispatch_facts(False, True)
        assert exe.paths() == 0
        st = _kernels(exe, lambda: exe.moe_decode(cfg, layer, dx, y))
        assert "decode_fused" not in st and "decode_gateup" in st, sorted(st)
        assert np.array_equal(y.download(), y_multi)
        # asking for the fused path where the facts rule it out is an error, not a silent choice
        exe.set_decode_path(oh.OBS_DECODE_FUSED)
        with pytest.raises(oh.ObsError) as ei:
            exe.moe_decode(cfg, layer, dx, y)
        assert ei.value.code == oh.OBS_E_UNSUPPORTED
        exe.device_status()


def test_prefill_without_in_order_dispatch_takes_two_launches(table):
    rng = np.random.default_rng(4)
    T = 200
    X = synth.bf16_normal(rng, (T, H))
    ids, w = synth.zipf_routing(T, E, K, 1.1, seed=4)
    cfg = oh.MoeConfig(E, K, H, I, 64, True)
    with oh.ObsidianExecutor(0) as exe:
        layer = oh.MoeLayer.upload(exe, table)
        ws_bytes = exe.moe_prefill_workspace(cfg, T)
        ws = exe.alloc(ws_bytes, np.uint8)
        dX, dids, dw = exe.upload(X), exe.upload(ids), exe.upload(w)
        Y = exe.alloc((T, H), np.uint16)

        def run():
            exe.moe_prefill(cfg, layer, dX, Y, T, ids=dids, weights=dw, ws=ws, ws_bytes=ws_bytes)

        st = _kernels(exe, run)
        assert "moe_ffn" in st, sorted(st)
        y_one = Y.download()
        exe.set_dispatch_facts(True, False)
        assert exe.paths() == oh.OBS_PATH_FUSED_DECODE | oh.OBS_PATH_FUSED_ATTN
        st = _kernels(exe, run)
        assert "moe_ffn" not in st and "grouped_gemm_gateup" in st and "grouped_gemm_down" in st, sorted(st)
        assert np.array_equal(Y.download(), y_one)
        exe.device_status()


def test_ffn_wait_timeout_is_reported_once_per_context(table):
    """The one-launch FFN's down items wait, bounded, for their tile's gate/up
    items. The test hook makes them wait for one count more than ever comes,
    with a 200 us limit: every item still runs and the grid drains, the
    context's obs_device_status reports the time-out once (another context's
    does not), and the defaults restore correct results."""
    rng = np.random.default_rng(5)
    T = 64
    X = synth.bf16_normal(rng, (T, H))
    ids, w = synth.zipf_routing(T, E, K, 1.1, seed=5)
    cfg = oh.MoeConfig(E, K, H, I, 64, True)
    with oh.ObsidianExecutor(0) as exe, oh.ObsidianExecutor(0) as other:
        layer = oh.MoeLayer.upload(exe, table)
        ws_bytes = exe.moe_prefill_workspace(cfg, T)
        ws = exe.alloc(ws_bytes, np.uint8)
        dX, dids, dw = exe.upload(X), exe.upload(ids), exe.upload(w)
        Y = exe.alloc((T, H), np.uint16)

        def run():
            exe.moe_prefill(cfg, layer, dX, Y, T, ids=dids, weights=dw, ws=ws, ws_bytes=ws_bytes)

        run()
        exe.device_status()
        y_ok = Y.download()
        exe.debug_ffn_wait(1, 200)
        st = _kernels(exe, run)
        assert "moe_ffn" in st
        other.device_status()  # the flag is the calling context's
        with pytest.raises(oh.ObsError) as ei:
            exe.device_status()
        assert ei.value.code == oh.OBS_E_HIP and "timed out" in str(ei.value)
        exe.device_status()  # reported once, then cleared
        with pytest.raises(oh.ObsError):
            exe.debug_ffn_wait(0, 0)
        exe.debug_ffn_wait(0, 100000)
        run()
        exe.device_status()
        assert np.array_equal(Y.download(), y_ok)
