"""GPU parity beyond the Qwen3-30B-A3B layer: other expert counts and model
widths the boundary accepts (forward.rs:421-441 decode, :164-247 prefill).

* 256 experts takes the fused decode's four-slot routing variant; 64 experts
  leaves half of its two-slot key lanes absent.
* hidden 4096 / inter 2048 is the widest decode shape (4-launch path).
* prefill at 64 and 256 experts and at hidden 1024 / inter 512.

Bars as elsewhere: routing ids and weights bit-exact with the oracle, layer
outputs within 1e-2 relative of the fp64 oracle on the GPU's routing (per
element with a 1e-2 * rms floor), and within 5e-3 of the oracle evaluated with
the prefill GEMM's own bf16 operand roundings.
"""
import numpy as np
import pytest

import oracle as O
import obsidian_hip as oh
from obsidian_hip import synth

pytestmark = pytest.mark.gpu


def _f32(b):
    return synth.bf16_bits_to_f32(b).astype(np.float64)


def _close(y, ref, tol, elem_tol=None):
    """2-norm relative error <= tol; every element within elem_tol (default
    tol) relative with an absolute floor of elem_tol * rms(ref)."""
    rel = float(np.linalg.norm(y - ref) / np.linalg.norm(ref))
    assert rel <= tol, rel
    et = tol if elem_tol is None else elem_tol
    floor = et * np.sqrt(np.mean(ref ** 2))
    assert np.all(np.abs(y - ref) <= et * np.abs(ref) + floor)
    return rel


# Against the oracle evaluated with the GEMM's own bf16 roundings the 2-norm bar
# is 5e-3, but a single element may sit one bf16 step away: the expert outputs
# are rounded to bf16 before the combine, and a different fp32 summation order
# can round one of them to the neighbouring bf16 value (2^-8 relative).
BF_NORM, BF_ELEM = 5e-3, 1e-2


def _decode(exe, cfg, layer, x, path):
    exe.set_decode_path(path)
    try:
        y = exe.alloc(cfg.hidden, np.uint16)
        ids = exe.alloc(cfg.top_k, np.int32)
        w = exe.alloc(cfg.top_k, np.float32)
        exe.moe_decode(cfg, layer, exe.upload(x), y, ids_out=ids, w_out=w)
        exe.device_status()
        return y.download(), ids.download(), w.download()
    finally:
        exe.set_decode_path(oh.OBS_DECODE_AUTO)


@pytest.mark.parametrize("E,seed", [(256, 31), (64, 32)])
def test_decode_expert_counts_fused_and_multi(exe, E, seed):
    H, I, K = 2048, 768, 8
    t = synth.moe_layer(seed, E, H, I, 64)
    layer = oh.MoeLayer.upload(exe, t)
    L = O.Layer(t, E, H, I, 64)
    cfg = oh.MoeConfig(E, K, H, I, 64, True)
    for s in range(2):
        x = synth.bf16_normal(np.random.default_rng(seed * 10 + s), H)
        _, ri, rw = O.router(L, x, K, True)
        outs = {}
        for name, path in (("fused", oh.OBS_DECODE_FUSED), ("multi", oh.OBS_DECODE_MULTI)):
            y, gi, gw = _decode(exe, cfg, layer, x, path)
            assert np.array_equal(gi, ri[0]), (name, gi, ri[0])
            assert np.array_equal(gw.view(np.uint32), rw[0].view(np.uint32)), name
            outs[name] = _f32(y)
        y64, _, _ = O.moe_decode(L, x, K, True, ids=ri, w=rw)
        for name, y in outs.items():
            rel = _close(y, y64[0], 1e-2)
            print(f"E={E} seed {s} {name}: rel {rel:.2e}")


def test_decode_widest_shape(exe):
    E, H, I, K = 16, 4096, 2048, 6
    t = synth.moe_layer(33, E, H, I, 64)
    layer = oh.MoeLayer.upload(exe, t)
    L = O.Layer(t, E, H, I, 64)
    cfg = oh.MoeConfig(E, K, H, I, 64, True)
    x = synth.bf16_normal(np.random.default_rng(330), H)
    y, gi, gw = _decode(exe, cfg, layer, x, oh.OBS_DECODE_AUTO)
    _, ri, rw = O.router(L, x, K, True)
    assert np.array_equal(gi, ri[0]) and np.array_equal(gw.view(np.uint32), rw[0].view(np.uint32))
    y64, _, _ = O.moe_decode(L, x, K, True, ids=ri, w=rw)
    _close(_f32(y), y64[0], 1e-2)


@pytest.mark.parametrize("E,H,I,K,T", [(256, 2048, 768, 8, 96), (64, 2048, 768, 8, 130), (32, 1024, 512, 4, 77)])
def test_prefill_shapes(exe, E, H, I, K, T):
    t = synth.moe_layer(40 + E + H, E, H, I, 64)
    layer = oh.MoeLayer.upload(exe, t)
    L = O.Layer(t, E, H, I, 64)
    cfg = oh.MoeConfig(E, K, H, I, 64, True)
    rng = np.random.default_rng(400 + T)
    X = synth.bf16_normal(rng, (T, H))
    res = synth.bf16_normal(rng, (T, H))
    ws_bytes = exe.moe_prefill_workspace(cfg, T)
    ws = exe.alloc(ws_bytes, np.uint8)
    Y = exe.alloc((T, H), np.uint16)
    exe.moe_prefill(cfg, layer, exe.upload(X), Y, T, residual=exe.upload(res), ws=ws, ws_bytes=ws_bytes)
    y = _f32(Y.download())
    _, ids, w = O.router(L, X, K, True)
    ref_bf = O.moe_prefill(L, X, ids, w, O.MODE_MFMA_BF16) + _f32(res)
    ref64 = O.moe_prefill(L, X, ids, w, O.MODE_F64) + _f32(res)
    _close(y, ref_bf, BF_NORM, BF_ELEM)
    _close(y, ref64, 1e-2)
