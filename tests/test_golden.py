"""Known-answer vectors (tests/golden/kats.json, written from closed forms by
tests/golden/make_kats.py) checked against the oracle on the CPU and against
the HIP kernels through the C ABI on the GPU.

Bars: dequant and one-hot mat-vec bit-exact (integer/format work with a single
fp32 rounding); routing ids bit-exact, routing weights within 2e-6 of the
float64 closed form; SwiGLU within 1 bf16 ulp of the float64 value rounded to
bf16 (bf16 in and out).
"""
import json
import math
import os

import numpy as np
import pytest

import oracle as O
from obsidian_hip import synth

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "kats.json")))


def _row_tensors(case):
    """One 64-column row whose first word is the case's word (one quant group)."""
    per = 32 // case["bits"]
    w = np.zeros((1, 64 // per), np.uint32)
    w[0, 0] = case["word"]
    s = np.array([[case["scale_bf16"]]], np.uint16)
    b = np.array([[case["bias_bf16"]]], np.uint16)
    return w, s, b, per


def _onehot_tensors():
    m = KATS["matvec_onehot"]
    w = np.array(m["words"], np.uint32).reshape(m["out"], m["in"] // 8)
    s = np.array(m["scales_bf16"], np.uint16).reshape(m["out"], m["in"] // 64)
    b = np.array(m["biases_bf16"], np.uint16).reshape(m["out"], m["in"] // 64)
    return m, w, s, b


def _logits(case):
    return np.array([np.nan if v is None else v for v in case["logits"]], np.float32)


def _bf16_bits_of(v: float) -> int:
    return int(synth.f32_to_bf16_bits(np.array([v], np.float32))[0])


# ---------------------------------------------------------------- oracle (CPU)

@pytest.mark.parametrize("i", range(len(KATS["dequant"])))
def test_oracle_dequant_kat(i):
    c = KATS["dequant"][i]
    w, s, b, per = _row_tensors(c)
    got = O.dequant(c["bits"], w, s, b, 1, 64, 64)[0, :per]
    assert [int(v) for v in got.view(np.uint32)] == c["f32_bits"]


def test_oracle_matvec_onehot_kat():
    m, w, s, b = _onehot_tensors()
    for j in m["onehot_cols"]:
        x = np.zeros(m["in"], np.float32)
        x[j] = 1.0
        for kind in ("shader", "lanes"):
            y = O.qmatvec(kind, 4, w, s, b, x, m["in"], m["out"], 64)
            assert [int(v) for v in np.asarray(y, np.float32).view(np.uint32)] == m["y_f32_bits"][str(j)], (kind, j)


_RULES = {"ref": O.ROUTE_REF, "f32": O.ROUTE_F32}


def _route_weights_ok(got, c) -> bool:
    """fp32 rule: within 2e-6 of the float64 closed form. Reference rule: the
    weights are f16 values, within one f16 step of the closed form (its fp32 p
    and the oracle's can differ by an ulp before the f16 rounding)."""
    want = np.asarray(c["weights"], np.float64)
    got = np.asarray(got, np.float64)
    if c["rule"] == "f32":
        return bool(np.allclose(got, want, rtol=0, atol=2e-6))
    is_f16 = np.array_equal(got.astype(np.float16).astype(np.float64), got)
    step = np.where(want > 0, 2.0 ** (np.floor(np.log2(np.maximum(want, 2.0 ** -24))) - 10), 2.0 ** -24)
    return is_f16 and bool(np.all(np.abs(got - want) <= step))


@pytest.mark.parametrize("i", range(len(KATS["route_topk"])))
def test_oracle_route_kat(i):
    c = KATS["route_topk"][i]
    ids, w = O.route_topk(_logits(c)[None, :], c["k"], c["norm_topk"], rule=_RULES[c["rule"]])
    assert list(ids[0]) == c["ids"], c["name"]
    assert _route_weights_ok(w[0], c), (c["name"], w[0], c["weights"])


def test_oracle_silu_kat():
    for c in KATS["swiglu"]:
        assert math.isclose(O.silu_mul(c["g"], c["u"]), c["h"], rel_tol=1e-6, abs_tol=1e-30)


# ---------------------------------------------------------------- kernels (GPU)

@pytest.mark.gpu
def test_gpu_dequant_kat(exe):
    for c in KATS["dequant"]:
        w, s, b, per = _row_tensors(c)
        o32 = exe.alloc((1, 64), np.float32)
        o16 = exe.alloc((1, 64), np.uint16)
        exe.dequant_tensor(c["bits"], exe.upload(w), exe.upload(s), exe.upload(b), 1, 64, 64,
                           out_f32=o32, out_bf16=o16)
        assert [int(v) for v in o32.download()[0, :per].view(np.uint32)] == c["f32_bits"]
        assert [int(v) for v in o16.download()[0, :per]] == c["bf16_bits"]


@pytest.mark.gpu
def test_gpu_matvec_onehot_kat(exe):
    m, w, s, b = _onehot_tensors()
    dw, ds, db = exe.upload(w), exe.upload(s), exe.upload(b)
    for j in m["onehot_cols"]:
        x = np.zeros(m["in"], np.uint16)
        x[j] = 0x3F80  # bf16 1.0
        y = exe.alloc((m["out"],), np.float32)
        exe.q4_matvec(dw, ds, db, exe.upload(x), m["in"], m["out"], 64, y_f32=y)
        assert [int(v) for v in y.download().view(np.uint32)] == m["y_f32_bits"][str(j)], j


@pytest.mark.gpu
def test_gpu_route_kat(exe):
    for c in KATS["route_topk"]:
        lg = _logits(c)[None, :]
        n, k = lg.shape[1], c["k"]
        ids = exe.alloc((1, k), np.int32)
        w = exe.alloc((1, k), np.float32)
        exe.route_topk(exe.upload(lg), ids, w, 1, n, k, c["norm_topk"], rule=_RULES[c["rule"]])
        assert list(ids.download()[0]) == c["ids"], c["name"]
        assert _route_weights_ok(w.download()[0], c), c["name"]


@pytest.mark.gpu
def test_gpu_swiglu_kat(exe):
    g = np.array([_bf16_bits_of(c["g"]) for c in KATS["swiglu"]], np.uint16)
    u = np.array([_bf16_bits_of(c["u"]) for c in KATS["swiglu"]], np.uint16)
    h = exe.alloc(g.shape, np.uint16)
    exe.swiglu_raw(exe.upload(g), exe.upload(u), h, len(g))
    got = h.download().astype(np.int64)
    want = np.array([_bf16_bits_of(c["h"]) for c in KATS["swiglu"]], np.int64)
    # same sign, at most one bf16 ulp apart (float64 truth rounded once vs fp32 math rounded once)
    assert np.all((got >> 15) == (want >> 15)) and np.all(np.abs(got - want) <= 1), (got, want)
