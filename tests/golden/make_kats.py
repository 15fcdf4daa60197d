#!/usr/bin/env python3
"""Writes tests/golden/kats.json: known-answer vectors for the MoE expert path,
derived from closed forms only (no call into the oracle or the library).

The reference ships no test vectors (its only known answer needs the 17 GB
checkpoint), so every expected value here follows from the mathematics of the
format and of the operators:

* dequant (MLX affine, tools/split_experts.py:9-19, fused_dequant_matvec_4bit.metal:39-42,
  dequant_matvec_8bit.metal:26-27): element c of a row is field c % 8 (4-bit) or
  c % 4 (8-bit) of word c // per_word, low bits first; w = q*s + b. With bf16
  s and b, q*s is exact in fp32, so the fp32 result is the exact sum rounded
  once; float64 holds that sum exactly for the values below, and one
  float64 -> float32 conversion rounds it.
* mat-vec with one-hot x (fused_dequant_matvec_4bit.metal:14-53): y[o] = W[o, j]
  exactly (every other product is an exact zero).
* top-k routing (moe_routing_topk.metal:24-56), in IEEE fp32 semantics: under
  the reference rule ("ref") each logit is first rounded to f16, the half that
  dequant_matvec_8bit.metal:30 stores (numpy's float16 conversion is round to
  nearest even); e_i = fl32(exp(l_i - m)) with gradual underflow (numpy's
  float64 -> float32 conversion of the float64 exp), p_i = fl32(e_i / S); the
  ids are the k largest p, ties (including p that underflowed to 0) to the
  lower id. Weights: "f32" rule p_i, renormalised exp(l_i - m) / sum over the
  chosen exp(l_j - m) (the full-softmax denominator cancels, float64); "ref"
  rule f16(p_i), renormalised f16(f16(p_i) / wsum) with wsum the fp32 sum of
  the chosen p (moe_routing_topk.metal:47, :55). A -inf logit has p = 0 and is
  still chosen, after every positive p (strict > against a -inf start,
  :44-46). A NaN logit makes the softmax sum NaN (:33-39: max skips it, exp
  does not), so every p is NaN, no comparison succeeds and no id is chosen:
  ids -1 (weights 0 here; the shader writes -inf halves and indexes out of
  range, :48-51).
* SwiGLU (ops.metal:18-22): g / (1 + exp(-g)) * u in float64.

Run:  python3 tests/golden/make_kats.py   (rewrites kats.json deterministically)
"""
import json
import math
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def f32_bits(v: float) -> int:
    return struct.unpack("<I", struct.pack("<f", v))[0]


def bf16_bits_exact(v: float) -> int:
    """bf16 pattern of a value that bf16 represents exactly (asserted)."""
    b = f32_bits(v)
    assert b & 0xFFFF == 0, v
    return b >> 16


def bf16_value(bits: int) -> float:
    return struct.unpack("<f", struct.pack("<I", bits << 16))[0]


def rne_f32_to_bf16(fbits: int) -> int:
    """Round-to-nearest-even of an fp32 pattern to bf16 (finite inputs)."""
    lsb = (fbits >> 16) & 1
    return ((fbits + 0x7FFF + lsb) >> 16) & 0xFFFF


def dequant_cases():
    rng = np.random.default_rng(20261201)
    cases = []
    fixed = [
        (0x76543210, 1.0, 0.0),            # q = 0..7 in column order
        (0xFEDCBA98, 1.0, 0.0),            # q = 8..15
        (0x00000000, 0.5, -0.25),          # every element is the bias
        (0xFFFFFFFF, 0.0078125, 0.125),    # 15 s + b
        (0x0F0F0F0F, -3.0, 2.0),           # alternating 15 and 0
        (0x12345678, 0.01171875, -0.0625),
    ]
    for _ in range(6):
        s = bf16_value(int(rng.integers(0x3A00, 0x3D80)))      # |s| in about [5e-4, 6e-2]
        b = bf16_value(int(rng.integers(0x3A00, 0x3D00)) | (0x8000 if rng.integers(2) else 0))
        fixed.append((int(rng.integers(0, 2**32)), s, b))
    for word, s, b in fixed:
        sb, bb = bf16_bits_exact(s), bf16_bits_exact(b)
        q = [(word >> (4 * j)) & 0xF for j in range(8)]
        vals = [np.float32(qq * bf16_value(sb) + bf16_value(bb)) for qq in q]  # float64 exact, one rounding
        cases.append({"bits": 4, "word": word, "scale_bf16": sb, "bias_bf16": bb, "q": q,
                      "f32_bits": [f32_bits(float(v)) for v in vals],
                      "bf16_bits": [rne_f32_to_bf16(f32_bits(float(v))) for v in vals]})
    for word, s, b in [(0x03020100, 1.0, 0.0), (0xFF80017F, 0.00390625, -0.5), (0xDEADBEEF, -0.0625, 1.5)]:
        sb, bb = bf16_bits_exact(s), bf16_bits_exact(b)
        q = [(word >> (8 * j)) & 0xFF for j in range(4)]
        vals = [np.float32(qq * bf16_value(sb) + bf16_value(bb)) for qq in q]
        cases.append({"bits": 8, "word": word, "scale_bf16": sb, "bias_bf16": bb, "q": q,
                      "f32_bits": [f32_bits(float(v)) for v in vals],
                      "bf16_bits": [rne_f32_to_bf16(f32_bits(float(v))) for v in vals]})
    return cases


def onehot_matvec_case():
    """A [4 x 128] q4 matrix (2 groups per row); x = e_j for a few j; y = W[:, j]."""
    rng = np.random.default_rng(7)
    out_f, in_f = 4, 128
    words = rng.integers(0, 2**32, size=(out_f, in_f // 8), dtype=np.uint64).astype(np.uint32)
    sc = rng.integers(0x3B00, 0x3D00, size=(out_f, in_f // 64)).astype(np.uint16)
    bi = (rng.integers(0x3A00, 0x3C80, size=(out_f, in_f // 64)) | 0x8000).astype(np.uint16)
    cols = [0, 7, 8, 63, 64, 127]
    expect = {}
    for j in cols:
        col = []
        for o in range(out_f):
            q = (int(words[o, j // 8]) >> (4 * (j % 8))) & 0xF
            v = np.float32(q * bf16_value(int(sc[o, j // 64])) + bf16_value(int(bi[o, j // 64])))
            col.append(f32_bits(float(v)))
        expect[str(j)] = col
    return {"out": out_f, "in": in_f, "group": 64, "words": [int(w) for w in words.ravel()],
            "scales_bf16": [int(v) for v in sc.ravel()], "biases_bf16": [int(v) for v in bi.ravel()],
            "onehot_cols": cols, "y_f32_bits": expect}


def route_cases():
    def f16(v):
        return float(np.float16(v))

    def top(logits, k, norm, rule):
        n = len(logits)
        if any(math.isnan(v) for v in logits):
            return [-1] * k, [0.0] * k
        lg = [f16(v) for v in logits] if rule == "ref" else list(logits)
        m = max(lg)
        ed = [math.exp(v - m) for v in lg]               # float64
        e32 = [float(np.float32(v)) for v in ed]         # one rounding, gradual underflow
        S = float(np.float32(sum(e32)))
        p32 = [float(np.float32(v / S)) for v in e32]
        order = sorted(range(n), key=lambda i: (-p32[i], i))  # larger p first, lower id on ties
        sel = order[:k]
        ids = sel + [-1] * (k - len(sel))
        if rule == "f32":
            if norm:
                tot = sum(ed[i] for i in sel)
                w = [ed[i] / tot for i in sel] if tot > 0 else [p32[i] for i in sel]
            else:
                w = [ed[i] / sum(ed) for i in sel]
        else:
            wsum = 0.0
            for i in sel:
                wsum = float(np.float32(wsum + p32[i]))
            w = [f16(p32[i]) for i in sel]
            if norm and wsum > 0:
                w = [f16(v / wsum) for v in w]
        return ids, w + [0.0] * (k - len(sel))

    cases = []
    base = [0.5, -1.0, 2.0, 2.0, 0.25, 3.0, -7.5, 2.0, 1.0, 0.0, -0.5, 1.5, 2.0, -2.0, 0.75, 3.0]
    cases.append(("ties_lower_id_first", base, 8, True))
    cases.append(("ties_no_renorm", base, 4, False))
    cases.append(("all_equal", [1.25] * 16, 8, True))
    cases.append(("nan_poisons_row", [float("nan"), 1.0, float("-inf"), 0.5, float("nan"), 2.0, -1.0, 0.0,
                                      3.0, float("nan"), -2.0, 1.5, 0.25, -0.25, 4.0, -3.0], 8, True))
    cases.append(("neg_inf_chosen_last", [float("-inf")] * 5 + [1.0, float("-inf"), 0.5, float("-inf"), 2.0]
                  + [float("-inf")] * 6, 8, True))
    rng = np.random.default_rng(3)
    wide = [float(np.float32(v)) for v in rng.standard_normal(128) * 3.0]
    wide[17] = wide[90] = float(np.float32(max(wide) + 1.0))  # an exact tie at the top
    cases.append(("n128_tie_at_top", wide, 8, True))
    cases.append(("top1", wide, 1, True))
    # fp32 logits that one f16 rounding makes equal: 2 + 2^-11 (id 9) rounds to 2.0
    # (id 3), so the lower id goes first under the reference rule and last in fp32
    near = [0.5, -1.0, 0.25, 2.0, 1.0, -0.5, 0.0, 1.5, -2.0, 2.0 + 2.0 ** -11, 0.75, -0.25, 1.25, -1.5, 0.125, 1.75]
    cases.append(("f16_rounding_tie", near, 4, True))
    # one f16 ulp apart at 4.0 (2^-8): still ordered under both rules
    cases.append(("one_f16_ulp_apart", [4.0, 4.0 + 2.0 ** -8, 3.0, 4.0 - 2.0 ** -9] + [0.0] * 12, 4, True))
    # logit gaps below -87.3 give subnormal p (ordered by value), below -104 p = 0 (ties by id)
    cases.append(("subnormal_p", [0.0, -95.0, -90.0, -300.0, -200.0, -100.0] + [-500.0] * 10, 6, False))
    # spread of the 30B-A3B router at the bench's weight scale (logit sd ~100): several p underflow
    wide100 = [float(np.float32(v)) for v in np.random.default_rng(5).standard_normal(128) * 100.0]
    cases.append(("sd100_spread", wide100, 8, True))
    out = []
    for rule in ("f32", "ref"):
        for name, lg, k, norm in cases:
            ids, w = top(lg, k, norm, rule)
            out.append({"name": f"{name}/{rule}", "rule": rule, "logits": [None if math.isnan(v) else v for v in lg],
                        "k": k, "norm_topk": norm, "ids": ids, "weights": w})
    return out


def swiglu_cases():
    gs = [-20.0, -3.5, -1.0, -0.125, 0.0, 0.0625, 0.5, 1.0, 2.75, 8.0, 30.0]
    us = [1.0, -2.0, 0.5, 3.0, 7.0, -1.0, 1.5, -0.25, 2.0, -4.0, 0.75]
    return [{"g": g, "u": u, "h": g / (1.0 + math.exp(-g)) * u} for g, u in zip(gs, us)]


def main():
    kats = {"about": "closed-form known answers; regenerate with tests/golden/make_kats.py",
            "dequant": dequant_cases(), "matvec_onehot": onehot_matvec_case(),
            "route_topk": route_cases(), "swiglu": swiglu_cases()}
    with open(os.path.join(HERE, "kats.json"), "w") as f:
        json.dump(kats, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
