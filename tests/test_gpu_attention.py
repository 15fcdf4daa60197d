"""GPU parity of the decode step around the MoE block (forward.rs:398-419,
:445-462, :552-567): the fused 4-bit mat-vec (q/k/v/o projections, lm_head),
q/k RMSNorm + NeoX RoPE + cache append, GQA decode attention, the embedding
row and the greedy argmax, each against the oracle.

Bars: embedding and argmax bit-exact; the norm + RoPE output within one bf16
step of the oracle (cos and sin come from double-precision library calls on
both sides); mat-vec within the bound of f16 activations and fp32 sums;
attention within 1e-2 of the fp64 oracle (the softmax weights enter the
value product as bf16)."""
import numpy as np
import pytest

import oracle as O
import obsidian_hip as oh
from obsidian_hip import synth

pytestmark = pytest.mark.gpu

NH, NKV, HD = 32, 4, 128
EPS, THETA = 1e-6, 1e7


def _f(b):
    return synth.bf16_bits_to_f32(b).astype(np.float64)


def _state(exe, pos, tok=0):
    return exe.upload(np.array([pos, tok], np.int32))


@pytest.mark.parametrize("in_f", [2048, 4096])
def test_q4_gemv_parts_vs_oracle(exe, in_f):
    rng = np.random.default_rng(500 + in_f)
    rows = (640, 128, 64)
    mats = [synth.quant_tensor(rng, r, in_f, 4, 64) for r in rows]
    x = synth.bf16_normal(rng, in_f)
    res = synth.bf16_normal(rng, rows[2], 4.0)
    y0 = exe.alloc(rows[0], np.float32)
    y1 = exe.alloc(rows[1], np.uint16)
    y2 = exe.alloc(rows[2], np.uint16)
    d = [tuple(exe.upload(a) for a in m) for m in mats]
    exe.q4_gemv(exe.upload(x), in_f, [(*d[0], rows[0], y0, None, None), (*d[1], rows[1], None, y1, None),
                                      (*d[2], rows[2], None, y2, exe.upload(res))])
    xf = synth.bf16_bits_to_f32(x)
    outs = [y0.download().astype(np.float64), _f(y1.download()), _f(y2.download())]
    for i, (m, got) in enumerate(zip(mats, outs)):
        y64, ab = O.qmatvec("f64", 4, *m, xf, in_f, rows[i])
        if i == 2:
            y64 = y64 + _f(res)
            ab = ab + np.abs(_f(res))
        # f16 activations (2^-11 relative each) and fp32 sums; bf16 outputs add 2^-9 of |y|
        bound = 1e-3 * ab + (2.0 ** -8 * np.abs(y64) if i else 0.0)
        assert np.all(np.abs(got - y64) <= bound), (i, float(np.max(np.abs(got - y64) / (ab + 1e-30))))


@pytest.mark.parametrize("in_f", [2048, 4096])
def test_q4_gemv_fused_rmsnorm(exe, in_f):
    """norm_w: x is replaced by bf16(rmsnorm(x) * w) first (the input / final
    norms fused); against the oracle norm then the oracle mat-vec."""
    rng = np.random.default_rng(520 + in_f)
    rows = 384
    w, s, b = synth.quant_tensor(rng, rows, in_f, 4, 64)
    x = synth.bf16_normal(rng, in_f, 3.0)
    nw = synth.norm_weight(rng, in_f)
    y = exe.alloc(rows, np.float32)
    exe.q4_gemv(exe.upload(x), in_f, [(exe.upload(w), exe.upload(s), exe.upload(b), rows, y, None, None)],
                norm_w=exe.upload(nw), eps=EPS)
    xn = O.rmsnorm(x, nw, EPS)
    y64, ab = O.qmatvec("f64", 4, w, s, b, synth.bf16_bits_to_f32(xn), in_f, rows)
    got = y.download().astype(np.float64)
    # in = 2048: the norm is obs_rmsnorm's sequence exactly; 4096 sums in another order (one bf16 step)
    bound = (1e-3 if in_f == 2048 else 5e-3) * ab
    assert np.all(np.abs(got - y64) <= bound), float(np.max(np.abs(got - y64) / ab))


@pytest.mark.parametrize("in_f,rows", [(2048, 16421), (4096, 16389)])
def test_q4_gemv_large_matrix(exe, in_f, rows):
    """Above 16,384 rows each wave takes 16 (in 2048) or 8 (in 4096) rows; a
    row count that leaves the last wave partly empty, one bf16 part with a
    residual next to an fp32 part, and the fused norm."""
    rng = np.random.default_rng(540 + in_f)
    r1 = 7
    w, s, b = synth.quant_tensor(rng, rows - r1, in_f, 4, 64)
    w1, s1, b1 = synth.quant_tensor(rng, r1, in_f, 4, 64)
    x = synth.bf16_normal(rng, in_f, 2.0)
    nw = synth.norm_weight(rng, in_f)
    res = synth.bf16_normal(rng, r1, 4.0)
    y = exe.alloc(rows - r1, np.float32)
    y1 = exe.alloc(r1, np.uint16)
    exe.q4_gemv(exe.upload(x), in_f, [(exe.upload(w), exe.upload(s), exe.upload(b), rows - r1, y, None, None),
                                      (exe.upload(w1), exe.upload(s1), exe.upload(b1), r1, None, y1, exe.upload(res))],
                norm_w=exe.upload(nw), eps=EPS)
    xn = synth.bf16_bits_to_f32(O.rmsnorm(x, nw, EPS))
    tol = 1e-3 if in_f == 2048 else 5e-3
    y64, ab = O.qmatvec("f64", 4, w, s, b, xn, in_f, rows - r1)
    got = y.download().astype(np.float64)
    assert np.all(np.abs(got - y64) <= tol * ab), float(np.max(np.abs(got - y64) / ab))
    y64, ab = O.qmatvec("f64", 4, w1, s1, b1, xn, in_f, r1)
    y64, ab = y64 + _f(res), ab + np.abs(_f(res))
    got = _f(y1.download())
    assert np.all(np.abs(got - y64) <= tol * ab + 2.0 ** -8 * np.abs(y64))


def test_q4_gemv_rejects_bad_shapes(exe):
    x = exe.alloc(3072, np.uint16)
    y = exe.alloc(4, np.float32)
    w = exe.alloc((4, 384), np.uint32)
    s = exe.alloc((4, 48), np.uint16)
    with pytest.raises(oh.ObsError, match="OBS_E_SHAPE"):
        exe.q4_gemv(x, 3072, [(w, s, s, 4, y, None, None)])
    with pytest.raises(oh.ObsError, match="residual needs"):
        exe.q4_gemv(x, 2048, [(w, s, s, 4, y, None, x)])


@pytest.mark.parametrize("pos", [0, 1, 517, 4095])
def test_attn_prep_vs_oracle(exe, pos):
    rng = np.random.default_rng(600 + pos)
    ml = 4096
    q = synth.bf16_normal(rng, (NH, HD), 2.0)
    k = synth.bf16_normal(rng, (NKV, HD), 2.0)
    v = synth.bf16_normal(rng, (NKV, HD))
    qn_w = synth.bf16_normal(rng, HD, 0.5)
    kn_w = synth.bf16_normal(rng, HD, 0.5)
    kc0 = synth.bf16_normal(rng, (NKV, ml, HD))
    vc0 = synth.bf16_normal(rng, (NKV, HD, ml))
    dq, dk, dv = exe.upload(q), exe.upload(k), exe.upload(v)
    kc, vc = exe.upload(kc0), exe.upload(vc0)
    exe.attn_prep(dq, dk, dv, exe.upload(qn_w), exe.upload(kn_w), kc, vc, NH, NKV, HD, ml, EPS, THETA,
                  _state(exe, pos))
    want_q = O.rope_neox(O.rmsnorm(q, qn_w, EPS), pos, THETA)
    want_k = O.rope_neox(O.rmsnorm(k, kn_w, EPS), pos, THETA)
    got_q, got_kc, got_vc = dq.download(), kc.download(), vc.download()
    # within one bf16 step (ordinarily identical)
    assert np.max(np.abs(got_q.astype(np.int32) - want_q.astype(np.int32))) <= 1
    assert np.max(np.abs(got_kc[:, pos].astype(np.int32) - want_k.astype(np.int32))) <= 1
    assert np.array_equal(got_vc[:, :, pos], v)
    # nothing else in the caches moved
    others = np.ones(ml, bool)
    others[pos] = False
    assert np.array_equal(got_kc[:, others], kc0[:, others])
    assert np.array_equal(got_vc[:, :, others], vc0[:, :, others])
    print(f"pos {pos}: q exact {np.array_equal(got_q, want_q)}, k exact {np.array_equal(got_kc[:, pos], want_k)}")


def test_attn_prep_out_of_range_position_appends_nothing(exe):
    rng = np.random.default_rng(610)
    ml = 64
    kc0 = synth.bf16_normal(rng, (NKV, ml, HD))
    vc0 = synth.bf16_normal(rng, (NKV, HD, ml))
    kc, vc = exe.upload(kc0), exe.upload(vc0)
    x = exe.upload(synth.bf16_normal(rng, (NH, HD)))
    w = exe.upload(synth.bf16_normal(rng, HD))
    exe.attn_prep(x, x, x, w, w, kc, vc, NH, NKV, HD, ml, EPS, THETA, _state(exe, ml))
    assert np.array_equal(kc.download(), kc0) and np.array_equal(vc.download(), vc0)


def _sdpa_case(rng, seq, ml, qscale):
    q = synth.bf16_normal(rng, (NH, HD), qscale)
    kc = synth.bf16_normal(rng, (NKV, ml, HD))
    vc = synth.bf16_normal(rng, (NKV, ml, HD))
    return q, kc, vc


@pytest.mark.parametrize("seq,qscale", [(1, 1.0), (31, 1.0), (32, 1.0), (33, 3.0), (100, 1.0), (1000, 3.0),
                                        (4095, 1.0), (4096, 3.0)])
def test_sdpa_decode_vs_oracle(exe, seq, qscale):
    rng = np.random.default_rng(700 + seq)
    ml = 4096
    q, kc, vc = _sdpa_case(rng, seq, ml, qscale)
    ws = exe.alloc(exe.sdpa_workspace(NH, NKV, HD, ml), np.uint8)
    out = exe.alloc((NH, HD), np.uint16)
    exe.sdpa_decode(exe.upload(q), exe.upload(kc), exe.upload(np.ascontiguousarray(vc.transpose(0, 2, 1))), out,
                    NH, NKV, HD, ml, _state(exe, seq - 1), ws)
    want = O.sdpa_decode(q, kc, vc, seq, HD ** -0.5)
    got = _f(out.download())
    err = np.abs(got - want)
    scale = np.abs(want).max(axis=1, keepdims=True)
    assert np.all(err <= 1e-2 * scale), float((err / scale).max())
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel < 5e-3, rel
    print(f"seq {seq}: rel err {rel:.2e}")


def test_sdpa_single_position_is_v(exe):
    """seq = 1: softmax of one score is 1, so every head returns its kv head's
    first value row exactly (P = 1 is exact in bf16)."""
    rng = np.random.default_rng(790)
    ml = 64
    q, kc, vc = _sdpa_case(rng, 1, ml, 1.0)
    vc[:, 1:, :] = 0x7FC0  # NaN beyond the attended position: must not leak
    ws = exe.alloc(exe.sdpa_workspace(NH, NKV, HD, ml), np.uint8)
    out = exe.alloc((NH, HD), np.uint16)
    exe.sdpa_decode(exe.upload(q), exe.upload(kc), exe.upload(np.ascontiguousarray(vc.transpose(0, 2, 1))), out,
                    NH, NKV, HD, ml, _state(exe, 0), ws)
    got = out.download()
    for h in range(NH):
        assert np.array_equal(got[h], vc[h // (NH // NKV), 0])


def test_embed_q4_bit_exact(exe):
    rng = np.random.default_rng(800)
    vocab, hidden = 1000, 2048
    w, s, b = synth.quant_tensor(rng, vocab, hidden, 4, 64)
    dw, ds, db = exe.upload(w), exe.upload(s), exe.upload(b)
    out = exe.alloc(hidden, np.uint16)
    for tok in (0, 1, 517, vocab - 1):
        exe.embed_q4(dw, ds, db, hidden, vocab, _state(exe, 0, tok), out)
        want = synth.f32_to_bf16_bits(O.dequant(4, w[tok:tok + 1], s[tok:tok + 1], b[tok:tok + 1], 1, hidden)[0])
        assert np.array_equal(out.download(), want), tok


@pytest.mark.parametrize("case", ["random", "ties", "nan", "all_neg_inf", "last"])
def test_argmax_vs_oracle_and_state(exe, case):
    rng = np.random.default_rng(900)
    n = 151936
    x = rng.standard_normal(n).astype(np.float32)
    if case == "ties":
        x[[5, 70000, 151935]] = 100.0
    elif case == "nan":
        x[rng.integers(0, n, 1000)] = np.nan
        x[3] = np.nan
    elif case == "all_neg_inf":
        x[:] = -np.inf
        x[12345] = np.nan
    elif case == "last":
        x[n - 1] = 50.0
    state = _state(exe, 41, 7)
    ws = exe.alloc(oh.lib().obs_argmax_workspace(), np.uint8)
    exe.argmax(exe.upload(x), n, state, ws)
    pos, tok = state.download()
    assert (pos, tok) == (42, O.argmax(x)), (case, tok, O.argmax(x))
