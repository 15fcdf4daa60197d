"""GPU parity: dequant, mat-vec, router, elementwise — HIP kernels through the
C ABI against the CPU oracle on the same seeded inputs.

Bars: dequant bit-exact (fp32 and its bf16 rounding); router logits, ids and
weights bit-exact (documented reduction order); SwiGLU bit-exact; mat-vec
within the fp32 summation bound |y - y64| <= gamma_K * sum|w x| (+ one bf16
rounding for bf16 outputs).
"""
import numpy as np
import pytest

import oracle as O
import obsidian_hip as oh
from obsidian_hip import synth

pytestmark = pytest.mark.gpu
U = 2.0 ** -24


def _f32(b):
    return synth.bf16_bits_to_f32(b)


@pytest.mark.parametrize("bits,rows,cols", [(4, 2048, 768), (4, 768, 2048), (8, 128, 2048), (4, 3, 64)])
def test_dequant_bit_exact(exe, bits, rows, cols):
    rng = np.random.default_rng(100 + bits + rows)
    w, s, b = synth.quant_tensor(rng, rows, cols, bits, 64)
    dw, ds, db = exe.upload(w), exe.upload(s), exe.upload(b)
    of = exe.alloc((rows, cols), np.float32)
    ob = exe.alloc((rows, cols), np.uint16)
    exe.dequant_tensor(bits, dw, ds, db, rows, cols, 64, out_f32=of, out_bf16=ob)
    got, gotb = of.download(), ob.download()
    ref = O.dequant(bits, w, s, b, rows, cols, 64)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(gotb, synth.f32_to_bf16_bits(ref))


def test_dequant_known_answer_word(exe):
    w = np.array([[0x76543210, 0xFEDCBA98] + [0] * 6], np.uint32)
    s = synth.f32_to_bf16_bits(np.array([[0.5]], np.float32))
    b = synth.f32_to_bf16_bits(np.array([[-1.0]], np.float32))
    of = exe.alloc((1, 64), np.float32)
    exe.dequant_tensor(4, exe.upload(w), exe.upload(s), exe.upload(b), 1, 64, 64, out_f32=of)
    assert list(of.download()[0, :16]) == [0.5 * q - 1.0 for q in range(16)]


@pytest.mark.parametrize("in_f,out_f", [(768, 2048), (2048, 768), (512, 5)])
def test_q4_matvec_within_fp32_bound(exe, in_f, out_f):
    """The down_proj shape [2048, 768] and the gate/up shape."""
    rng = np.random.default_rng(200 + in_f)
    w, s, b = synth.quant_tensor(rng, out_f, in_f, 4, 64)
    x = synth.bf16_normal(rng, in_f)
    yf = exe.alloc(out_f, np.float32)
    yb = exe.alloc(out_f, np.uint16)
    exe.q4_matvec(exe.upload(w), exe.upload(s), exe.upload(b), exe.upload(x), in_f, out_f, 64, y_f32=yf, y_bf16=yb)
    y = yf.download().astype(np.float64)
    y64, ab = O.qmatvec("f64", 4, w, s, b, _f32(x), in_f, out_f)
    gamma = in_f * U / (1 - in_f * U)
    assert np.all(np.abs(y - y64) <= 2 * gamma * ab + 1e-30)
    assert np.array_equal(yb.download(), synth.f32_to_bf16_bits(y.astype(np.float32)))
    # and against the reference's serial shader order, same bound
    ys = O.qmatvec("shader", 4, w, s, b, _f32(x), in_f, out_f).astype(np.float64)
    assert np.all(np.abs(y - ys) <= 2 * gamma * ab + 1e-30)


def test_q4_matvec_one_hot(exe):
    rng = np.random.default_rng(201)
    w, s, b = synth.quant_tensor(rng, 64, 2048, 4, 64)
    W = O.dequant(4, w, s, b, 64, 2048)
    dw, ds, db = exe.upload(w), exe.upload(s), exe.upload(b)
    for j in (0, 63, 64, 1000, 2047):
        x = np.zeros(2048, np.uint16)
        x[j] = 0x3F80  # 1.0
        yf = exe.alloc(64, np.float32)
        exe.q4_matvec(dw, ds, db, exe.upload(x), 2048, 64, 64, y_f32=yf)
        assert np.array_equal(yf.download(), W[:, j])


@pytest.mark.parametrize("T", [1, 7, 512, 1100, 2048])
def test_q8_gate_logits_bit_exact(exe, T):
    """The router gate [128, 2048] 8-bit, T = 1 and 512; at 1,100 and
    2,048 tokens a workgroup runs several 8-token chunks (1,100: a partial
    last chunk)."""
    E, H = 128, 2048
    rng = np.random.default_rng(300 + T)
    w, s, b = synth.quant_tensor(rng, E, H, 8, 64)
    x = synth.bf16_normal(rng, (T, H))
    lg = exe.alloc((T, E), np.float32)
    exe.q8_gate_logits(exe.upload(w), exe.upload(s), exe.upload(b), exe.upload(x), lg, T, H, E, 64)
    got = lg.download()
    xf = _f32(x)
    for t in range(T):
        ref = O.qmatvec("lanes", 8, w, s, b, xf[t], H, E, lanes=64)
        assert np.array_equal(got[t].view(np.uint32), ref.view(np.uint32)), f"token {t}"


@pytest.mark.parametrize("H,E,T", [(512, 60, 9), (1024, 128, 17), (4096, 256, 11), (4096, 37, 3)])
def test_q8_gate_logits_other_widths_bit_exact(exe, H, E, T):
    """The router kernel's other row widths (4, 16 or 64 columns per lane) and
    expert counts that leave a workgroup's rows partly past the last expert."""
    rng = np.random.default_rng(310 + H + E)
    w, s, b = synth.quant_tensor(rng, E, H, 8, 64)
    x = synth.bf16_normal(rng, (T, H))
    lg = exe.alloc((T, E), np.float32)
    exe.q8_gate_logits(exe.upload(w), exe.upload(s), exe.upload(b), exe.upload(x), lg, T, H, E, 64)
    got = lg.download()
    xf = _f32(x)
    for t in range(T):
        ref = O.qmatvec("lanes", 8, w, s, b, xf[t], H, E, lanes=64)
        assert np.array_equal(got[t].view(np.uint32), ref.view(np.uint32)), f"token {t}"


@pytest.mark.parametrize("rule", [O.ROUTE_REF, O.ROUTE_F32], ids=["ref", "f32"])
@pytest.mark.parametrize("n_exp,k,norm", [(128, 8, True), (128, 8, False), (64, 4, True), (256, 8, True),
                                          (100, 7, True), (16, 16, True), (128, 1, True)])
def test_route_topk_bit_exact(exe, n_exp, k, norm, rule):
    rng = np.random.default_rng(400 + n_exp + k)
    T = 512
    lg = (rng.standard_normal((T, n_exp)) * 3).astype(np.float32)
    # forced ties in a few tokens, including at the top-k boundary
    lg[0, :] = 1.0
    lg[1, [5 % n_exp, 17 % n_exp, 40 % n_exp]] = 9.0
    lg[2, :] = np.round(lg[2, :])
    dl = exe.upload(lg)
    ids = exe.alloc((T, k), np.int32)
    w = exe.alloc((T, k), np.float32)
    exe.route_topk(dl, ids, w, T, n_exp, k, norm, rule=rule)
    gi, gw = ids.download(), w.download()
    ri, rw = O.route_topk(lg, k, norm, O.SUM_WAVE, rule=rule)
    assert np.array_equal(gi, ri)
    assert np.array_equal(gw.view(np.uint32), rw.view(np.uint32))
    # the reference's serial softmax order gives the same ids on this data
    si, _ = O.route_topk(lg, k, norm, O.SUM_SERIAL, rule=rule)
    assert np.array_equal(gi, si)
    assert list(gi[0]) == list(range(k))


def test_route_topk_nan_logits_are_memory_safe(exe):
    lg = np.full((2, 128), np.nan, np.float32)
    lg[1, :] = 0.0
    lg[1, 3] = np.nan
    ids = exe.alloc((2, 8), np.int32)
    w = exe.alloc((2, 8), np.float32)
    exe.route_topk(exe.upload(lg), ids, w, 2, 128, 8, True)
    ri, rw = O.route_topk(lg, 8, True, O.SUM_WAVE)
    assert np.array_equal(ids.download(), ri) and np.array_equal(w.download(), rw)
    assert list(ri[0]) == [-1] * 8


def test_router_end_to_end_matches_oracle(exe):
    """gate_gpu + MoeRouter.route (forward.rs:386-397, router.rs:25-56)."""
    import obsidian_hip as oh
    E, H = 128, 2048
    rng = np.random.default_rng(500)
    t = {k: v for k, v in synth.moe_layer(7, 4, H, 256, 64).items()}
    w, s, b = synth.quant_tensor(rng, E, H, 8, 64)
    x = synth.bf16_normal(rng, H)
    layer = oh.MoeLayer({"router_w": exe.upload(w).ptr, "router_s": exe.upload(s).ptr, "router_b": exe.upload(b).ptr})
    cfg = oh.MoeConfig(E, 8, H, 768, 64, True)
    logits = oh.gate_gpu(exe, layer, cfg, exe.upload(x))
    ids, wts = oh.MoeRouter(E, 8, True).route(exe, logits)
    lg_ref = O.qmatvec("lanes", 8, w, s, b, _f32(x), H, E)
    ri, rw = O.route_topk(lg_ref, 8, True, O.SUM_WAVE)
    assert ids == [int(i) for i in ri[0]]
    assert np.array_equal(np.float32(wts), rw[0])
    del t


def test_swiglu_and_scaled_add(exe):
    rng = np.random.default_rng(600)
    n = 4096
    g = synth.bf16_normal(rng, n, 4.0)
    u = synth.bf16_normal(rng, n, 2.0)
    h = exe.alloc(n, np.uint16)
    exe.swiglu_raw(exe.upload(g), exe.upload(u), h, n)
    ref = np.array([O.f32_to_bf16(O.silu_mul(float(a), float(c))) for a, c in zip(_f32(g), _f32(u))], np.uint16)
    assert np.array_equal(h.download(), ref)
    for m in (n, 1001):  # 16-byte vector path, then the one-element path (n % 8 != 0)
        acc = synth.bf16_normal(rng, m)
        y = synth.bf16_normal(rng, m)
        da = exe.upload(acc)
        exe.scaled_add_raw(da, exe.upload(y), 0.37, m)
        exact = np.float32(0.37).astype(np.float64) * _f32(y).astype(np.float64) + _f32(acc).astype(np.float64)
        assert np.array_equal(da.download(), synth.f32_to_bf16_bits(exact.astype(np.float32))), m


@pytest.mark.parametrize("rows,dim", [(1, 2048), (7, 2048), (300, 2048), (5, 1024), (3, 4096), (4, 192)])
def test_rmsnorm_bit_exact(exe, rows, dim):
    """obs_rmsnorm (rmsnorm.metal / Model::rmsnorm) equals the oracle bit for
    bit: same sum-of-squares order, IEEE sqrt and division, one bf16 rounding.
    dim 192 takes the generic (unvectorized) kernel."""
    rng = np.random.default_rng(rows * 7 + dim)
    x = synth.bf16_normal(rng, (rows, dim), 2.0)
    w = synth.bf16_normal(rng, dim, 1.0)
    eps = 1e-6
    out = exe.alloc((rows, dim), np.uint16)
    dx, dw = exe.upload(x), exe.upload(w)
    exe.rmsnorm_raw(dx, dw, out, rows, dim, eps)
    want = O.rmsnorm(x, w, eps)
    assert np.array_equal(out.download(), want)
    exe.rmsnorm_raw(dx, dw, dx, rows, dim, eps)  # in place (x and out alias)
    assert np.array_equal(dx.download(), want)


def test_rmsnorm_rejects_bad_dim(exe):
    buf = exe.alloc(256, np.uint16)
    with pytest.raises(oh.ObsError) as e:
        exe.rmsnorm_raw(buf, buf, buf, 1, 100, 1e-6)
    assert e.value.code == oh.OBS_E_SHAPE


def test_argument_validation_errors(exe):
    import obsidian_hip as oh
    buf = exe.alloc(1024, np.uint32)
    with pytest.raises(oh.ObsError) as ei:
        exe.q4_matvec(buf, buf, buf, buf, 96, 8, 64, y_f32=buf)  # 96 % 64 != 0
    assert ei.value.code == oh.OBS_E_SHAPE and "multiple of group" in str(ei.value)
    with pytest.raises(oh.ObsError) as ei:
        exe.route_topk(buf, buf, buf, 1, 300, 8, True)  # n_exp > 256
    assert ei.value.code == oh.OBS_E_SHAPE
    with pytest.raises(oh.ObsError) as ei:
        exe.route_topk(buf, buf, buf, 1, 128, 129, True)
    assert ei.value.code == oh.OBS_E_SHAPE
    with pytest.raises(oh.ObsError) as ei:
        exe.dequant_tensor(5, buf, buf, buf, 1, 64, 64, out_f32=buf)
    assert ei.value.code == oh.OBS_E_INVALID
