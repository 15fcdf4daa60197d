"""GPU parity of the decoder around the MoE block (forward.rs:398-443,
:445-462, :552-567) on a small seeded model: stage by stage against the
oracle with the GPU's own stage inputs (so one stage's rounding does not
compound into the next), the routing bit-exact, and the captured step graph
equal to eager steps bit for bit.

Bars: the attention half and the MoE half within 1e-2 of the fp64 oracle
(2-norm, and elementwise with a floor of 1e-2 rms), routing ids and weights
bit-exact with the oracle router on the GPU's post-attention state, logits
within 1e-2, the greedy token equal to the oracle argmax of the same logits."""
import numpy as np
import pytest

import oracle as O
import obsidian_hip as oh
from obsidian_hip import decoder as D
from obsidian_hip import synth

pytestmark = pytest.mark.gpu

# 16 query heads: the attention half as separate launches; the Qwen3-30B-A3B
# attention shape (32 / 4 heads): one launch (obs_attn_decode)
CFGS = {
    "split": D.DecoderConfig(n_layers=2, hidden=2048, n_heads=16, n_kv=2, head_dim=128, n_exp=8, top_k=2,
                             inter=256, vocab=512, max_len=64),
    "fused": D.DecoderConfig(n_layers=2, hidden=2048, n_heads=32, n_kv=4, head_dim=128, n_exp=8, top_k=2,
                             inter=256, vocab=512, max_len=64),
    # the Qwen3-30B-A3B expert shape too (inter 768, top-8, with 16 experts):
    # the MoE half runs as the one-launch kernel with its norm and residual
    "q30": D.DecoderConfig(n_layers=2, hidden=2048, n_heads=32, n_kv=4, head_dim=128, n_exp=16, top_k=8,
                           inter=768, vocab=512, max_len=64),
}


def _ocfg(c):
    return {"hidden": c.hidden, "n_heads": c.n_heads, "n_kv": c.n_kv, "head_dim": c.head_dim, "eps": c.rms_eps,
            "theta": c.rope_theta, "top_k": c.top_k, "norm_topk": c.norm_topk, "vocab": c.vocab}


@pytest.fixture(scope="module", params=sorted(CFGS))
def model(exe, request):
    cfg = CFGS[request.param]
    layers, glob = synth.decoder_weights(3, cfg.n_layers, cfg.hidden, cfg.n_heads, cfg.n_kv, cfg.head_dim,
                                         cfg.n_exp, cfg.inter, cfg.vocab)
    dl, dg = D.upload_weights(exe, layers, glob)
    m = D.Model(exe, cfg, dl, dg)
    assert m.fused_attention() == (request.param != "split")
    moes = [O.Layer(t, cfg.n_exp, cfg.hidden, cfg.inter) for t in layers]
    yield m, layers, glob, moes
    m.close()


def _f(b):
    return synth.bf16_bits_to_f32(b).astype(np.float64)


def _close(got, want, tol=1e-2):
    rel = float(np.linalg.norm(got - want) / np.linalg.norm(want))
    assert rel <= tol, rel
    floor = tol * np.sqrt(np.mean(want ** 2))
    assert np.all(np.abs(got - want) <= tol * np.abs(want) + floor)
    return rel


def test_decoder_stages_match_oracle(exe, model):
    m, layers, glob, moes = model
    CFG, OCFG = m.cfg, _ocfg(m.cfg)
    caches = [(np.zeros((CFG.n_kv, CFG.max_len, CFG.head_dim), np.uint16),
               np.zeros((CFG.n_kv, CFG.max_len, CFG.head_dim), np.uint16)) for _ in range(CFG.n_layers)]
    ids_buf = exe.alloc(CFG.top_k, np.int32)
    w_buf = exe.alloc(CFG.top_k, np.float32)
    toks = [5, 17, 300, 2, 511, 9]
    worst = 0.0
    for pos, tok in enumerate(toks):
        m.set_state(pos, tok)
        m.embed()
        want_x = synth.f32_to_bf16_bits(O.dequant(4, glob["embed_w"][tok:tok + 1], glob["embed_s"][tok:tok + 1],
                                                  glob["embed_b"][tok:tok + 1], 1, CFG.hidden)[0])
        assert np.array_equal(m.x.download(), want_x)
        for il in range(CFG.n_layers):
            x_in = m.x.download()
            m.forward_layer(il, ids_buf, w_buf)
            x1, x_out = m.x1.download(), m.x.download()
            kc, vc = caches[il]
            x1_ref = O.attention_half(layers[il], x_in, kc, vc, pos, OCFG)
            worst = max(worst, _close(_f(x1), _f(x1_ref)))
            # routing on the GPU's own post-attention state: bit-exact
            gi, gw = ids_buf.download(), w_buf.download()
            out_ref, ri, rw = O.moe_half(layers[il], moes[il], x1, OCFG)
            assert np.array_equal(gi, ri[0]) and np.array_equal(gw.view(np.uint32), rw[0].view(np.uint32))
            worst = max(worst, _close(_f(x_out), _f(out_ref)))
        m.head()
        logits = m.logits.download()
        xn = O.rmsnorm(m.x.download(), glob["final_norm"], CFG.rms_eps)
        ref, _ = O.qmatvec("f64", 4, glob["lm_w"], glob["lm_s"], glob["lm_b"], synth.bf16_bits_to_f32(xn),
                           CFG.hidden, CFG.vocab)
        worst = max(worst, _close(logits.astype(np.float64), ref))
        pos_after, tok_after = m.read_state()
        assert (pos_after, tok_after) == (pos + 1, O.argmax(logits))
    print(f"worst stage error {worst:.2e}")


def test_graph_replay_equals_eager_steps(exe, model):
    m = model[0]
    CFG = m.cfg
    m.close()
    eager = m.generate(7, 10, 6, graph=False)
    logits_eager = m.logits.download()
    graph = m.generate(7, 10, 6, graph=True)
    assert graph == eager
    assert np.array_equal(m.logits.download(), logits_eager)
    print("tokens", eager)


def test_graph_survives_another_models_rope_table(exe, model):
    """A second model on the same executor with another RoPE theta (and a
    longer cache) builds its own table; the first model's captured graph keeps
    its table and still replays equal to eager steps."""
    import dataclasses
    m = model[0]
    m.close()
    eager = m.generate(7, 10, 6, graph=False)
    logits_eager = m.logits.download()
    assert m.generate(7, 10, 6, graph=True) == eager
    for theta, max_len in ((5e5, m.cfg.max_len), (1e6, 2 * m.cfg.max_len)):
        m2 = D.Model(exe, dataclasses.replace(m.cfg, rope_theta=theta, max_len=max_len), m.layers, m.glob)
        m2.generate(7, 10, 6, graph=False)
        assert not np.array_equal(m2.logits.download(), logits_eager)  # theta reaches the result
        m2.close()
        assert m.generate(7, 10, 6, graph=True) == eager
        assert np.array_equal(m.logits.download(), logits_eager)
    m.close()


def test_generation_stays_in_the_cache(exe, model):
    m = model[0]
    CFG = m.cfg
    with pytest.raises(ValueError):
        m.generate(1, CFG.max_len - 2, 5)
    with pytest.raises(ValueError):
        m.set_state(CFG.max_len, 0)
