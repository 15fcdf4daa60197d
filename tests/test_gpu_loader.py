"""Checkpoint -> HBM expert table on the GPU (obs_ckpt_load_moe_layer,
obs_ckpt_load_tensor): the resident table holds exactly the checkpoint's
bytes (stacked, sharded and split layouts; split f16 scales converted to
bf16 with round to nearest even, checked over all 65,536 f16 values), and a
decode over the loaded table equals the decode over the same arrays uploaded
directly, bit for bit, at the Qwen3-30B-A3B shape.

Reference: Weights::load_non_expert (src/weight_loader.rs:19-71), ExpertIndex
and read_experts_parallel (src/disk_io.rs:36-102), tools/split_experts.py:9-19.
"""
import ctypes as C
import time

import numpy as np
import pytest

import oracle as O
import obsidian_hip as oh
from obsidian_hip import synth

pytestmark = pytest.mark.gpu

E, H, I, G, K = 8, 128, 64, 64, 2


def view(exe, ptr, shape, dtype):
    """Host copy of a device region the loader filled."""
    dt = np.dtype(dtype)
    return oh.DeviceBuffer(exe, ptr, int(np.prod(shape)) * dt.itemsize, dt, tuple(shape), owned=False).download()


def small_layer(seed):
    t = synth.moe_layer(seed, n_exp=E, hidden=H, inter=I, group=G)
    t["norm_w"] = synth.bf16_normal(np.random.default_rng(seed + 7), (H,))
    return t


def expected_table(layout, key, a):
    if layout == "split" and key in synth.BF16_KEYS and key[:-2] in ("gate", "up", "down"):
        return synth.f32_to_bf16_bits(synth.bf16_bits_to_f32(a).astype(np.float16).astype(np.float32))
    return a


@pytest.mark.parametrize("layout", ["single", "sharded", "split"])
def test_loaded_table_holds_the_checkpoint_bytes(exe, tmp_path, layout):
    layers = {0: small_layer(3), 1: small_layer(4)}
    synth.write_checkpoint(str(tmp_path), layers, synth.hf_config(2, E, K, H, I, G), layout=layout, shards=3)
    with oh.Checkpoint(str(tmp_path)) as ck:
        cfg, _ = ck.config()
        for il in (1, 0):
            layer = ck.load_moe_layer(exe, il, cfg)
            for key in oh.PROJ_KEYS + ("norm_w",):
                want = expected_table(layout, key, layers[il][key])
                got = view(exe, layer.ptrs[key], want.shape, want.dtype)
                assert np.array_equal(got, want), (layout, il, key)
            assert layer.block is not None and layer.ptrs["gate_w"] == layer.block.ptr
            # a tensor loaded on its own keeps its on-disk bytes
            buf = ck.load_tensor(exe, f"model.layers.{il}.mlp.gate.scales")
            assert np.array_equal(buf.download(), layers[il]["router_s"])


def test_f16_to_bf16_conversion_covers_every_f16(exe, tmp_path):
    """Split files carry f16 scales (tools/split_experts.py:72-73); the loader
    widens each exactly to fp32 and rounds to bf16 (nearest even, NaN quiet).
    gate_s [8, 512, 16] holds all 65,536 f16 bit patterns."""
    e, h, i, g = 8, 512, 512, 32
    t = synth.moe_layer(5, n_exp=e, hidden=h, inter=i, group=g)
    allf16 = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).reshape(e, i, h // g)
    t["gate_s"] = allf16
    synth.write_checkpoint(str(tmp_path), {0: t}, synth.hf_config(1, e, 2, h, i, g), layout="split")
    with oh.Checkpoint(str(tmp_path)) as ck:
        assert ck.tensor_info("model.layers.0.mlp.switch_mlp.gate_proj.scales").dtype == "F16"
        layer = ck.load_moe_layer(exe, 0)
        got = view(exe, layer.ptrs["gate_s"], allf16.shape, np.uint16)
    want = synth.f32_to_bf16_bits(allf16.astype(np.float32))
    assert np.array_equal(got, want)
    # spot values: the f16 extremes and the halfway case
    flat = got.reshape(-1)
    assert flat[0x3C00] == 0x3F80            # 1.0
    assert flat[0x7BFF] == 0x4780            # 65504 -> 65536 (rounds up past 7 mantissa bits)
    assert flat[0x0001] == 0x3380            # 2^-24 (f16 subnormal) is a bf16 normal
    assert flat[0x7C00] == 0x7F80 and flat[0xFC00] == 0xFF80
    assert flat[0x3C01] == 0x3F80            # 1 + 2^-10 rounds to 1.0


def test_layer_load_errors(exe, tmp_path):
    t = small_layer(6)
    synth.write_checkpoint(str(tmp_path), {0: t}, synth.hf_config(1, E, K, H, I, G), layout="single")
    L = oh.lib()
    with oh.Checkpoint(str(tmp_path)) as ck:
        cfg, _ = ck.config()
        n = L.obs_moe_layer_bytes(C.byref(cfg.to_c()))
        bad = oh.MoeConfig(E, K, H, I * 2, G)
        n_bad = L.obs_moe_layer_bytes(C.byref(bad.to_c()))
        block = exe.alloc((max(n, n_bad),), np.uint8)
        out = oh.ObsMoeLayer()

        def load(c, ptr, nbytes, layer=0):
            return L.obs_ckpt_load_moe_layer(exe.ctx, ck.h, layer, C.byref(c.to_c()), ptr, nbytes, C.byref(out))

        assert load(cfg, block.ptr, n) == oh.OBS_OK
        assert load(cfg, block.ptr + 16, n) == oh.OBS_E_ALIGN
        assert load(cfg, block.ptr, n - 1) == oh.OBS_E_NOMEM
        assert load(bad, block.ptr, n_bad) == oh.OBS_E_SHAPE
        assert "the config needs [8, 128, 16]" in exe.last_error()
        assert load(cfg, block.ptr, n, layer=3) == oh.OBS_E_INVALID
        assert "not found" in exe.last_error()
    # a 4-bit router gate is refused with the reason
    t4 = dict(t)
    t4["router_w"], t4["router_s"], t4["router_b"] = synth.quant_tensor(np.random.default_rng(0), E, H, 4, G)
    d2 = tmp_path / "g4"
    synth.write_checkpoint(str(d2), {0: t4}, synth.hf_config(1, E, K, H, I, G), layout="single")
    with oh.Checkpoint(str(d2)) as ck:
        with pytest.raises(oh.ObsError, match="8-bit router gate"):
            ck.load_moe_layer(exe, 0)
    # no norm weight in the checkpoint: norm_w stays NULL
    t0 = dict(t)
    t0.pop("norm_w")
    d3 = tmp_path / "nonorm"
    synth.write_checkpoint(str(d3), {0: t0}, synth.hf_config(1, E, K, H, I, G), layout="sharded")
    with oh.Checkpoint(str(d3)) as ck:
        assert "norm_w" not in ck.load_moe_layer(exe, 0).ptrs


@pytest.fixture(scope="module")
def full_ckpt(tmp_path_factory):
    """One Qwen3-30B-A3B-shaped layer (128 experts, H 2048, I 768) as a
    two-shard checkpoint, stored as layer 5."""
    d = tmp_path_factory.mktemp("qwen_ckpt")
    t = synth.moe_layer(21, 128, 2048, 768, 64)
    t["norm_w"] = synth.bf16_normal(np.random.default_rng(22), 2048, 0.5)
    synth.write_checkpoint(str(d), {5: t}, synth.hf_config(48), layout="sharded", shards=2)
    return str(d), t


def test_decode_on_loaded_table_equals_uploaded(exe, full_ckpt):
    d, t = full_ckpt
    with oh.Checkpoint(d) as ck:
        cfg, n_layers = ck.config()
        assert n_layers == 48 and (cfg.n_exp, cfg.hidden, cfg.inter) == (128, 2048, 768)
        t0 = time.perf_counter()
        loaded = ck.load_moe_layer(exe, 5, cfg)
        dt = time.perf_counter() - t0
    nbytes = loaded.block.nbytes
    print(f"layer table {nbytes / 1e6:.1f} MB loaded in {dt * 1e3:.1f} ms ({nbytes / dt / 1e9:.2f} GB/s, page cache warm)")
    uploaded = oh.MoeLayer.upload(exe, t)
    L = O.Layer(t, 128, 2048, 768, 64)
    for seed in range(3):
        x1 = synth.bf16_normal(np.random.default_rng(300 + seed), 2048, 3.0)
        dx = exe.upload(x1)
        outs = []
        for layer in (loaded, uploaded):
            y = exe.alloc(2048, np.uint16)
            ids = exe.alloc(8, np.int32)
            w = exe.alloc(8, np.float32)
            exe.moe_decode(cfg, layer, dx, y, residual=dx, ids_out=ids, w_out=w)
            exe.device_status()
            outs.append((y.download(), ids.download(), w.download()))
        assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
        # and the loaded layer agrees with the oracle on the normalised input
        x1n = O.rmsnorm(x1, t["norm_w"], cfg.rms_eps)
        _, ri, rw = O.router(L, x1n, 8, True)
        assert np.array_equal(outs[0][1], ri[0])
        assert np.array_equal(outs[0][2].view(np.uint32), rw[0].view(np.uint32))
        y64, _, _ = O.moe_decode(L, x1n, 8, True, ids=outs[0][1][None], w=outs[0][2][None])
        y64 = y64[0] + synth.bf16_bits_to_f32(x1).astype(np.float64)
        y = synth.bf16_bits_to_f32(outs[0][0]).astype(np.float64)
        assert np.linalg.norm(y - y64) / np.linalg.norm(y64) <= 1e-2
