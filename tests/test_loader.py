"""Checkpoint reading without a GPU: safetensors parsing, config.json, the
stacked / sharded / split layouts, and host reads (obs_ckpt_*).

Reference: Qwen3MoeConfig::from_file (src/model.rs:7-35), Weights::load_non_expert
(src/weight_loader.rs:19-71), ExpertIndex::open (src/disk_io.rs:36-63) and the
split format of tools/split_experts.py:9-19. Files are written by the
`safetensors` package (an independent writer); for malformed files the same
package's reader is the second opinion: every file the native parser rejects
here, it rejects too, and every file it accepts, it reads back identically.
"""
import json
import os
import struct

import numpy as np
import pytest

import obsidian_hip as oh
from obsidian_hip import synth

E, H, I, G, K = 8, 128, 64, 64, 2


def small_layer(seed: int):
    t = synth.moe_layer(seed, n_exp=E, hidden=H, inter=I, group=G)
    t["norm_w"] = synth.bf16_normal(np.random.default_rng(seed + 100), (H,))
    return t


@pytest.fixture(scope="module")
def layers():
    return {0: small_layer(1), 1: small_layer(2)}


@pytest.fixture(scope="module", params=["single", "sharded", "split"])
def ckdir(request, tmp_path_factory, layers):
    d = str(tmp_path_factory.mktemp(f"ck_{request.param}"))
    synth.write_checkpoint(d, layers, synth.hf_config(2, E, K, H, I, G), layout=request.param, shards=3)
    return request.param, d


def expected_bytes(layout, key, arr):
    """What the checkpoint holds for a MoeLayer key: the array itself, or, for
    split files, scales and biases cast to f16 (tools/split_experts.py:72-73)."""
    if layout == "split" and key[:-2] in ("gate", "up", "down") and key in synth.BF16_KEYS:
        return synth.bf16_bits_to_f32(arr).astype(np.float16)
    return arr


def test_every_layer_tensor_reads_back(ckdir, layers):
    layout, d = ckdir
    with oh.Checkpoint(d) as ck:
        for il, t in layers.items():
            for key, name in synth.CKPT_NAMES.items():
                full = f"model.layers.{il}.{name}"
                info = ck.tensor_info(full)
                want = expected_bytes(layout, key, t[key])
                got = ck.read(full)
                assert info.shape == want.shape, (full, info)
                assert info.nbytes == want.nbytes
                split_expert = layout == "split" and key[:-2] in ("gate", "up", "down")
                assert info.n_pieces == (E if split_expert else 1)
                assert info.dtype == ("F16" if split_expert and key in synth.BF16_KEYS else
                                      "BF16" if key in synth.BF16_KEYS else "U32")
                assert np.array_equal(got.view(want.dtype), want), full


def test_config_matches_the_written_json(ckdir):
    _, d = ckdir
    with oh.Checkpoint(d) as ck:
        cfg, n_layers = ck.config()
    assert n_layers == 2
    assert (cfg.n_exp, cfg.top_k, cfg.hidden, cfg.inter, cfg.group, cfg.norm_topk) == (E, K, H, I, G, True)
    assert cfg.rms_eps == np.float32(1e-6)


def test_stacked_tensor_wins_over_split_files(tmp_path, layers):
    d = str(tmp_path)
    synth.write_checkpoint(d, layers, synth.hf_config(2, E, K, H, I, G), layout="split")
    # Add the stacked switch_mlp tensors as well: they keep bf16 scales exactly.
    from safetensors.torch import save_file
    import torch
    stacked = {f"model.layers.0.{synth.CKPT_NAMES[k]}": torch.from_numpy(layers[0][k].copy()).view(torch.bfloat16)
               for k in ("gate_s",)}
    save_file(stacked, os.path.join(d, "extra.safetensors"))
    idx = {"weight_map": {n: "model.safetensors" for n in _names(os.path.join(d, "model.safetensors"))}}
    idx["weight_map"].update({n: "extra.safetensors" for n in stacked})
    json.dump(idx, open(os.path.join(d, "model.safetensors.index.json"), "w"))
    with oh.Checkpoint(d) as ck:
        info = ck.tensor_info("model.layers.0.mlp.switch_mlp.gate_proj.scales")
        assert (info.dtype, info.n_pieces) == ("BF16", 1)
        assert np.array_equal(ck.read("model.layers.0.mlp.switch_mlp.gate_proj.scales"), layers[0]["gate_s"])
        # the other projections still come from the split file
        assert ck.tensor_info("model.layers.0.mlp.switch_mlp.up_proj.scales").n_pieces == E


def _names(path):
    raw = open(path, "rb").read()
    n = struct.unpack("<Q", raw[:8])[0]
    return [k for k in json.loads(raw[8:8 + n]) if k != "__metadata__"]


def test_explicit_expert_dir_and_missing_expert(tmp_path, layers):
    d = str(tmp_path / "m")
    synth.write_checkpoint(d, layers, synth.hf_config(2, E, K, H, I, G), layout="split")
    os.rename(os.path.join(d, "splitted_moe"), str(tmp_path / "experts"))
    with oh.Checkpoint(d) as ck:  # no splitted_moe: the experts are not found
        with pytest.raises(oh.ObsError, match="not found"):
            ck.tensor_info("model.layers.0.mlp.switch_mlp.gate_proj.weight")
    with oh.Checkpoint(d, str(tmp_path / "experts")) as ck:
        assert ck.tensor_info("model.layers.0.mlp.switch_mlp.gate_proj.weight").shape == (E, I, H // 8)
    # config says more experts than the split file holds
    cfgp = os.path.join(d, "config.json")
    c = json.load(open(cfgp))
    c["num_experts"] = E + 1
    json.dump(c, open(cfgp, "w"))
    with oh.Checkpoint(d, str(tmp_path / "experts")) as ck:
        with pytest.raises(oh.ObsError, match=f"e{E}.gate_proj.weight' missing"):
            ck.tensor_info("model.layers.0.mlp.switch_mlp.gate_proj.weight")


def test_read_errors(ckdir):
    _, d = ckdir
    with oh.Checkpoint(d) as ck:
        with pytest.raises(oh.ObsError, match="not found"):
            ck.tensor_info("model.layers.7.mlp.gate.weight")
        name = "model.layers.0.mlp.gate.weight"
        small = np.empty(3, np.uint8)
        rc = oh.lib().obs_ckpt_read(ck.h, name.encode(), small.ctypes.data, small.nbytes)
        assert rc == oh.OBS_E_NOMEM and "needs" in oh.lib().obs_ckpt_error(ck.h).decode()


def test_open_errors(tmp_path):
    with pytest.raises(oh.ObsError, match="not a directory"):
        oh.Checkpoint(str(tmp_path / "nope"))
    (tmp_path / "config.json").write_text("{not json")
    with pytest.raises(oh.ObsError, match="config.json"):
        oh.Checkpoint(str(tmp_path))
    (tmp_path / "config.json").write_text("{}")
    (tmp_path / "model.safetensors.index.json").write_text('{"weight_map": {"a": "../x.safetensors"}}')
    with pytest.raises(oh.ObsError, match="not a file name"):
        oh.Checkpoint(str(tmp_path))


def _cfg_dir(tmp_path, **over):
    c = synth.hf_config(4, E, K, H, I, G)
    for k, v in over.items():
        if v is None:
            c.pop(k)
        else:
            c[k] = v
    (tmp_path / "config.json").write_text(json.dumps(c))
    return oh.Checkpoint(str(tmp_path))


@pytest.mark.parametrize("field", ["num_hidden_layers", "hidden_size", "num_attention_heads", "num_key_value_heads",
                                   "num_experts", "num_experts_per_tok", "moe_intermediate_size", "rms_norm_eps",
                                   "rope_theta", "vocab_size"])
def test_config_requires_the_reference_fields(tmp_path, field):
    # serde fails on a missing non-default field of Qwen3MoeConfig (model.rs:9-22)
    ck = _cfg_dir(tmp_path, **{field: None})
    with pytest.raises(oh.ObsError, match=f"missing field `{field}`"):
        ck.config()


def test_config_defaults_and_types(tmp_path):
    cfg, n = _cfg_dir(tmp_path, norm_topk_prob=None, quantization=None).config()
    assert (cfg.norm_topk, cfg.group, n) == (False, 64, 4)  # #[serde(default)]; group 64 as forward.rs:306
    cfg, _ = _cfg_dir(tmp_path, quantization={"group_size": 32, "bits": 4}, rms_norm_eps=1e-5).config()
    assert (cfg.group, cfg.rms_eps) == (32, np.float32(1e-5))
    for bad in ({"hidden_size": 2048.0}, {"hidden_size": -1}, {"num_experts": "128"},
                {"norm_topk_prob": 1}, {"rms_norm_eps": "1e-6"}):
        with pytest.raises(oh.ObsError):
            _cfg_dir(tmp_path, **bad).config()


def test_layer_table_size():
    cfg = oh.MoeConfig(E, K, H, I, G)
    a = lambda n: (n + 255) // 256 * 256
    want = (3 * (a(E * I * H // 2) + 2 * a(E * I * H // G * 2))  # gate, up, down: weight + scales + biases
            + a(E * H) + 2 * a(E * H // G * 2) + a(H * 2))      # router (8-bit), norm
    assert oh.lib().obs_moe_layer_bytes(oh.C.byref(cfg.to_c())) == want
    full = oh.MoeConfig()
    n = oh.lib().obs_moe_layer_bytes(oh.C.byref(full.to_c()))
    assert n == 128 * synth.bytes_per_expert() + synth.router_bytes() + 4096  # every piece is 256-aligned here
    assert oh.lib().obs_moe_layer_bytes(oh.C.byref(oh.MoeConfig(hidden=100).to_c())) == 0


# ---- malformed safetensors files ------------------------------------------------

def raw_file(header, data=b"", n=None, pad=True):
    h = header if isinstance(header, bytes) else json.dumps(header).encode()
    if pad:
        h += b" " * (-len(h) % 8)
    return struct.pack("<Q", len(h) if n is None else n) + h + data


def ok_header():
    return {"__metadata__": {"format": "pt"},
            "a": {"dtype": "F32", "shape": [2, 2], "data_offsets": [0, 16]},
            "b": {"dtype": "U8", "shape": [3], "data_offsets": [16, 19]}}


BAD = {
    "too_small": b"\x01\x00\x00",
    "header_too_large": struct.pack("<Q", 100_000_001) + b"{}",
    "header_beyond_file": raw_file(ok_header(), bytes(19), n=10_000),
    "not_utf8": raw_file(b'{"\xff": {"dtype": "U8", "shape": [0], "data_offsets": [0, 0]}}'),
    "no_brace": raw_file(b'[]'),
    "bad_json": raw_file(b'{"a": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]'),
    "unknown_dtype": raw_file({"a": {"dtype": "Q4", "shape": [1], "data_offsets": [0, 1]}}, b"\0"),
    "hole": raw_file({"a": {"dtype": "U8", "shape": [1], "data_offsets": [1, 2]}}, b"\0\0"),
    "overlap": raw_file({"a": {"dtype": "U8", "shape": [2], "data_offsets": [0, 2]},
                         "b": {"dtype": "U8", "shape": [2], "data_offsets": [1, 3]}}, b"\0\0\0"),
    "size_mismatch": raw_file({"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 4]}}, b"\0" * 4),
    "trailing_bytes": raw_file(ok_header(), bytes(20)),
    "short_data": raw_file(ok_header(), bytes(18)),
    "reversed_offsets": raw_file({"a": {"dtype": "U8", "shape": [0], "data_offsets": [1, 0]}}, b"\0"),
    "metadata_not_string": raw_file({"__metadata__": {"k": 1}}),
    "negative_dim": raw_file({"a": {"dtype": "U8", "shape": [-1], "data_offsets": [0, 0]}}),
    "float_offset": raw_file({"a": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1.0]}}, b"\0"),
}


def _native_open(tmp_path, blob):
    d = tmp_path / "m"
    d.mkdir(exist_ok=True)
    (d / "model.safetensors").write_bytes(blob)
    return oh.Checkpoint(str(d))


@pytest.mark.parametrize("case", sorted(BAD))
def test_malformed_file_is_rejected(tmp_path, case):
    from safetensors.numpy import load
    blob = BAD[case]
    with pytest.raises(Exception):  # the safetensors package rejects it too
        load(blob)
    with _native_open(tmp_path, blob) as ck:
        with pytest.raises(oh.ObsError) as ei:
            ck.tensor_info("a")
        assert ei.value.code == oh.OBS_E_SHAPE, str(ei.value)


def test_duplicate_names_are_rejected(tmp_path):
    blob = raw_file(b'{"a": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}, '
                    b'"a": {"dtype": "U8", "shape": [1], "data_offsets": [1, 2]}}', b"\0\0")
    with _native_open(tmp_path, blob) as ck:
        with pytest.raises(oh.ObsError, match="listed twice"):
            ck.tensor_info("a")


GOOD = {
    "plain": (raw_file(ok_header(), np.arange(4, dtype=np.float32).tobytes() + b"\x07\x08\x09"), ["a", "b"]),
    "unpadded": (raw_file(ok_header(), bytes(19), pad=False), ["a", "b"]),
    "empty": (raw_file({}), []),
    "null_metadata": (raw_file({"__metadata__": None}), []),
    "zero_size_and_scalar": (raw_file({"z": {"dtype": "F64", "shape": [0, 3], "data_offsets": [0, 0]},
                                       "s": {"dtype": "I32", "shape": [], "data_offsets": [0, 4]}},
                                      struct.pack("<i", -5)), ["z", "s"]),
    "escaped_names": (raw_file(b'{"\\u00e9t\\u00e9.w\\ud83d\\ude00": {"dtype": "U8", "shape": [2], '
                               b'"data_offsets": [0, 2]}, "tab\\tq\\"": {"dtype": "I16", "shape": [1], '
                               b'"data_offsets": [2, 4]}}', b"\x01\x02\x03\x04"),
                      ["été.w\U0001F600", 'tab\tq"']),
    "out_of_order": (raw_file({"b": {"dtype": "U8", "shape": [1], "data_offsets": [4, 5]},
                               "a": {"dtype": "F32", "shape": [1], "data_offsets": [0, 4]}}, bytes(5)), ["a", "b"]),
}


@pytest.mark.parametrize("case", sorted(GOOD))
def test_valid_file_reads_like_the_safetensors_package(tmp_path, case):
    from safetensors.numpy import load
    blob, names = GOOD[case]
    ref = load(blob)
    assert sorted(ref) == sorted(names)
    with _native_open(tmp_path, blob) as ck:
        for n in names:
            info = ck.tensor_info(n)
            assert info.shape == ref[n].shape
            got = ck.read(n)
            assert got.tobytes() == ref[n].tobytes()
        with pytest.raises(oh.ObsError, match="not found"):
            ck.tensor_info("missing")


def test_dtype_codes_follow_the_header():
    names = [v[0] for _, v in sorted(oh.DTYPES.items())]
    text = open(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                             "include", "obsidian_hip.h")).read()
    for code, n in enumerate(names):
        assert f"OBS_DT_{n} = {code}" in text
