"""The checkpoint reader under AddressSanitizer and UBSan, and against the
`safetensors` package on mutated files (no GPU).

`make -f sanitize.mk` in project-obsidian_amd rebuilds every source with both
sanitizers on the host pass only (the GPU code is built as usual) and links
them into tests/loader_check.cpp, which runs obs_ckpt_open / _config /
_tensor_info / _read over a job list. The corpus: the malformed and valid
files of test_loader.py, seeded mutations of valid files (a header byte
overwritten, inserted or deleted, the length field moved, the file cut short
or extended) and whole checkpoints in the three layouts with damaged
config.json and index files. The checker must exit cleanly (a sanitizer report
aborts it) and print exactly what the regular build returns through ctypes.
For every single-file case the regular build must accept what the package
accepts, with the same shapes and bytes, and reject what it rejects
(SafeTensors::deserialize, used at disk_io.rs:43 and weight_loader.rs:38).
"""
import json
import os
import shutil
import struct
import subprocess

import numpy as np
import pytest

import obsidian_hip as oh
from obsidian_hip import synth
from test_loader import BAD, GOOD, raw_file

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "project-obsidian_amd")
CHECKER = os.path.join(PKG, "_build_san", "loader_check")
C = oh.C

N_MUTANTS = 400


@pytest.fixture(scope="module")
def checker():
    if not shutil.which("make") or not os.path.exists("/opt/rocm/bin/hipcc"):
        pytest.skip("make or hipcc missing")
    subprocess.run(["make", "-C", PKG, "-f", "sanitize.mk", "-j", str(min(16, os.cpu_count() or 4))], check=True,
                   stdout=subprocess.DEVNULL)
    return CHECKER


# ---- the corpus ------------------------------------------------------------------

def rich_file():
    """A valid file with several dtypes, a zero-size tensor, a scalar and metadata,
    written by the package (an independent writer)."""
    from safetensors.numpy import save
    rng = np.random.default_rng(7)
    return save({"w": rng.standard_normal((3, 4)).astype(np.float32), "b": np.arange(7, dtype=np.uint8),
                 "i": np.array([-2, 5], dtype=np.int64), "h": rng.standard_normal(5).astype(np.float16),
                 "z": np.zeros((0, 3), dtype=np.int8), "s": np.array(2.5, dtype=np.float64)},
                metadata={"format": "pt", "note": "x"})


JSON_BYTES = b'{}[]",:0123456789-+.eE \\u\x00\xff\xc3'


def mutate(blob: bytes, rng) -> bytes:
    b = bytearray(blob)
    n = struct.unpack("<Q", bytes(b[:8]))[0] if len(b) >= 8 else 0
    end = min(len(b), 8 + n)
    kind = int(rng.integers(7))
    if kind <= 2 and end > 8:
        i = int(rng.integers(8, end))
        c = JSON_BYTES[int(rng.integers(len(JSON_BYTES)))]
        if kind == 0:
            b[i] = c  # overwrite
        elif kind == 1:
            b.insert(i, c)  # insert (the length field now splits the header differently)
        else:
            del b[i]
    elif kind == 3 and len(b) >= 8:  # move the length field
        d = int(rng.choice([-9, -8, -2, -1, 1, 2, 8, 9, 1 << 20, 1 << 40]))
        b[:8] = struct.pack("<Q", max(0, min(n + d, (1 << 64) - 1)))
    elif kind == 4:  # cut short
        del b[int(rng.integers(0, max(1, len(b)))):]
    elif kind == 5:  # extend
        b += bytes(int(rng.integers(1, 17)))
    elif end > 8:  # a digit changed: offsets and shapes
        digits = [i for i in range(8, end) if 48 <= b[i] <= 57]
        if digits:
            b[digits[int(rng.integers(len(digits)))]] = 48 + int(rng.integers(10))
    return bytes(b)


def header_names(blob: bytes):
    """Tensor names in a blob's header, if it parses as JSON (for the queries)."""
    try:
        n = struct.unpack("<Q", blob[:8])[0]
        h = json.loads(blob[8:8 + n].decode("utf-8"))
        names = [k for k in h if k != "__metadata__"] if isinstance(h, dict) else []
    except Exception:
        return []
    out = []
    for k in names:  # a lone surrogate escape names no UTF-8 string: such a file is rejected anyway
        try:
            k.encode("utf-8")
            out.append(k)
        except UnicodeEncodeError:
            pass
    return out


def reformat(blob: bytes, rng) -> bytes:
    """The same file with its header JSON re-serialized: keys in another order,
    other whitespace and escapes (still valid: both readers must accept it)."""
    n = struct.unpack("<Q", blob[:8])[0]
    h = json.loads(blob[8:8 + n].decode("utf-8"))
    keys = list(h)
    rng.shuffle(keys)
    seps = [(",", ":"), (", ", ": "), (" ,\n", " :\t")][int(rng.integers(3))]
    text = json.dumps({k: h[k] for k in keys}, separators=seps, ensure_ascii=bool(rng.integers(2)),
                      indent=[None, 1, "\t"][int(rng.integers(3))])
    return raw_file(text.encode("utf-8"), blob[8 + n:], pad=bool(rng.integers(2)))


def single_file_cases():
    cases = {f"bad_{k}": (v, ["a"]) for k, v in BAD.items()}
    cases.update({f"good_{k}": (v[0], list(v[1])) for k, v in GOOD.items()})
    bases = [GOOD["plain"][0], GOOD["escaped_names"][0], GOOD["zero_size_and_scalar"][0], rich_file()]
    rng = np.random.default_rng(2024)
    for i in range(N_MUTANTS):
        base = bases[i % len(bases)]
        blob = base
        for _ in range(1 + int(rng.integers(3))):
            blob = mutate(blob, rng)
        cases[f"mut{i}"] = (blob, sorted(set(header_names(base)) | set(header_names(blob))))
    for i in range(40):
        base = bases[i % len(bases)]
        cases[f"fmt{i}"] = (reformat(base, rng), header_names(base))
    return cases


# ---- the regular build through ctypes, rendered like the checker -------------------

def render(model_dir: str, names) -> str:
    L = oh.lib()
    h = C.c_void_p()
    rc = L.obs_ckpt_open(os.fsencode(model_dir), None, C.byref(h))
    out = f"open {rc}"
    if rc == oh.OBS_OK:
        cfg, nl = oh.ObsMoeConfig(), C.c_uint32()
        rcc = L.obs_ckpt_config(h, C.byref(cfg), C.byref(nl))
        out += f" config {rcc}"
        if rcc == oh.OBS_OK:
            out += f" {cfg.n_exp} {cfg.top_k} {cfg.hidden} {cfg.inter} {cfg.group} {nl.value}"
        for name in names:
            info = oh.ObsTensorInfo()
            ri = L.obs_ckpt_tensor_info(h, name.encode(), C.byref(info))
            out += f" | {ri}"
            if ri != oh.OBS_OK:
                continue
            shape = ",".join(str(int(info.shape[d])) for d in range(min(info.ndim, 8)))
            buf = (C.c_ubyte * max(1, int(info.nbytes)))()
            rr = L.obs_ckpt_read(h, name.encode(), buf, info.nbytes)
            hv = 0xcbf29ce484222325
            if rr == oh.OBS_OK:
                for x in bytes(buf)[:int(info.nbytes)]:
                    hv = ((hv ^ x) * 0x100000001b3) & 0xFFFFFFFFFFFFFFFF
            else:
                hv = 0
            out += f" {info.dtype} [{shape}] {int(info.nbytes)} {rr} {hv:016x}"
        L.obs_ckpt_close(h)
    return out


def job_line(model_dir: str, names) -> str:
    return " ".join([model_dir.encode().hex()] + [n.encode().hex() for n in names])


def run_checker(checker, tmp_path, jobs):
    jf = tmp_path / "jobs.txt"
    jf.write_text("".join(job_line(d, n) + "\n" for d, n in jobs))
    env = dict(os.environ, ASAN_OPTIONS="abort_on_error=0:halt_on_error=1:detect_leaks=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([checker, str(jf)], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0, r.stderr[-4000:]
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-4000:]
    return r.stdout.splitlines()


# ---- the tests ---------------------------------------------------------------------

def test_single_files_match_the_package_and_the_sanitized_build(checker, tmp_path):
    from safetensors.numpy import load
    known = {v[0] for v in oh.DTYPES.values()}
    cases = single_file_cases()
    jobs, mismatch = [], []
    accepted = rejected = 0
    for key, (blob, names) in sorted(cases.items()):
        d = tmp_path / key
        d.mkdir()
        (d / "model.safetensors").write_bytes(blob)
        jobs.append((str(d), names))
        try:
            ref = load(blob)
        except Exception:
            ref = None
        got = render(str(d), names)
        fields = got.split(" | ")[1:]
        if ref is None:
            rejected += 1
            if any(f.split()[0] == "0" for f in fields):
                mismatch.append((key, "package rejects, native accepts", got))
            continue
        h = json.loads(blob[8:8 + struct.unpack("<Q", blob[:8])[0]].decode("utf-8"))
        if any(isinstance(v, dict) and v.get("dtype") not in known for k, v in h.items() if k != "__metadata__"):
            continue  # a dtype newer than the reference's safetensors 0.4.5 (Cargo.lock:1313-1314)
        accepted += 1
        with oh.Checkpoint(str(d)) as ck:
            for n in names:
                if n in ref:
                    info = ck.tensor_info(n)
                    if info.shape != ref[n].shape or ck.read(n).tobytes() != ref[n].tobytes():
                        mismatch.append((key, f"tensor {n!r} differs", got))
                else:
                    with pytest.raises(oh.ObsError):
                        ck.tensor_info(n)
    assert not mismatch, mismatch[:5]
    assert accepted >= 50 and rejected >= 300, (accepted, rejected)  # the corpus exercises both sides
    assert run_checker(checker, tmp_path, jobs) == [render(d, n) for d, n in jobs]


def test_checkpoints_and_damaged_configs_under_the_sanitized_build(checker, tmp_path):
    E, K, H, I, G = 8, 2, 128, 64, 64
    layers = {0: synth.moe_layer(1, n_exp=E, hidden=H, inter=I, group=G)}
    layers[0]["norm_w"] = synth.bf16_normal(np.random.default_rng(3), (H,))
    names = [f"model.layers.0.{synth.CKPT_NAMES[k]}" for k in sorted(layers[0])] + ["model.layers.1.missing"]
    cfg = synth.hf_config(1, E, K, H, I, G)
    jobs = []
    rng = np.random.default_rng(11)
    for layout in ("single", "sharded", "split"):
        base = tmp_path / f"ck_{layout}"
        synth.write_checkpoint(str(base), layers, cfg, layout=layout, shards=2)
        jobs.append((str(base), names))
        for i in range(12):  # config.json and index damage
            d = tmp_path / f"ck_{layout}_{i}"
            shutil.copytree(base, d)
            c = dict(cfg)
            if i < 4:
                c.pop(sorted(c)[int(rng.integers(len(c)))])
            elif i < 8:
                c[sorted(c)[int(rng.integers(len(c)))]] = [None, "x", -1, 1.5, {"a": 1}, 1 << 40][i % 6]
            (d / "config.json").write_text(json.dumps(c) if i != 8 else json.dumps(c)[:-3])
            idx = d / "model.safetensors.index.json"
            if i >= 9 and idx.exists():
                t = idx.read_text()
                idx.write_text([t[: len(t) // 2], t.replace("weight_map", "weight_mop"),
                                t.replace(".safetensors", "/../x.safetensors", 1)][i - 9])
            jobs.append((str(d), names))
    want = [render(d, n) for d, n in jobs]
    assert want[0].startswith("open 0 config 0 ") and " | 0 " in want[0]  # the intact checkpoint reads back
    assert run_checker(checker, tmp_path, jobs) == want
