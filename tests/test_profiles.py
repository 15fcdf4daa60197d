"""The rocprofv3 summarizer behind profiles/ (obsidian_hip.profiles): counter
CSVs become bytes per launch scaled by a device-copy calibration, with the
digest of each kernel's sources, which bench.py compares before it reports a
traffic figure."""
import csv
import os

import obsidian_hip.profiles as P


def _csv(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for r in rows:
            w.writerow(r)


def test_traffic_scales_by_the_copy_calibration(tmp_path):
    k = "void (anonymous namespace)::decode_fused_kernel<2, false>(FusedArgs)"
    cp = "__amd_rocclr_copyBuffer"
    _csv(tmp_path / "f.csv", [{"Dispatch_Id": i, "Kernel_Name": k, "Counter_Name": "FETCH_SIZE", "Counter_Value": 10000 + i}
                              for i in (1, 2)])
    _csv(tmp_path / "w.csv", [{"Dispatch_Id": 1, "Kernel_Name": k, "Counter_Name": "WRITE_SIZE", "Counter_Value": 100}])
    _csv(tmp_path / "cf.csv", [{"Dispatch_Id": 1, "Kernel_Name": cp, "Counter_Name": "FETCH_SIZE", "Counter_Value": 512},
                               {"Dispatch_Id": 2, "Kernel_Name": cp, "Counter_Name": "FETCH_SIZE", "Counter_Value": 1}])
    _csv(tmp_path / "cw.csv", [{"Dispatch_Id": 1, "Kernel_Name": cp, "Counter_Name": "WRITE_SIZE", "Counter_Value": 1024}])
    res = P.traffic(*(str(tmp_path / n) for n in ("f.csv", "w.csv", "cf.csv", "cw.csv")), copy_bytes=1 << 20)
    assert res["_calibration"]["fetch_scale"] == 2.0 and res["_calibration"]["write_scale"] == 1.0
    e = res["decode_fused"]
    assert e["dispatches"] == 2 and e["traffic_bytes_per_launch"] == int(10001.5 * 1024 * 2 + 100 * 1024)
    assert e["source_sha"] == P.source_digest("decode_fused") and len(e["source_sha"]) == 16


def test_digest_follows_the_sources():
    a = P.source_digest("grouped_gemm_gateup")
    assert a == P.source_digest("grouped_gemm_down")  # one source file holds both
    assert a != P.source_digest("decode_fused") and P.source_digest("nope") is None
    assert all(os.path.exists(os.path.join(P.PKG, f)) for _, fs in P.KERNELS.values() for f in fs)


def test_mfma_util_fractions(tmp_path):
    """Busy fractions per SIMD from the counters: 8 XCDs x 1,000 cycles each,
    1,024 SIMDs; MFMA busy 40%, VALU busy 50% (SQ_ACTIVE_INST_VALU counts 4
    cycles), both 15%, so neither 25%."""
    k = "void (anonymous namespace)::moe_ffn_kernel<2u>(GemmArgs, GemmArgs, FfnSync)"
    cyc, simds = 1000.0, 1024
    vals = {"GRBM_GUI_ACTIVE": 8 * cyc, "SQ_VALU_MFMA_BUSY_CYCLES": 0.4 * cyc * simds,
            "SQ_ACTIVE_INST_VALU": 0.5 * cyc * simds / 4, "SQ_VALU_MFMA_COEXEC_CYCLES": 0.15 * cyc * simds,
            "SQ_INSTS_MFMA": 0.4 * cyc * simds / 32, "SQ_INSTS_VALU": 3.0 * 0.4 * cyc * simds / 32,
            "SQ_WAVE_CYCLES": 1.0, "SQ_WAIT_INST_ANY": 1.0}
    path = tmp_path / "m.csv"
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value",
                                          "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        for d in (5, 9):
            for c, v in vals.items():
                w.writerow({"Dispatch_Id": d, "Kernel_Name": k, "Counter_Name": c, "Counter_Value": v,
                            "Start_Timestamp": 0, "End_Timestamp": 500})  # 0.5 us: 2 GHz
    r = P.mfma_util(str(path), "moe_ffn")
    assert r["dispatches"] == 2 and abs(r["clock_ghz"] - 2.0) < 1e-9
    assert abs(r["mfma_util"] - 0.4) < 1e-9 and abs(r["valu_busy"] - 0.5) < 1e-9
    assert abs(r["coexec"] - 0.15) < 1e-9 and abs(r["neither"] - 0.25) < 1e-9 and abs(r["valu_per_mfma"] - 3.0) < 1e-9
    assert "| moe_ffn | 2 |" in P.mfma_md(r, "moe_ffn", "cmd")
