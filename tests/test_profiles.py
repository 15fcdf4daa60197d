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
