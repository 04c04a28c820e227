"""bench.py's contract and its profile readers, on the CPU: `--gpus N` above 1 exits with a message
(one GPU is measured), and the rocprofv3 CSV readers that the summaries under profiles/ are made
with assign each launch its kind by its position in the token and scale the counters as their
docstrings state. The CSVs here are synthetic, in rocprofv3's column layout."""
import csv
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402

FIELDS = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def _token_kernels(layers, wf):
    names = {"qkv": f"void gemv_kernel<1, true, 3, {wf}, 1>(GemvArgs)",
             "o": f"void gemv_kernel<1, false, 1, {wf}, 1>(GemvArgs)",
             "gate_up": f"void gemv_kernel<1, true, 2, {wf}, 1>(GemvArgs)",
             "down": f"void gemv_kernel<1, false, 1, {wf}, 1>(GemvArgs)"}
    seq = [(k, names[k]) for _ in range(layers) for k in ("qkv", "o", "gate_up", "down")]
    return seq + [("lm_head", f"void gemv_kernel<1, true, 0, {wf}, 1>(GemvArgs)")]


def _write(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS)
        w.writeheader()
        w.writerows(rows)


def test_gemv_counters_kinds_scaling_and_shares(tmp_path, capsys):
    """Two passes over 2 tokens of a 2-layer model: per-kind values are chosen so that every column
    has a known answer (kind by position, o and down told apart, FETCH_SIZE scaled by the 1 GiB copy)."""
    layers, us = 2, 10.0
    per_kind = {"qkv": 1.0, "o": 2.0, "gate_up": 3.0, "down": 4.0, "lm_head": 5.0}
    a_rows, b_rows, d = [], [], 0
    for _ in range(2):  # tokens
        for kind, name in _token_kernels(layers, 1):
            d += 1
            v = per_kind[kind]
            t0 = d * 100_000
            common = {"Dispatch_Id": d, "Kernel_Name": name, "Start_Timestamp": t0, "End_Timestamp": t0 + int(us * 1e3)}
            # 1024 SIMDs at 2.4 GHz: 600 four-cycle units per us per SIMD; VALU share = v * 10 %
            valu = v * 0.1 * 1024 * 600 * us
            for c, val in [("SQ_WAVES", 2048.0), ("SQ_WAVE_CYCLES", 2 * 1024 * 600 * us), ("SQ_INSTS_VALU", 2048.0 * v),
                           ("SQ_ACTIVE_INST_VALU", valu), ("SQ_WAIT_INST_ANY", 0.0), ("SQ_INSTS_LDS", 0.0),
                           ("SQ_WAIT_INST_LDS", 0.0)]:
                a_rows.append(dict(common, Counter_Name=c, Counter_Value=val))
            b_rows.append(dict(common, Counter_Name="FETCH_SIZE", Counter_Value=1000.0 * v))
    d += 1
    b_rows.append({"Dispatch_Id": d, "Kernel_Name": "__amd_rocclr_copyBuffer", "Counter_Name": "FETCH_SIZE",
                   "Counter_Value": 2.0 ** 19, "Start_Timestamp": 0, "End_Timestamp": 1})
    _write(tmp_path / "a.csv", a_rows)
    _write(tmp_path / "b.csv", b_rows)
    bench.gemv_counters([str(tmp_path / "a.csv"), str(tmp_path / "b.csv")], layers=layers)
    out = capsys.readouterr().out
    assert "FETCH_SIZE scale: 2.0000 (from the 1 GiB copy" in out
    rows = {r.split("|")[1].strip(): [c.strip() for c in r.split("|")[1:-1]] for r in out.splitlines()
            if r.startswith("| ") and "gemv_kernel" in r}
    assert set(rows) == set(per_kind)
    for kind, v in per_kind.items():
        r = rows[kind]
        assert r[1] == "int8" and r[2] == "1"
        assert int(r[4]) == (2 if kind == "lm_head" else 2 * layers)  # launches over the two tokens
        assert r[5] == "2048" and float(r[6]) == pytest.approx(us)
        assert float(r[7]) == pytest.approx(v)  # VALU instructions per wave
        assert float(r[8]) == pytest.approx(10 * v, abs=0.05)  # SIMD VALU share %
        assert float(r[9]) == pytest.approx(2.0, abs=0.01)  # resident waves per SIMD
        assert float(r[14]) == pytest.approx(1000 * v * 1024 * 2 / 1e6, abs=0.01)  # MB per launch, scaled


def test_timeline_kinds_and_gaps(tmp_path, capsys):
    """Five 129-launch tokens (32 layers + lm_head), each launch 2 us long with a 0.5 us gap before it:
    the reader names o and down by their position and skips the eager pass and first replay."""
    rows, t = [], 0
    for _ in range(5):
        for kind, name in _token_kernels(32, 0):
            t += 500
            rows.append({"Dispatch_Id": len(rows) + 1, "Kernel_Name": name, "Counter_Name": "", "Counter_Value": 0,
                         "Start_Timestamp": t, "End_Timestamp": t + 2000})
            t += 2000
    _write(tmp_path / "trace.csv", rows)
    bench.timeline(str(tmp_path / "trace.csv"))
    out = capsys.readouterr().out
    assert out.startswith("tokens analysed: 3;")
    table = {r.split("|")[1].strip(): r for r in out.splitlines() if r.startswith("| ")}
    for kind, per in [("qkv", 32), ("o", 32), ("gate_up", 32), ("down", 32), ("lm_head", 1)]:
        cols = [c.strip() for c in table[kind].split("|")[1:-1]]
        assert int(cols[1]) == per and float(cols[2]) == pytest.approx(2.0) and float(cols[3]) == pytest.approx(0.5)
