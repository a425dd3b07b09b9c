"""CPU checks of bench.py's parts that need no GPU: the one-GPU guard, the
rocprofv3 CSV reductions the committed profiles are made with, and the CPU
baseline leg (the oracle, timed on a short sample)."""
import csv
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    out = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120)
    assert out.returncode == 2
    assert "one GPU" in out.stdout + out.stderr


def _write_csv(path, fields, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        w.writerows(rows)


def test_pmc_summary_sums_instances_and_averages_dispatches(tmp_path, capsys):
    # Kernel A: two dispatches, FETCH_SIZE collected on two instances each
    # (summed within a dispatch: 3 + 5 and 7 + 9, averaged: 12); kernel B one.
    rows = []
    for disp, vals in ((1, (3, 5)), (2, (7, 9))):
        for v in vals:
            rows.append({"Kernel_Name": "kernel_a", "Dispatch_Id": disp, "Counter_Name": "FETCH_SIZE",
                         "Counter_Value": v})
    rows.append({"Kernel_Name": "kernel_b", "Dispatch_Id": 3, "Counter_Name": "FETCH_SIZE", "Counter_Value": 40})
    path = tmp_path / "pmc.csv"
    _write_csv(path, ["Kernel_Name", "Dispatch_Id", "Counter_Name", "Counter_Value"], rows)
    bench.pmc_summary([str(path)])
    out = capsys.readouterr().out.splitlines()
    a = next(l for l in out if l.endswith("kernel_a"))
    b = next(l for l in out if l.endswith("kernel_b"))
    assert a.split("|")[0].strip() == "2 dispatches" and "FETCH_SIZE=12" in a
    assert b.split("|")[0].strip() == "1 dispatches" and "FETCH_SIZE=40" in b


def test_trace_summary_maps_launches_onto_the_stack(tmp_path, capsys):
    """Two whole steps of the ModernBERT-base stack (88 projection launches
    each) after a partial one that is dropped; other kernels are ignored.
    Each projection gets its own duration, so the mapping and the rates
    are checked against closed forms."""
    from sys1_amd.stacks import CONFIGS
    cfg = CONFIGS["modernbert-base"]()
    seq = [p for layer in cfg.layers for p in layer]
    dur_ns = {"Wqkv": 30000, "attn.Wo": 15000, "Wi+geglu": 32000, "mlp.Wo": 20000}
    rows, t = [], 0
    for i in range(5):  # a stray launch of a partial step first
        rows.append({"Kernel_Name": "void sys1::gemm_tile_kernel<1>(sys1::GemmArgs)", "Start_Timestamp": t,
                     "End_Timestamp": t + 999})
        t += 1000
    for step in range(2):
        for p in seq:
            rows.append({"Kernel_Name": f"void sys1::gemm_tile_kernel<{p.name}>(sys1::GemmArgs)",
                         "Start_Timestamp": t, "End_Timestamp": t + dur_ns[p.name]})
            rows.append({"Kernel_Name": "some_other_kernel", "Start_Timestamp": t + 1,
                         "End_Timestamp": t + 2})
            t += dur_ns[p.name] + 100
    path = tmp_path / "trace.csv"
    _write_csv(path, ["Kernel_Name", "Start_Timestamp", "End_Timestamp"], rows)
    M = 1024
    bench.trace_summary(str(path), "modernbert-base", M)
    out = capsys.readouterr().out.splitlines()
    assert out[0].startswith("modernbert-base M=1024: 2 steps")
    per_step_us = sum(dur_ns[p.name] for p in seq) / 1e3
    assert f"kernel time per step {per_step_us:.1f} us" in out[0]
    for p in cfg.layers[1]:
        line = next(l for l in out[1:] if l.split()[0] == p.name)
        us = dur_ns[p.name] / 1e3
        assert f"{us:8.2f} us" in line
        assert f"{p.flops(M) / us / 1e6:7.1f} TFLOP/s" in line
        assert f"gemm_tile_kernel<{p.name}>" in line
        assert f"{2 * sum(q.name == p.name for q in seq):5d} launches" in line


def test_cpu_baseline_reports_a_port_on_a_short_sample():
    r = bench.cpu_baseline(0.2)
    assert r["kind"] == "port" and r["unit"] == "TFLOP/s"
    assert r["value"] > 0 and r["cores"] >= 1
    assert "M=1024" in r["sample"]
