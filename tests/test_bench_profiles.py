"""bench.py's profile summaries (CPU only): the rocprofv3 CSV parsers, the machine-readable
lines they write, and that a stored figure is used only with the kernel sources it was made
from."""
import csv
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402

PMC_FIELDS = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id", "Grid_Size",
              "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size", "Scratch_Size", "VGPR_Count",
              "Accum_VGPR_Count", "SGPR_Count", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]


def _pmc_csv(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, PMC_FIELDS)
        w.writeheader()
        for d, (kernel, counter, value) in enumerate(rows):
            r = {k: 0 for k in PMC_FIELDS}
            r.update(Dispatch_Id=d + 1, Kernel_Name=kernel, Counter_Name=counter, Counter_Value=value)
            w.writerow(r)


def test_traffic_summary_scales_by_the_copy_kernel(tmp_path):
    copy = "__amd_rocclr_copyBuffer(void)"
    gate = "void (anonymous namespace)::slot_gate_kernel<unsigned short, 64, 64, false, true>(int)"
    _pmc_csv(tmp_path / "f.csv", [(copy, "FETCH_SIZE", 32768.0), (gate, "FETCH_SIZE", 100.0), (gate, "FETCH_SIZE", 300.0)])
    _pmc_csv(tmp_path / "w.csv", [(copy, "WRITE_SIZE", 65536.0), (gate, "WRITE_SIZE", 50.0)])
    text = bench.pmc_summary(tmp_path / "f.csv", tmp_path / "w.csv", copy_bytes=64 << 20)
    assert "FETCH_SIZE x 2.0000, WRITE_SIZE x 1.0000" in text
    line = [ln for ln in text.splitlines() if ln.startswith("traffic_bytes_per_launch:")]
    assert line == [f"traffic_bytes_per_launch: slot_gate {(200 * 2 + 50) * 1024}"]


def test_mfma_summary_and_stored_metric(tmp_path, monkeypatch):
    gemm = "void (anonymous namespace)::gemm_bt_kernel<2, false>(int)"
    _pmc_csv(tmp_path / "m.csv", [(gemm, "MfmaUtil", 40.0), (gemm, "SQ_INSTS_VALU_MFMA_MOPS_BF16", 1e6)])
    text = bench.mfma_summary(tmp_path / "m.csv")
    assert "mfma_busy: out_proj 0.4" in text
    path = tmp_path / "mfma.md"
    path.write_text("# header\n" + text)
    assert bench.stored_metric(str(path), "mfma_busy") == {"out_proj": 0.4}
    monkeypatch.setattr(bench, "source_hash", lambda: "another build")
    assert bench.stored_metric(str(path), "mfma_busy") == {}


def test_stats_summary_lines(tmp_path):
    path = tmp_path / "s.csv"
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs", "StdDev"])
        w.writeheader()
        w.writerow(dict(Name="void (anonymous namespace)::norm_conv_kernel<unsigned short, 2, 16>(int)", Calls=312,
                        TotalDurationNs=0, AverageNs=29500.0, Percentage=5.0, MinNs=0, MaxNs=0, StdDev=0))
    text = bench.stats_summary(path)
    assert "avg_us: norm_conv 29.5" in text
    assert text.splitlines()[0].startswith(bench.SOURCE_KEY)


def test_cpu_baselines_of_the_block_and_decode_workloads():
    """The CPU-baseline legs of the block and decode workloads on a tiny model (CPU tensors,
    no GPU): they run the oracle's block forward, prefill and recurrent steps and report
    tokens/s with the sample they timed."""
    import torch

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from cfgs import make_lm  # noqa: E402
    from hdcmamba_amd import HdcMamba9v3Block

    torch.manual_seed(0)
    blk = HdcMamba9v3Block(64, 16, 4, 8).to(torch.bfloat16)
    x = torch.randn(2, 24, 64).to(torch.bfloat16)
    cfg = {"d_model": 64, "d_state": 16, "num_heads": 4, "chunk": 8}
    r = bench.cpu_baseline_block(blk, x, cfg, warmup=1, runs=2)
    assert r["value"] > 0 and r["kind"] == "port" and len(r["run_seconds"]) == 2 and "B=2, L=24" in r["sample"]

    lm = make_lm("lm_c3", n_layers=2).to(torch.bfloat16)
    ids = torch.randint(0, 50304, (2, 16 + 4))
    cfg = {"d_model": 768, "d_state": 64, "num_heads": 12, "chunk": 64, "n_layers": 2}
    r = bench.cpu_baseline_decode(lm, ids, cfg, L=16, prefill_layers=1, steps=16)
    assert r["value"] > 0 and r["prefill_extrapolated"] and r["prefill_tokens_per_s"] > 0
    assert "3 timed decode steps" in r["sample"]  # capped by the ids past the prefill
