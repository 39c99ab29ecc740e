"""The recorded GEMM solution file: versions it was recorded under and the signatures the
workloads' projections use (CPU only; the solutions themselves run in the GPU bench)."""
import csv

from hdcmamba_amd.gemm_tuning import TUNED_FILE, use_tuned_gemms


def _rows():
    with open(TUNED_FILE) as f:
        return list(csv.reader(f))


def test_tuned_file_validators():
    val = {r[1]: r[2] for r in _rows() if r[0] == "Validator"}
    assert set(val) >= {"PT_VERSION", "HIP_VERSION", "HIPBLASLT_VERSION", "ROCBLAS_VERSION", "GCN_ARCH_NAME"}
    assert val["GCN_ARCH_NAME"].startswith("gfx950")


def test_tuned_file_covers_the_projections():
    sigs = {r[1] for r in _rows() if r[0] != "Validator"}
    T = 32768
    # d_model 1024, d_state 128 at B*L = 32768: in_proj (with bias), out_proj, tied LM head
    assert f"tn_4480_{T}_1024_ld_1024_1024_4480" in sigs
    assert f"tn_1024_{T}_1152_ld_1152_1152_1024" in sigs
    assert f"tn_50304_{T}_1024_ld_1024_1024_50304" in sigs
    # d_model 2048 prefill (B*L = 131072) and B=16 decode
    assert "tn_8576_131072_2048_ld_2048_2048_8576" in sigs
    assert "tn_8576_16_2048_ld_2048_2048_8576" in sigs
    for r in _rows():
        if r[0] != "Validator":
            assert r[0].endswith("_BFloat16_TN") and float(r[3]) > 0


def test_missing_file_loads_nothing(tmp_path):
    assert use_tuned_gemms(tmp_path / "absent.csv") == 0
