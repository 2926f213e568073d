"""bench.py's per-kernel roofline tables (host arithmetic only): the algorithmic work
per launch each kernel is credited with, and the fractions derived from it."""
import math

import bench
from ditserve_amd.sd35 import SD35_MEDIUM
from ditserve_amd.wan import WAN21_T2V_1_3B


def test_wan_kernel_work_per_launch():
    """Wan2.1 480p CFG pair: 2 x 32760 rows, D = 1536, F = 8960, 512 text keys per segment."""
    spec = bench._wan_kernel_spec(WAN21_T2V_1_3B, [32760, 32760], 512)
    M, D, F = 65520, 1536, 8960
    assert spec["attn_self"][1] == 4.0 * 2 * 32760 ** 2 * D == 1.31876978688e13
    assert spec["attn_cross"][1] == 4.0 * M * 512 * D
    assert spec["gemm_qkv"][1] == 2.0 * M * 3 * D * D
    assert spec["gemm_ffn_up_gelu"][1] == spec["gemm_ffn_down_gate"][1] == 2.0 * M * D * F
    assert spec["adaln"][1] == 4.0 * M * D and spec["qk_norm_rope"][1] == 8.0 * M * D
    assert {v[0] for k, v in spec.items() if k.startswith(("gemm", "attn"))} == {"mfma"}
    assert {spec[k][0] for k in ("adaln", "qk_norm_rope", "transpose_v")} == {"hbm"}


def test_sd35_kernel_work_per_launch():
    """SD3.5 packed segments: joint attention over (image + text) rows per segment,
    dual attention over image rows only, pairs credited with both products."""
    img, txt = [4096, 4096, 1024], [333, 333, 333]
    spec = bench._sd35_kernel_spec(SD35_MEDIUM, img, txt)
    D, F = 1536, 6144
    assert spec["attn_joint"][1] == 4.0 * (2 * 4429 ** 2 + 1357 ** 2) * D
    assert spec["attn_dual_core"][1] == 4.0 * (2 * 4096 ** 2 + 1024 ** 2) * D
    assert spec["gemm_out_pair"][1] == 2.0 * (9216 + 999) * D * D
    assert spec["gemm_ffn_down_pair"][1] == 2.0 * (9216 + 999) * D * F


def test_kernel_table_fractions():
    spec = {"k_mfma": ("mfma", 2.5e12, "one PFLOP-second at peak per ms"), "k_hbm": ("hbm", 8e9, "8 GB"),
            "missing": ("mfma", 1.0, "not timed")}
    t = bench._kernel_table({"k_mfma": {"avg_ms": 1.0, "count": 3}, "k_hbm": {"avg_ms": 2.0, "count": 5}}, spec)
    assert set(t) == {"k_mfma", "k_hbm"}
    assert math.isclose(t["k_mfma"]["achieved"], 2500.0) and math.isclose(t["k_mfma"]["frac"], 1.0)
    assert t["k_mfma"]["unit"] == "TFLOP/s" and t["k_mfma"]["flops_per_launch"] == 2.5e12
    assert math.isclose(t["k_hbm"]["achieved"], 4.0) and math.isclose(t["k_hbm"]["frac"], 0.5)
    assert t["k_hbm"]["unit"] == "TB/s" and t["k_hbm"]["launches"] == 5 and t["k_hbm"]["bytes_per_launch"] == 8e9
