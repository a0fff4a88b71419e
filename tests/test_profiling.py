"""rocprofv3 summary helpers (CPU) and the committed traffic profile that bench.py reads."""
import csv
from pathlib import Path

from agent_factory_3_amd import profiling

ROOT = Path(__file__).resolve().parents[1]


def test_short_name_keeps_template_arguments():
    n = "void (anonymous namespace)::gemm4_fwd_kernel<2, 4, 0>((anonymous namespace)::Params)"
    assert profiling.short_name(n) == "gemm4_fwd_kernel<2, 4, 0>"
    assert profiling.short_name("(anonymous namespace)::combine_kernel(unsigned short const*, long)") == \
        "combine_kernel"


def test_ktrace_groups_by_kernel_and_grid(tmp_path):
    p = tmp_path / "t.csv"
    with open(p, "w", newline="") as f:
        w = csv.DictWriter(f, ["Kernel_Name", "Grid_Size_X", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        for s, e, g in ((0, 2000, 64), (10000, 14000, 64), (20000, 21000, 128)):
            w.writerow({"Kernel_Name": "k(int)", "Grid_Size_X": g, "Start_Timestamp": s, "End_Timestamp": e})
    table = profiling.ktrace(str(p))
    assert "| `k` | 64 | 2 | 3.00 | 2.00 | 6.0 |" in table
    assert "| `k` | 128 | 1 | 1.00 | 1.00 | 1.0 |" in table


def test_committed_traffic_profile_parses():
    tj = profiling.read_traffic(str(ROOT / "profiles" / "traffic_cfg4.md"))
    assert tj is not None
    assert 0.5 < tj["fetch_scale"] < 8 and 0.5 < tj["write_scale"] < 8
    names = [k.split("|")[0] for k in tj["kernels"]]
    for kernel in profiling.GEMM_KERNELS.values():   # the kernels bench.py reads traffic for
        assert any(kernel in n for n in names), kernel


def test_ktrace_window_and_entry_point_average(tmp_path):
    kt, mk = tmp_path / "kt.csv", tmp_path / "mk.csv"
    with open(kt, "w", newline="") as f:
        w = csv.DictWriter(f, ["Kernel_Name", "Grid_Size_X", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        # one dispatch before the range (slow, cold), two inside: grids of both GEMM shapes
        for s, e, g in ((0, 9000, 64), (10000, 12000, 64), (20000, 21000, 32), (30000, 39000, 64)):
            w.writerow({"Kernel_Name": "void gemm7_fwd_kernel<0>(Params)", "Grid_Size_X": g,
                        "Start_Timestamp": s, "End_Timestamp": e})
    with open(mk, "w", newline="") as f:
        w = csv.DictWriter(f, ["Domain", "Function", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        w.writerow({"Domain": "MARKER_CORE_API", "Function": "other", "Start_Timestamp": 0, "End_Timestamp": 50000})
        w.writerow({"Domain": "MARKER_CORE_API", "Function": "bench_timed", "Start_Timestamp": 9500,
                    "End_Timestamp": 25000})
    win = profiling.marker_window(str(mk), "bench_timed")
    assert win == (9500, 25000)
    table = profiling.ktrace(str(kt), win)
    assert "| `gemm7_fwd_kernel<0>` | 64 | 1 | 2.00 |" in table
    assert "| moe_gemm_fwd | `gemm7_fwd_kernel` | 2 | 1.50 |" in table
    assert "| moe_gemm_fwd | `gemm7_fwd_kernel` | 4 | 5.25 |" in profiling.ktrace(str(kt))


def test_mfma_busy_share_normalisation(tmp_path):
    """GRBM_GUI_ACTIVE comes summed over the XCDs; the MFMA-busy counter over
    every SIMD: a kernel whose MFMA pipes are busy half of the active cycles
    on every SIMD reads 0.5."""
    ag, pc = tmp_path / "agent.csv", tmp_path / "pmc.csv"
    with open(ag, "w", newline="") as f:
        w = csv.DictWriter(f, ["Agent_Type", "Num_Xcc", "Cu_Count", "Simd_Per_Cu"])
        w.writeheader()
        w.writerow({"Agent_Type": "CPU", "Num_Xcc": 1, "Cu_Count": 16, "Simd_Per_Cu": 0})
        w.writerow({"Agent_Type": "GPU", "Num_Xcc": 8, "Cu_Count": 256, "Simd_Per_Cu": 4})
    active = 1000.0  # cycles per XCD
    with open(pc, "w", newline="") as f:
        w = csv.DictWriter(f, ["Dispatch_Id", "Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for name, v in (("GRBM_GUI_ACTIVE", 8 * active), ("SQ_VALU_MFMA_BUSY_CYCLES", 0.5 * active * 256 * 4),
                        ("SQ_BUSY_CU_CYCLES", 0.9 * active * 256)):
            w.writerow({"Dispatch_Id": 1, "Kernel_Name": "void gemm4_fwd_kernel<2, 4, 0>(Params)",
                        "Grid_Size": 512, "Counter_Name": name, "Counter_Value": v})
    table = profiling.mfma(str(pc), str(ag))
    assert "GPU: 8 XCDs, 256 CUs, 4 SIMDs per CU." in table
    assert "| `gemm4_fwd_kernel<2, 4, 0>` | 512 | 1000 | 0.500 | 0.900 |" in table
