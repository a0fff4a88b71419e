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
