"""The forward grouped GEMM's inline-assembly weight loads, checked in the
compiled gfx950 code (CPU; needs hipcc): no read or write of a load's
destination registers before a wait covers it (tests/isa_hazards.py), and a
planted hazard is found."""
import shutil
import subprocess
from pathlib import Path

import pytest

from tests import isa_hazards as H

ROOT = Path(__file__).resolve().parents[1]
CSRC = ROOT / "agent-factory-3_amd" / "csrc"
HIPCC = shutil.which("hipcc") or ("/opt/rocm/bin/hipcc" if Path("/opt/rocm/bin/hipcc").exists() else None)
# the forward kernel with two weight-register buffers and with three (k-steps a
# multiple of 3), the latter with 64-bit addresses and with a scalar base
SYMBOLS = ["_ZN12_GLOBAL__N_116gemm7_fwd_kernelILi0ELi2ELb0EEEvNS_6ParamsE",
           "_ZN12_GLOBAL__N_116gemm7_fwd_kernelILi0ELi3ELb0EEEvNS_6ParamsE",
           "_ZN12_GLOBAL__N_116gemm7_fwd_kernelILi0ELi3ELb1EEEvNS_6ParamsE"]


@pytest.fixture(scope="module")
def moe_gemm_asm(tmp_path_factory):
    if HIPCC is None:
        pytest.skip("hipcc not available")
    from agent_factory_3_amd import build
    out = tmp_path_factory.mktemp("isa") / "moe_gemm.s"
    flags = [f for f in build.HIPCC_FLAGS if f not in ("-fPIC",)]
    subprocess.run([HIPCC, *flags, "-I", str(CSRC), "--cuda-device-only", "-S", str(CSRC / "moe_gemm.hip"),
                    "-o", str(out)], check=True, capture_output=True)
    return out.read_text()


@pytest.mark.timeout(600)
@pytest.mark.parametrize("symbol", SYMBOLS)
def test_forward_weight_loads_have_no_register_hazard(moe_gemm_asm, symbol):
    n, bad = H.violations(H.function_body(moe_gemm_asm, symbol))
    assert n >= 4, "expected the k-loop's inline-assembly weight loads"
    assert not bad, bad[:5]


def test_checker_finds_planted_hazards():
    base = ["s_waitcnt vmcnt(0)", ";;#ASMSTART", "global_load_dwordx4 v[8:11], v[2:3], off", ";;#ASMEND"]
    ok = base + ["global_load_lds_dwordx4 v[4:5], off", "s_waitcnt vmcnt(1)", "v_mov_b32_e32 v0, v8", "s_endpgm"]
    assert H.violations(ok) == (1, [])
    read = base + ["global_load_lds_dwordx4 v[4:5], off", "s_waitcnt vmcnt(2)", "v_mov_b32_e32 v0, v8", "s_endpgm"]
    assert len(H.violations(read)[1]) == 1          # vmcnt(2) with one newer op does not cover the load
    write = base + ["scratch_load_dword v9, off, off", "s_waitcnt vmcnt(0)", "s_endpgm"]
    assert len(H.violations(write)[1]) == 1         # a reload into a pending destination register
    branch = base + ["s_cbranch_scc1 .LBB0_1", "s_waitcnt vmcnt(0)", ".LBB0_1:", "v_add_u32_e32 v10, v1, v1",
                     "s_endpgm"]
    assert len(H.violations(branch)[1]) == 1        # the path around the wait
