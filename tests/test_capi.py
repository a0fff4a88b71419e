"""The C-ABI library loads and exports every symbol include/af3_mi355x.h declares (CPU)."""
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "af3_mi355x.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(af3_\w+)\s*\(", text, re.M)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "af3_moe_gemm" in syms and "af3_mxfp4_to_bf16" in syms and len(syms) >= 14


def test_library_exports_every_declared_symbol():
    from agent_factory_3_amd import _capi
    path = _capi.lib_path()
    if not path.exists():
        pytest.skip("library not built (run __graft_entry__.build())")
    out = subprocess.run(["nm", "-D", "--defined-only", str(path)], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\sT\s(af3_\w+)", out))
    missing = [s for s in declared_symbols() if s not in exported]
    assert not missing, missing
    # the Python binding knows every declared symbol with a signature
    assert sorted(declared_symbols()) == sorted(_capi.exported_symbols())


def test_library_loads_and_reports_abi():
    from agent_factory_3_amd import _capi
    if not _capi.lib_path().exists():
        pytest.skip("library not built")
    lib = _capi.load()
    assert lib.af3_abi_version() == _capi.ABI_VERSION
    # argument errors come back as a Python exception with the library's message, no GPU needed
    with pytest.raises(RuntimeError, match="n_groups"):
        _capi.call("af3_mxfp4_to_bf16", None, None, None, -1, None)
    assert _capi.workspace_bytes(16, 4, 2) > 0


def test_noalloc_routing_rejects_shapes_beyond_its_scratch():
    """af3_routing_replay_noalloc checks the shape against its built-in scratch
    array before touching the device (no GPU needed for the error path)."""
    from agent_factory_3_amd import _capi
    if not _capi.lib_path().exists():
        pytest.skip("library not built")
    lib = _capi.load()
    T, E, K = 1 << 20, 128, 4
    assert _capi.workspace_bytes(T, E, K) > int(lib.af3_routing_scratch_bytes()) == 4 << 20
    with pytest.raises(RuntimeError, match="scratch"):
        _capi.call("af3_routing_replay_noalloc", 1, E, 1, T, E, K, 1, 1, 1, 1, 1, None)


def test_product_path_has_no_oracle_dependency():
    pkg = ROOT / "agent-factory-3_amd" / "agent_factory_3_amd"
    for f in pkg.glob("*.py"):
        assert "oracle" not in re.findall(r"^\s*(?:from|import)\s+(\w+)", f.read_text(), re.M), f.name
