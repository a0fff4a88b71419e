"""ctypes binding of ``libaf3_mi355x.so`` (the C ABI in ``include/af3_mi355x.h``).

The library is loaded after ``import torch`` so that its HIP symbols resolve to
the ``libamdhip64.so.7`` torch already mapped (one HIP runtime per process).
There is no fallback: if the library is missing, every call raises.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import torch  # noqa: F401  (must precede the library load: shared HIP runtime)

_LIB_PATH = Path(__file__).resolve().parent / "libaf3_mi355x.so"
ABI_VERSION = 2

_p = C.c_void_p
_i32 = C.c_int
_i64 = C.c_int64
_f32 = C.c_float
_sz = C.c_size_t

# name -> (restype, argtypes)
_SIGNATURES = {
    "af3_abi_version": (_i32, []),
    "af3_last_error": (C.c_char_p, []),
    "af3_mxfp4_to_bf16": (_i32, [_p, _p, _p, _i64, _p]),
    "af3_swiglu_fwd": (_i32, [_p, _i64, _p, _i64, _p, _p, _i64, _i64, _i64, _f32, _f32, _p]),
    "af3_swiglu_bwd": (_i32, [_p, _i64, _p, _p, _i64, _p, _i64, _i64, _i64, _f32, _f32, _p]),
    "af3_swiglu_bwd_raw": (_i32, [_p, _i64, _p, _i64, _p, _i64, _i64, _i64, _f32, _f32, _p]),
    "af3_routing_workspace_bytes": (_sz, [_i64, _i32, _i32]),
    "af3_routing_replay": (_i32, [_p, _i64, _p, _i64, _i32, _i32, _p, _p, _p, _p, _p, _p, _sz, _p]),
    "af3_routing_topk": (_i32, [_p, _i64, _i64, _i32, _i32, _p, _p, _p, _p, _p, _p, _sz, _p]),
    "af3_routing_scratch_bytes": (_sz, []),
    "af3_routing_replay_noalloc": (_i32, [_p, _i64, _p, _i64, _i32, _i32, _p, _p, _p, _p, _p, _p]),
    "af3_expt_data": (_i32, [_p, _i32, _p, _i32, _i32, _p, _p, _p]),
    "af3_router_logits": (_i32, [_p, _i64, _p, _i64, _p, _i64, _i32, _i32, _p, _i64, _p]),
    "af3_tile_order": (_i32, [_p, _i32, _i32, _p, _i32, _p, _p]),
    "af3_mxfp4_tile_fwd": (_i32, [_p, _i64, _i32, _i32, _p, _p]),
    "af3_mxfp4_tile_dx_scales": (_i32, [_p, _i64, _i32, _i32, _p, _p]),
    "af3_moe_gemm": (_i32, [_p, _i64, _p, _i32, _p, _p, _i32, _p, _p, _i32, _p, _i64, _p, _i32,
                            _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _p, _i64, _p]),
    "af3_moe_gemm_swiglu": (_i32, [_p, _i64, _p, _i32, _p, _p, _i32, _p, _p, _i32, _p, _i64, _p, _i32,
                                   _p, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _p, _i64, _i32, _p, _i64,
                                   _f32, _f32, _p]),
    "af3_moe_gemm_rowscale": (_i32, [_p, _i64, _p, _i32, _p, _p, _i32, _p, _p, _i32, _p, _p, _p, _i32, _i32,
                                     _i32, _i32, _i32, _i32, _p, _i64, _p, _p]),
    "af3_moe_gemm_f8": (_i32, [_p, _i64, _p, _i32, _p, _p, _i32, _p, _p, _i32, _p, _p, _p, _i32, _i32, _i32, _i32,
                               _i32, _i32, _p, _i64, _p, _p]),
    "af3_moe_combine": (_i32, [_p, _i64, _p, _i64, _i32, _i32, _p, _i64, _p]),
    "af3_mxfp4_to_fp8_e5m2": (_i32, [_p, _p, _p, _i64, _p]),
    "af3_mxfp4_to_fp8_e5m2_colmajor": (_i32, [_p, _p, _p, _i32, _i32, _i32, _p]),
    "af3_quantize_per_token_e4m3": (_i32, [_p, _i64, _i64, _i32, _p, _i64, _p, _p, _i64, _p]),
    "af3_lm_head_workspace_bytes": (_sz, [_i32, _i32]),
    "af3_lm_head_logprobs": (_i32, [_p, _i64, _p, _i64, _i32, _i32, _i32, _p, _f32, _p, _p, _p, _p, _p, _sz, _p]),
    "af3_lm_head_dlogits": (_i32, [_p, _i64, _p, _i64, _i32, _i32, _i32, _p, _f32, _p, _p, _p, _i64, _f32, _p, _p,
                                   _i64, _p]),
    "af3_lm_head_dlogits_range": (_i32, [_p, _i64, _p, _i64, _i32, _i32, _i32, _i32, _p, _f32, _p, _p, _p, _i64, _f32,
                                         _p, _p, _i64, _p]),
    "af3_lm_head_chunk_stats": (_i32, [_p, _i64, _i32, _i32, _i32, _p, _f32, _p, _p, _p]),
    "af3_lm_head_reduce": (_i32, [_p, _i32, _i32, _p, _p, _i32, _p, _p, _p, _p, _p]),
    "af3_lm_head_dz_chunk": (_i32, [_p, _i64, _i32, _i32, _i32, _p, _f32, _p, _p, _p, _i64, _f32, _p, _p, _i64, _p]),
    "af3_gamma_grad": (_i32, [_p, _i64, _p, _i64, _i32, _p, _i64, _p, _i32, _p, _i32, _p, _i32, _p, _i64, _p, _p]),
    "af3_mxfp4_lora_merge": (_i32, [_p, _p, _p, _p, _f32, _p, _i32, _i32, _i32, _i32, _i32, _p]),
    "af3_lora_rows": (_i32, [_p, _i64, _p, _i32, _p, _i32, _f32, _p, _p, _i32, _i32, _i32, _i32,
                             _p, _i64, _p]),
    "af3_lora_wgrad_workspace_bytes": (_sz, [_i32, _i32, _i32]),
    "af3_lora_wgrad": (_i32, [_p, _i64, _p, _i32, _p, _p, _i64, _p, _i32, _f32, _p, _i32, _i32,
                              _i32, _p, _p, _i32, _i32, _p, _sz, _p, _p]),
    "af3_lora_u_wgrad_workspace_bytes": (_sz, [_i32, _i64, _i32, _i32]),
    "af3_lora_u_wgrad": (_i32, [_p, _i64, _p, _i32, _p, _p, _p, _f32, _p, _i32, _i64, _i32, _i32,
                                _p, _p, _i32, _i32, _p, _sz, _p, _p, _p]),
}

_lib = None


def lib_path() -> Path:
    return _LIB_PATH


def load() -> C.CDLL:
    """Load (once) and return the library; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not _LIB_PATH.exists():
        raise ImportError(
            f"{_LIB_PATH} is missing: build it with `python -m agent_factory_3_amd.build` "
            "(the MI355X path has no CPU fallback)")
    lib = C.CDLL(str(_LIB_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.af3_abi_version()
    if ver != ABI_VERSION:
        raise ImportError(f"{_LIB_PATH}: ABI version {ver}, expected {ABI_VERSION}")
    _lib = lib
    return lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def call(name: str, *args) -> None:
    """Call an entry point; raise RuntimeError on a non-zero status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.af3_last_error().decode(errors="replace")
        kind = "argument error" if rc < 0 else f"HIP error {rc}"
        raise RuntimeError(f"{name}: {kind}: {msg}")


EUNSUPPORTED = -2
W_FWD_TILED = 0x10000  # tile_cfg flag: the weights are the af3_mxfp4_tile_fwd copy
X_OFFSETS_32 = 0x20000  # tile_cfg flag: every row of x the call reads lies within 4 GiB of x
S_DX_TILED = 0x40000  # tile_cfg flag: the scales are the af3_mxfp4_tile_dx_scales copy


def try_call(name: str, *args) -> bool:
    """Call an entry point that may decline a configuration: False when it
    returns AF3_EUNSUPPORTED (nothing was launched), True on success; raise
    RuntimeError on any other error."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc == EUNSUPPORTED:
        return False
    if rc != 0:
        msg = lib.af3_last_error().decode(errors="replace")
        kind = "argument error" if rc < 0 else f"HIP error {rc}"
        raise RuntimeError(f"{name}: {kind}: {msg}")
    return True


def workspace_bytes(n_tokens: int, n_expts_tot: int, n_expts_act: int) -> int:
    return int(load().af3_routing_workspace_bytes(n_tokens, n_expts_tot, n_expts_act))


def ptr(t) -> int | None:
    """Device address of a tensor (None for None)."""
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
