"""Keep bf16 NaN bit patterns intact in torch._foreach_copy_ (FSDP2 side effect).

The MXFP4 bytes live in bf16 "container" Parameters so FSDP2 can shard them;
some of those 16-bit patterns are NaNs.  A fused same-dtype bf16 foreach copy
may canonicalise NaN payloads, which would corrupt the packed weights (the
reference works around the same hazard in ``fsdp2_fix.py:16-28``).  Importing
this module routes every foreach copy that involves a bf16->bf16 pair through
per-tensor ``copy_``, which moves bits unchanged; other copies are untouched.
"""
import torch

_original_foreach_copy = torch._foreach_copy_


def _bit_preserving_foreach_copy_(dsts, srcs, *args, **kwargs):
    pairs = list(zip(dsts, srcs))
    if any(d.dtype == torch.bfloat16 and s.dtype == torch.bfloat16 for d, s in pairs):
        for d, s in pairs:
            d.copy_(s)
        return None
    return _original_foreach_copy(dsts, srcs, *args, **kwargs)


if not getattr(torch._foreach_copy_, "_af3_bit_preserving", False):
    _bit_preserving_foreach_copy_._af3_bit_preserving = True
    torch._foreach_copy_ = _bit_preserving_foreach_copy_
