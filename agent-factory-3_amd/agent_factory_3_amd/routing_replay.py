"""Routing replay: feed rollout-time expert choices to the training forward.

Same switch as the reference's ``routing_replay.py:257`` (``enable_routing_replay``):
after it, ``model(input_ids, routing_indices=[B, S, L, K])`` makes every MoE
layer use the given experts (``routing_replay`` in the MLP) instead of top-k.

Built differently from the reference, which re-implements the bodies of
``GptOssModel.forward`` and ``GptOssDecoderLayer.forward``: here the
``routing_indices`` keyword rides through transformers' own ``**kwargs``
plumbing (``GptOssModel.forward`` hands its kwargs to every decoder layer)
and a thin wrapper around the decoder layer slices layer ``l``'s ``[B, S, K]``
indices and exposes them to the MLP for the duration of that layer call.
Activation checkpointing re-runs the wrapper with the same saved kwargs, so
the recomputed forward replays the same experts.
"""
from __future__ import annotations

import logging

logger = logging.getLogger(__name__)

_ATTR = "_af3_replay_router_indices"


def current_router_indices(mlp):
    """Indices the enclosing decoder layer set for this MLP (None outside replay)."""
    return getattr(mlp, _ATTR, None)


def enable_routing_replay(model=None):
    """Patch GptOssDecoderLayer so ``routing_indices`` [B, S, L, K] reach the MLP.

    Call after the model is loaded with the MXFP4 quantizer (whose
    ``mlp_forward`` consumes the indices).  Idempotent.
    """
    from transformers.models.gpt_oss.modeling_gpt_oss import GptOssDecoderLayer

    if getattr(GptOssDecoderLayer, "_af3_routing_replay", False):
        logger.info("routing replay already enabled")
        return
    orig_forward = GptOssDecoderLayer.forward

    def forward(self, hidden_states, *args, routing_indices=None, router_indices=None, **kwargs):
        if router_indices is None and routing_indices is not None:
            if routing_indices.dim() != 4:
                raise ValueError(f"routing_indices must be [B, S, L, K], got {tuple(routing_indices.shape)}")
            router_indices = routing_indices[:, :, self.self_attn.layer_idx, :]
        prev = getattr(self.mlp, _ATTR, None)
        setattr(self.mlp, _ATTR, router_indices)
        try:
            return orig_forward(self, hidden_states, *args, **kwargs)
        finally:
            setattr(self.mlp, _ATTR, prev)

    GptOssDecoderLayer.forward = forward
    GptOssDecoderLayer._af3_routing_replay = True
    logger.info("routing replay enabled for GptOssDecoderLayer")
