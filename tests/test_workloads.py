"""Synthetic configuration generators (CPU)."""
import numpy as np
import torch

from agent_factory_3_amd import workloads


def test_zipf_counts_sum_and_shape():
    c = workloads.zipf_counts(65536, 120, 1.1)
    assert c.sum() == 65536 and c[0] == c.max() and c.max() <= 16384 and (np.diff(c) <= 0).all()


def test_zipf_routing_distinct_and_idle():
    g = torch.Generator().manual_seed(0)
    ids = workloads.zipf_routing(g, 1024, 128, 4, n_idle=8)
    assert ids.shape == (1024, 4)
    s = torch.sort(ids, 1).values
    assert (s[:, 1:] != s[:, :-1]).all()            # distinct per token
    hist = torch.bincount(ids.flatten().long(), minlength=128)
    assert (hist == 0).sum() == 8 and int(hist.sum()) == 4096


def test_layer_inputs_small():
    inp = workloads.layer(4, T=64, E=8, H=64, I=64, lora_r=8, zipf=False)
    assert inp.gu_blocks.shape == (8, 128, 2, 16) and inp.dn_blocks.shape == (8, 64, 2, 16)
    assert inp.lora["Agu"].shape == (8, 8, 64) and inp.lora["Bdn"].shape == (8, 64, 8)
    assert int(inp.gu_scales.min()) >= 118 and int(inp.gu_scales.max()) <= 130


def test_cfg4_flops_closed_form():
    """cfg4 work: the forward's 2 R H 2I + 2 R I H and the same again for
    the input gradients (6.523 TFLOP in all), and 6 R r (K + N) per LoRA
    projection (0.1812 TFLOP), R = 65,536 rows, H = I = 2880, r = 32."""
    f = workloads.layer_flops(16384, 4, lora_r=32)
    assert abs(f["base"] / 1e12 - 6.523) < 1e-3 and abs(f["lora"] / 1e12 - 0.1812) < 1e-3
