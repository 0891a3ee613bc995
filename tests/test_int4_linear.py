"""CPU tests of the Int4Linear helpers (kernels/int4_linear.py; reference
kernels/int4_linear.py:19-269): the group-size rules of from_float and
convert_model_to_int4, the constructor's checks and buffers, and
estimate_int4_memory against an independent count.  Quantisation and the
forward run on the GPU (tests/test_gpu_int4_linear.py)."""
import pytest
import torch
import torch.nn as nn

from hydranet_amd.kernels import int4_linear as il


@pytest.mark.parametrize("fin,g,want", [(4096, 128, 128), (192, 128, 64), (96, 128, 32),
                                        (256, 256, 256), (320, 256, 64)])
def test_from_float_group_rule(fin, g, want):
    # the requested group, else 64, else 32 (reference kernels/int4_linear.py:127-134)
    assert il._group_for_from_float(fin, g) == want


def test_from_float_group_rule_rejects():
    with pytest.raises(ValueError):
        il._group_for_from_float(48, 128)


@pytest.mark.parametrize("fin,g,want", [(4096, 128, 128), (192, 128, 64), (96, 128, 32),
                                        (48, 128, None), (320, 256, 64), (96, 96, 96),
                                        (144, 96, None)])
def test_convert_group_rule(fin, g, want):
    # halve from the requested group while it does not divide; none below 32
    # (reference kernels/int4_linear.py:205-214)
    assert il._group_for_convert(fin, g) == want


def test_constructor_checks_and_buffers():
    with pytest.raises(AssertionError):
        il.Int4Linear(33, 8, group_size=32)     # odd in_features
    with pytest.raises(AssertionError):
        il.Int4Linear(192, 8, group_size=128)   # group does not divide
    m = il.Int4Linear(256, 40, bias=True, group_size=64)
    assert m.weight_packed.shape == (40, 128) and m.weight_packed.dtype == torch.uint8
    assert m.weight_scale.shape == (40, 4) and m.weight_scale.dtype == torch.float16
    assert m.bias.dtype == torch.float16 and m.bias.shape == (40,)
    assert il.Int4Linear(256, 40, bias=False).bias is None
    # buffers travel with state_dict under the reference's names
    assert {"weight_packed", "weight_scale", "bias"} <= set(m.state_dict())


def test_estimate_int4_memory_counts():
    torch.manual_seed(0)
    model = nn.Sequential(nn.Linear(256, 96, bias=True), nn.LayerNorm(96),
                          nn.Linear(96, 200, bias=False))
    est = il.estimate_int4_memory(model, group_size=128)
    # independent count: per parameter, fp16 bytes; 2-D: half a byte per weight
    # plus one fp16 scale per row per started group of 128 columns
    fp16 = sum(p.numel() for p in model.parameters()) * 2
    w1 = 96 * 256 // 2 + 96 * 2 * 2          # 256 columns -> 2 groups
    w2 = 200 * 96 // 2 + 200 * 1 * 2         # 96 columns -> 1 (partial) group
    small = (96 + 96 + 96) * 2               # bias of layer 0, LayerNorm weight + bias
    assert est["fp16_mb"] == pytest.approx(fp16 / 1e6)
    assert est["int4_mb"] == pytest.approx((w1 + w2 + small) / 1e6)
    assert est["savings_mb"] == pytest.approx((fp16 - w1 - w2 - small) / 1e6)
    assert set(est) == {"fp16_mb", "int4_mb", "savings_mb"}
    # reference test_int4_loader.py:404 bound on the fp16/INT4 ratio of an expert-sized layer
    big = il.estimate_int4_memory(nn.Linear(4096, 14336, bias=False))
    assert 2.5 < big["fp16_mb"] / big["int4_mb"] < 4.5
