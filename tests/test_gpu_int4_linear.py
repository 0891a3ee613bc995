"""GPU tests of Int4Linear for non-expert weights (kernels/int4_linear.py;
reference kernels/int4_linear.py:19-269 and its use in test_glm4_generate.py:
262-280): convert_model_to_int4 over a module tree whose layers hit every
group-size case, bit-exact against the oracle's restatement of the
quantiser; the decoder harness and the GLM layer with INT4 attention / shared
expert against the same modules holding the dequantised weights in fp16; the
name-compatibility entry points ExpertMLPTriton and the package-level
expert_mlp_int4.

Bars: quantised bytes and scales bit-exact; fp16 outputs |got - ref| <=
1e-2 + 2e-3 |ref| (the path's tolerance); decoder logits 3e-2 + 1e-2 |ref|
(two residual layers and the LM head compound it)."""
import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
from oracle import torch_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _close(got, ref, atol=1e-2, rtol=2e-3):
    got, ref = got.float().cpu(), ref.float().cpu()
    err = (got - ref).abs()
    assert torch.isfinite(got).all()
    assert bool((err <= atol + rtol * ref.abs()).all()), f"max err {err.max().item():.3g}"


def _tree():
    torch.manual_seed(7)
    m = nn.Module()
    m.attn = nn.Module()
    m.attn.q_proj = nn.Linear(256, 128, bias=False)   # group 128
    m.attn.o_proj = nn.Linear(192, 256, bias=True)    # 192 -> group 64
    m.mlp = nn.Sequential(nn.Linear(96, 64, bias=True),  # 96 -> group 32
                          nn.Linear(48, 32),             # 48 -> no group >= 32: kept
                          nn.Linear(33, 32))             # odd: kept
    m.lm_head = nn.Linear(256, 64, bias=False)        # skipped by name
    return m.half()


def test_convert_model_to_int4_groups_bytes_and_forward():
    from hydranet_amd.kernels import Int4Linear, convert_model_to_int4, estimate_int4_memory
    src = _tree()
    fp16 = {n: (mod.weight.data.clone(), None if mod.bias is None else mod.bias.data.clone())
            for n, mod in src.named_modules() if isinstance(mod, nn.Linear)}
    est = estimate_int4_memory(src)
    m = convert_model_to_int4(src, skip_layers=["lm_head"], group_size=128, device=DEV)
    rep = m._int4_report
    assert sorted(rep.converted) == ["attn.o_proj", "attn.q_proj", "mlp.0"]
    assert set(rep.skipped) == {"mlp.1", "mlp.2", "lm_head"}
    assert isinstance(m.mlp[1], nn.Linear) and isinstance(m.lm_head, nn.Linear)
    groups = {"attn.q_proj": 128, "attn.o_proj": 64, "mlp.0": 32}
    for name, g in groups.items():
        layer = m.get_submodule(name)
        assert isinstance(layer, Int4Linear) and layer.group_size == g
        w, b = fp16[name]
        p_ref, s_ref = oracle.quantize(w.numpy(), g, mode=1)
        np.testing.assert_array_equal(layer.weight_packed.cpu().numpy(), p_ref, err_msg=name)
        np.testing.assert_array_equal(layer.weight_scale.cpu().numpy().view(np.uint16),
                                      s_ref.view(np.uint16), err_msg=name)
        x = (torch.randn(3, 5, w.shape[1], generator=torch.Generator().manual_seed(g)) * 1.0
             ).half()
        y = layer(x.to(DEV))
        assert y.shape == (3, 5, w.shape[0])
        ref = torch.from_numpy(oracle.int4_linear(x.view(15, -1).numpy(), p_ref, s_ref, g)
                               .astype(np.float32))
        if b is not None:
            ref = (ref.half() + b).float()
        _close(y.view(15, -1), ref)
    assert est["int4_mb"] < est["fp16_mb"]


def test_from_float_group_fallback():
    from hydranet_amd.kernels import Int4Linear
    lin = nn.Linear(96, 40, bias=True).half()
    q = Int4Linear.from_float(lin, group_size=128, device=torch.device(DEV))
    assert q.group_size == 32 and q.weight_scale.shape == (40, 3)
    p_ref, s_ref = oracle.quantize(lin.weight.data.numpy(), 32, mode=1)
    np.testing.assert_array_equal(q.weight_packed.cpu().numpy(), p_ref)
    assert torch.equal(q.bias.detach().cpu(), lin.bias.data)


def _load_dequantised(int4_model, ref):
    """Give every fp16 nn.Linear of ref the oracle's dequantised weights of the
    same-named Int4Linear of int4_model (the reference's torch path for them)."""
    from hydranet_amd.kernels import Int4Linear
    n = 0
    for name, mod in int4_model.named_modules():
        if isinstance(mod, Int4Linear):
            lin = ref.get_submodule(name)
            assert isinstance(lin, nn.Linear)
            w = oracle.dequant(mod.weight_packed.cpu().numpy(), mod.weight_scale.cpu().numpy(),
                               mod.group_size)
            lin.weight.data.copy_(torch.from_numpy(w.copy()))
            if mod.bias is not None:
                lin.bias.data.copy_(mod.bias.data)
            n += 1
    return n


def test_decoder_with_int4_attention_matches_dequantised_fp16():
    """convert_dense_to_int4 (q/k/v/o as Int4Linear, q/k/v in one stacked launch)
    against the same decoder whose projections hold the dequantised weights."""
    from hydranet_amd.kernels import Int4Linear
    from hydranet_amd.model.decoder import (MixtralDecoderConfig, build_synthetic_decoder,
                                            convert_dense_to_int4)
    cfg = MixtralDecoderConfig(num_layers=2, hidden_dim=512, intermediate_dim=1024,
                               num_attention_heads=8, num_kv_heads=2, head_dim=64,
                               vocab_size=512, num_experts=8, experts_per_token=2,
                               max_position_embeddings=64)
    model = build_synthetic_decoder(cfg, DEV, decode_top_k=1, seed=4)
    convert_dense_to_int4(model)
    att = model.layers[0].self_attn
    assert all(isinstance(getattr(att, n), Int4Linear) for n in ("q_proj", "k_proj", "v_proj",
                                                                 "o_proj"))
    assert not isinstance(model.lm_head, Int4Linear)
    assert not isinstance(model.layers[0].moe.router.gate, Int4Linear)
    ref = build_synthetic_decoder(cfg, DEV, decode_top_k=1, seed=4)  # same weights
    assert _load_dequantised(model, ref) == 4 * cfg.num_layers
    ids = torch.randint(0, cfg.vocab_size, (2, 8), device=DEV,
                        generator=torch.Generator(device=DEV).manual_seed(3))
    caches = [model.new_cache(2, 16), ref.new_cache(2, 16)]
    got, want = model(ids, caches[0]), ref(ids, caches[1])
    _close(got, want, atol=3e-2, rtol=1e-2)
    for _ in range(2):  # decode steps fed the same tokens
        tok = got[:, -1].argmax(-1, keepdim=True)
        got, want = model(tok, caches[0]), ref(tok, caches[1])
        _close(got, want, atol=3e-2, rtol=1e-2)


def test_glm_layer_with_int4_shared_expert():
    from hydranet_amd.kernels import Int4Linear, convert_model_to_int4
    from hydranet_amd.model.moe import GLM4MoELayer
    from hydranet_amd.preprocess.synthetic import make_expert_slot, slot_to_cpu
    H, I, E, k, T = 512, 256, 16, 4, 6
    slots = [make_expert_slot(500 + e, H, I, 128, slot_idx=e) for e in range(E)]
    layer = GLM4MoELayer(H, I, E, k, slots=slots).to(DEV).half()
    g = torch.Generator().manual_seed(12)
    layer.router.weight.data = (torch.randn(E, H, generator=g) * 0.02).float().to(DEV)
    for lin in (layer.shared_expert.gate_proj, layer.shared_expert.up_proj,
                layer.shared_expert.down_proj):
        lin.weight.data = (torch.randn(*lin.weight.shape, generator=g) * 0.02).half().to(DEV)
    convert_model_to_int4(layer, skip_layers=["router"])
    assert isinstance(layer.shared_expert.down_proj, Int4Linear)
    h = (torch.randn(1, T, H, generator=g)).half()
    out = layer(h.to(DEV))
    idx, w = layer.router(h.to(DEV))
    used = sorted(set(idx.view(-1).tolist()))
    shared = tuple(torch.from_numpy(oracle.dequant(m.weight_packed.cpu().numpy(),
                                                   m.weight_scale.cpu().numpy(), m.group_size)
                                    .copy())
                   for m in (layer.shared_expert.gate_proj, layer.shared_expert.up_proj,
                             layer.shared_expert.down_proj))
    ref = torch_ref.glm_moe(h.view(T, H), None, {e: slot_to_cpu(slots[e]) for e in used},
                            shared, routing=(idx.long().cpu(), w.cpu()))
    _close(out.view(T, H), ref)


def test_name_compatible_entry_points():
    """ExpertMLPTriton (kernels/expert_mlp.py:230-330) and the package-level
    expert_mlp_int4, which takes hidden_dim / intermediate_dim (the reference's
    kernels/__init__.py:15 name collision), against the oracle."""
    from hydranet_amd import kernels
    from hydranet_amd.kernels.expert_mlp import ExpertMLPTriton
    from hydranet_amd.kernels.int4_expert_mlp import expert_mlp_int4 as twin
    from hydranet_amd.preprocess.synthetic import make_expert_slot, slot_to_cpu
    H, I, T = 512, 384, 3
    slot = make_expert_slot(77, H, I, 128)
    e = tuple(getattr(slot, n) for n in ("gate_packed", "gate_scales", "up_packed", "up_scales",
                                         "down_packed", "down_scales"))
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(1)).half()
    ref = torch_ref.expert_mlp(x, *slot_to_cpu(slot), group_size=128)
    y_pkg = kernels.expert_mlp_int4(x.to(DEV), *e, H, I, 128)
    _close(y_pkg, ref)
    assert kernels.expert_mlp_int4 is not twin   # the collision is kept
    _close(twin(x.to(DEV), *e, 128), ref)
    mlp = ExpertMLPTriton(H, I, 128, torch.device(DEV))
    assert torch.equal(mlp.forward(x.to(DEV), *e), y_pkg)
    deq = mlp._dequant(e[0], e[1], I, H)
    np.testing.assert_array_equal(deq.cpu().numpy().view(np.uint16),
                                  oracle.dequant(e[0].cpu().numpy(), e[1].cpu().numpy(), 128)
                                  .view(np.uint16))
