"""Write the golden vectors in tests/golden/ by running the REFERENCE's own code.

Run in the build container only (the reference tree is not on the GPU box):

    python tests/golden/make_golden.py /root/reference
    python tests/golden/make_golden.py /root/reference grouped_router   # one fixture

The reference package is mapped to the name ``hydranet`` without executing its
package __init__ files (only the modules listed below are imported).  What it
pins, per fixture (all small, CPU, seeded):

  quantize_tensor.npz   ExpertWeightPacker.quantize_tensor      (preprocess/pack_weights.py:133-181)
                        + dequantize_tensor                      (:230-268)
  quantize_weight.npz   Int4Linear.quantize_weight               (kernels/int4_linear.py:68-107)
  expert_mlp.npz        ExpertMLPTriton.forward torch path       (kernels/expert_mlp.py:254-330)
  topk_router.npz       TopKRouter.forward, affinity off          (model/router.py:73-130)
  sigmoid_router.npz    GLM4SigmoidRouter.forward                 (model/glm4.py:261-309)
  grouped_router.npz    GLM4SigmoidRouter.forward with group-limited selection
                        (n_group > 1) and norm_topk_prob=False    (model/glm4.py:285-307)
  blob_layout.json      BlobLayout.from_dims at Mixtral/GLM dims  (cache/packed_expert_store.py:77-108)
  mixtral_moe_layer.npz MixtralMoELayer.forward, top-2 and top-1  (model/mixtral.py:259-370)
                        (fp16 dequantise-then-F.linear branch, every expert registered in a
                        CPU ExpertCacheManager, affinity off)
  glm_moe_layer.npz     GLM4MoELayer.forward with its fp16 shared expert (model/glm4.py:365-473)
  store_format/         pack_mixtral_experts' legacy per-expert files + metadata.json
                        (preprocess/pack_weights.py:271-381; files kept as SHA-256 digests)
                        and pack_to_single_blob's experts.bin / experts.idx
                        (cache/packed_expert_store.py:627-739)

The layer and store fixtures hold no weights: every expert weight comes from
gen.py (seeded, integer arithmetic), and the fixtures record the SHA-256 of
the packed bytes the reference's packer made from them, so a test that
regenerates the weights can check it packs the same bytes first.

Only data (inputs and the reference's outputs) is written; no reference
source is copied.
"""
from __future__ import annotations

import hashlib
import importlib
import json
import os
import shutil
import sys
import tempfile
import types
from pathlib import Path

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import gen  # noqa: E402

# Layer fixtures: (H, I, group, E, top-k list, tokens (B, S), case seed)
MIXTRAL_CASE = dict(H=128, I=256, g=128, E=8, topks=(2, 1), B=2, S=3, seed=5)
GLM_CASE = dict(H=128, I=256, g=128, E=16, k=4, B=1, S=5, seed=6)
# Store-format fixture: 2 layers x 2 experts
STORE_CASE = dict(L=2, E=2, H=128, I=128, g=128, seed=7)


def _map_reference(root: str) -> None:
    # bare package objects (their __init__ files would pull in the engine);
    # hydranet.cache is imported normally because model/glm4.py needs its exports
    for name, sub in [("hydranet", ""), ("hydranet.preprocess", "preprocess"),
                      ("hydranet.kernels", "kernels"), ("hydranet.model", "model")]:
        mod = types.ModuleType(name)
        mod.__path__ = [os.path.join(root, sub)] if sub else [root]
        sys.modules[name] = mod


def _f16(seed: int, shape, scale: float) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g, dtype=torch.float32) * scale).to(torch.float16)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def quantize_cases():
    cases = {}
    cases["randn_64x256_g128"] = (_f16(1, (64, 256), 0.02), 128)
    cases["randn_16x1408_g128"] = (_f16(2, (16, 1408), 0.02), 128)
    cases["randn_32x256_g64"] = (_f16(3, (32, 256), 0.1), 64)
    cases["randn_32x128_g32"] = (_f16(4, (32, 128), 1.0), 32)
    # exact .5 ties after w / s (absmax 7 -> s = 1), negatives, zeros,
    # an all-zero group (scale underflows to 0), subnormal-only group, huge values
    t = torch.zeros(4, 256, dtype=torch.float32)
    t[0, :128] = torch.tensor([7.0, -7.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, -3.5, 6.5, -6.5]
                              + [0.25 * i for i in range(116)])
    t[0, 128:] = torch.linspace(-1.0, 1.0, 128)
    t[1, :128] = 0.0
    t[1, 128:] = torch.linspace(-3e-7, 3e-7, 128)
    t[2, :] = torch.linspace(-60000.0, 60000.0, 256)
    t[3, :] = -0.0
    t[3, 5] = 1e-3
    cases["edge_4x256_g128"] = (t.to(torch.float16), 128)
    return cases


# Group-limited / unnormalised sigmoid routing cases:
# (E, top_k, n_group, topk_group, norm_topk_prob, routed_scaling_factor, seed)
GROUPED_ROUTER_CASES = {
    "g8_t3_k6_norm": (64, 6, 8, 3, True, 1.0, 51),
    "g1_k8_nonorm_s2.5": (128, 8, 1, 1, False, 2.5, 52),
    "g4_t2_k8_nonorm": (32, 8, 4, 2, False, 1.0, 53),
    "g16_t4_k8_norm_s1.5": (128, 8, 16, 4, True, 1.5, 54),
}


def grouped_router_fixture(glm4, cfg) -> None:
    """GLM4SigmoidRouter.forward with n_group > 1 / norm_topk_prob=False, 32
    tokens of H = 256 per case; inputs rejected unless the group choice and
    the top-k are tie-free (so the fixture pins the routing, not a tie-break)."""
    out = {}
    H, T = 256, 32
    for name, (E, k, ng, tg, norm, scale, seed) in GROUPED_ROUTER_CASES.items():
        gc = cfg.GLM4AirConfig()
        gc.hidden_dim = H
        gc.num_experts = E
        gc.experts_per_token = k
        gc.n_group = ng
        gc.topk_group = tg
        gc.norm_topk_prob = norm
        gc.routed_scaling_factor = scale
        sr = glm4.GLM4SigmoidRouter(gc, 0)
        g2 = torch.Generator().manual_seed(seed)
        sr.weight.data = torch.randn(E, H, generator=g2) * 0.05
        h = _f16(seed + 100, (1, T, H), 1.0)
        with torch.no_grad():
            ti, tw = sr(h)
            sc = torch.sigmoid(torch.nn.functional.linear(h.view(-1, H).float(), sr.weight.float()))
        if ng > 1:
            gmax = sc.view(T, ng, E // ng).max(dim=-1).values
            _assert_tie_free(gmax, tg, f"{name} group choice")
            keep = torch.zeros(T, ng)
            keep.scatter_(1, gmax.topk(tg, dim=-1).indices, 1.0)
            sc = (sc.view(T, ng, E // ng) * keep.unsqueeze(-1)).view(T, E)
        _assert_tie_free(sc, k, f"{name} top-k")
        out[f"{name}/w"] = sr.weight.data.numpy()
        out[f"{name}/h"] = _bits(h)
        out[f"{name}/idx"] = ti.numpy().astype(np.int32)
        out[f"{name}/wts"] = _bits(tw)
        out[f"{name}/cfg"] = np.array([E, k, ng, tg, int(norm)], dtype=np.int64)
        out[f"{name}/scaling"] = np.array(scale, dtype=np.float64)
    np.savez_compressed(os.path.join(HERE, "grouped_router.npz"), **out)


def main(root: str) -> None:
    _map_reference(root)
    pw = importlib.import_module("hydranet.preprocess.pack_weights")
    il = importlib.import_module("hydranet.kernels.int4_linear")
    em = importlib.import_module("hydranet.kernels.expert_mlp")
    cfg = importlib.import_module("hydranet.config")
    router = importlib.import_module("hydranet.model.router")
    glm4 = importlib.import_module("hydranet.model.glm4")
    store = importlib.import_module("hydranet.cache.packed_expert_store")

    # ---- ExpertWeightPacker.quantize_tensor / dequantize_tensor
    out = {}
    for name, (w, g) in quantize_cases().items():
        packer = pw.ExpertWeightPacker(pw.QuantConfig(bits=4, group_size=g, symmetric=True))
        packed, scales = packer.quantize_tensor(w)
        deq = packer.dequantize_tensor(packed, scales, w.shape[0], w.shape[1])
        out[f"{name}/w"] = _bits(w)
        out[f"{name}/group"] = np.array(g)
        out[f"{name}/packed"] = packed.numpy()
        out[f"{name}/scales"] = _bits(scales)
        out[f"{name}/dequant"] = _bits(deq)
    np.savez_compressed(os.path.join(HERE, "quantize_tensor.npz"), **out)

    # ---- Int4Linear.quantize_weight (fp32 and fp16 inputs)
    out = {}
    g = torch.Generator().manual_seed(11)
    for dt, dname in [(torch.float32, "f32"), (torch.float16, "f16")]:
        for gs in (128, 64, 32):
            w = (torch.randn(24, 256, generator=g) * 0.05).to(dt)
            if gs == 32:
                w[0, :32] = 0  # degenerate group
            packed, scale = il.Int4Linear.quantize_weight(w, gs)
            key = f"{dname}_g{gs}"
            out[f"{key}/w"] = w.numpy() if dt == torch.float32 else _bits(w)
            out[f"{key}/packed"] = packed.numpy()
            out[f"{key}/scales"] = _bits(scale)
    np.savez_compressed(os.path.join(HERE, "quantize_weight.npz"), **out)

    # ---- ExpertMLPTriton.forward (torch dequantise-then-matmul path), CPU
    out = {}
    H, I, gs = 128, 256, 128
    packer = pw.ExpertWeightPacker(pw.QuantConfig(group_size=gs))
    wts = {"gate_proj": _f16(21, (I, H), 0.02), "up_proj": _f16(22, (I, H), 0.02),
           "down_proj": _f16(23, (H, I), 0.02)}
    pe = packer.pack_expert(0, 0, wts)
    x = _f16(24, (5, H), 1.0)
    mlp = em.ExpertMLPTriton(H, I, gs, device=torch.device("cpu"))
    y = mlp.forward(x, pe.gate_proj_packed, pe.gate_proj_scales, pe.up_proj_packed,
                    pe.up_proj_scales, pe.down_proj_packed, pe.down_proj_scales)
    for k_, t_ in [("gate_packed", pe.gate_proj_packed), ("up_packed", pe.up_proj_packed),
                   ("down_packed", pe.down_proj_packed)]:
        out[k_] = t_.numpy()
    for k_, t_ in [("gate_scales", pe.gate_proj_scales), ("up_scales", pe.up_proj_scales),
                   ("down_scales", pe.down_proj_scales), ("x", x), ("y", y)]:
        out[k_] = _bits(t_)
    out["dims"] = np.array([H, I, gs])
    np.savez_compressed(os.path.join(HERE, "expert_mlp.npz"), **out)

    # ---- TopKRouter.forward (fp16 gate, affinity off), with forced ties
    out = {}
    mc = cfg.MixtralConfig()
    mc.hidden_dim = 256
    r = router.TopKRouter(mc, cfg.ExpertCacheConfig(enable_affinity_bonus=False), 0)
    gw = _f16(31, (8, 256), 0.02)
    gw[5] = gw[2]          # experts 2 and 5 tie on every token
    r.gate.weight.data = gw.clone()
    r.eval()
    h = _f16(32, (1, 24, 256), 1.0)
    h[0, 3] = 0.0          # all eight logits tie
    h[0, 7] = h[0, 6]
    with torch.no_grad():
        for k in (1, 2):
            ro = r(h, top_k_override=k, apply_affinity=False)
            out[f"k{k}/idx"] = ro.expert_indices.numpy().astype(np.int32)
            out[f"k{k}/w"] = _bits(ro.expert_weights)
            out[f"k{k}/logits"] = ro.router_logits.numpy()
    out["gate"] = _bits(gw)
    out["h"] = _bits(h)
    np.savez_compressed(os.path.join(HERE, "topk_router.npz"), **out)

    # ---- TopKRouter.forward with the cache-affinity bonus (model/router.py:132-175):
    #      experts 1, 4, 6 cached; hidden rows scaled so some tokens are below
    #      and some above the entropy threshold
    out = {}
    r = router.TopKRouter(mc, cfg.ExpertCacheConfig(enable_affinity_bonus=True), 0)
    ga = _f16(33, (8, 256), 0.02)
    r.gate.weight.data = ga.clone()
    r.eval()
    cached = {1, 4, 6}
    r.set_cache_checker(lambda e: e in cached)
    h = _f16(34, (1, 24, 256), 1.0)
    h[0, ::3] = h[0, ::3] * 40.0  # confident rows: low entropy, no bonus
    with torch.no_grad():
        for k in (1, 2):
            ro = r(h, top_k_override=k)
            out[f"k{k}/idx"] = ro.expert_indices.numpy().astype(np.int32)
            out[f"k{k}/w"] = _bits(ro.expert_weights)
            out[f"k{k}/logits"] = ro.router_logits.numpy()
    out["gate"] = _bits(ga)
    out["h"] = _bits(h)
    out["cached"] = np.array(sorted(cached), dtype=np.int32)
    out["bonus"] = np.array([r.affinity_bonus, r.entropy_threshold], dtype=np.float64)
    np.savez_compressed(os.path.join(HERE, "affinity_router.npz"), **out)

    # ---- GLM4SigmoidRouter.forward (fp32 weight, top-8 of 128)
    out = {}
    gc = cfg.GLM4AirConfig()
    gc.hidden_dim = 256
    sr = glm4.GLM4SigmoidRouter(gc, 1)
    g2 = torch.Generator().manual_seed(41)
    sr.weight.data = torch.randn(gc.num_experts, 256, generator=g2) * 0.02
    h = _f16(42, (1, 32, 256), 1.0)
    with torch.no_grad():
        ti, tw = sr(h)
    out["w"] = sr.weight.data.numpy()
    out["h"] = _bits(h)
    out["idx"] = ti.numpy().astype(np.int32)
    out["wts"] = _bits(tw)
    out["cfg"] = np.array([gc.num_experts, gc.experts_per_token, gc.n_group, gc.topk_group,
                           int(gc.norm_topk_prob)], dtype=np.int64)
    out["scaling"] = np.array(gc.routed_scaling_factor, dtype=np.float64)
    np.savez_compressed(os.path.join(HERE, "sigmoid_router.npz"), **out)
    grouped_router_fixture(glm4, cfg)

    # ---- BlobLayout
    lay = {}
    for name, (hd, idim, gs) in {"mixtral": (4096, 14336, 128), "glm4_air": (4096, 1408, 128),
                                 "small": (128, 256, 128)}.items():
        L = store.BlobLayout.from_dims(hd, idim, gs)
        lay[name] = {"dims": [hd, idim, gs], "total_size": L.total_size,
                     **{f: getattr(L, f) for f in L.__dataclass_fields__}}
    with open(os.path.join(HERE, "blob_layout.json"), "w") as f:
        json.dump(lay, f, indent=1, sort_keys=True)

    moe_layer_fixtures(pw, cfg)
    store_format_fixture(pw, cfg, store)
    print("golden vectors written to", HERE)


# ----------------------------------------------------------------------------- MoE layers
def _packed_expert(pw, case_seed: int, e: int, H: int, I: int, g: int, layer: int = 0):
    """The reference packer's PackedExpert of the seeded expert, its dequantised
    fp16 weights, and the SHA-256 of its packed bytes in blob order."""
    w = {k: torch.from_numpy(v) for k, v in gen.expert_weights(case_seed, e, H, I, layer).items()}
    packer = pw.ExpertWeightPacker(pw.QuantConfig(bits=4, group_size=g, symmetric=True))
    pe = packer.pack_expert(layer, e, w)
    deq = {"gate_proj": packer.dequantize_tensor(pe.gate_proj_packed, pe.gate_proj_scales, I, H),
           "up_proj": packer.dequantize_tensor(pe.up_proj_packed, pe.up_proj_scales, I, H),
           "down_proj": packer.dequantize_tensor(pe.down_proj_packed, pe.down_proj_scales, H, I)}
    h = hashlib.sha256()
    for t in (pe.gate_proj_packed, pe.gate_proj_scales, pe.up_proj_packed, pe.up_proj_scales,
              pe.down_proj_packed, pe.down_proj_scales):
        h.update(t.contiguous().numpy().tobytes())
    return pe, deq, h.hexdigest()


def _cpu_cache_manager(cfg, model_config, n_experts: int):
    """A CPU ExpertCacheManager with room for every expert (no eviction), no affinity."""
    cache_mod = importlib.import_module("hydranet.cache.expert_cache")
    half = (n_experts + 1) // 2
    cc = cfg.ExpertCacheConfig(pinned_slots=0, hot_slots=half, probation_slots=half,
                               enable_dynamic_slots=False, enable_affinity_bonus=False,
                               enable_prefetch=False)
    mgr = cache_mod.ExpertCacheManager(model_config=model_config, cache_config=cc,
                                       device=torch.device("cpu"), dtype=torch.float16)
    return mgr, cc


def _assert_tie_free(logits: torch.Tensor, k: int, what: str) -> None:
    srt = torch.sort(logits.reshape(-1, logits.shape[-1]).double(), dim=-1, descending=True)[0]
    assert bool((srt[:, k - 1] > srt[:, k]).all()), f"{what}: a top-{k} boundary tie"


def moe_layer_fixtures(pw, cfg) -> None:
    mixtral = importlib.import_module("hydranet.model.mixtral")
    glm4 = importlib.import_module("hydranet.model.glm4")

    # ---- MixtralMoELayer.forward
    C = MIXTRAL_CASE
    H, I, g, E = C["H"], C["I"], C["g"], C["E"]
    mc = cfg.MixtralConfig()
    mc.num_layers, mc.num_experts, mc.hidden_dim, mc.intermediate_dim = 1, E, H, I
    mgr, cc = _cpu_cache_manager(cfg, mc, E)
    out = {"dims": np.array([H, I, g, E, C["seed"]])}
    for e in range(E):
        _, deq, digest = _packed_expert(pw, C["seed"], e, H, I, g)
        mgr.register_expert(0, e, deq)
        out[f"sha/{e}"] = np.array(digest)
    layer = mixtral.MixtralMoELayer(mc, cc, 0, mgr)
    gate = torch.from_numpy(gen.normal_f16(C["seed"] * 1000 + 901, (E, H), 0.02))
    layer.router.gate.weight.data = gate.clone()
    layer.eval()
    hid = torch.from_numpy(gen.normal_f16(C["seed"] * 1000 + 902, (C["B"], C["S"], H), 1.0))
    out["gate"] = _bits(gate)
    out["h"] = _bits(hid)
    with torch.no_grad():
        for k in C["topks"]:
            ro = layer.router(hid, top_k_override=k, apply_affinity=False)
            _assert_tie_free(ro.router_logits, k, "mixtral fixture")
            y = layer(hid, top_k=k)
            out[f"k{k}/idx"] = ro.expert_indices.numpy().astype(np.int32)
            out[f"k{k}/w"] = _bits(ro.expert_weights)
            out[f"k{k}/logits"] = ro.router_logits.numpy()
            out[f"k{k}/out"] = _bits(y)
    mgr.shutdown()
    np.savez_compressed(os.path.join(HERE, "mixtral_moe_layer.npz"), **out)

    # ---- GLM4MoELayer.forward (shared fp16 expert + routed experts)
    C = GLM_CASE
    H, I, g, E, k = C["H"], C["I"], C["g"], C["E"], C["k"]
    gc = cfg.GLM4AirConfig()
    gc.hidden_dim, gc.moe_intermediate_dim, gc.num_experts, gc.experts_per_token = H, I, E, k
    adapter = types.SimpleNamespace(num_layers=1, num_experts=E,
                                    expert_size_bytes=3 * H * I * 2)
    mgr, _ = _cpu_cache_manager(cfg, adapter, E)
    out = {"dims": np.array([H, I, g, E, k, C["seed"]])}
    for e in range(E):
        _, deq, digest = _packed_expert(pw, C["seed"], e, H, I, g)
        mgr.register_expert(0, e, deq)
        out[f"sha/{e}"] = np.array(digest)
    layer = glm4.GLM4MoELayer(gc, 0, mgr)
    layer.eval()
    rw = torch.from_numpy(gen.normal(C["seed"] * 1000 + 901, (E, H), 0.02))
    layer.router.weight.data = rw.clone()
    sh = gen.expert_weights(C["seed"], 999, H, I)
    layer.shared_expert.half()
    for name in ("gate_proj", "up_proj", "down_proj"):
        getattr(layer.shared_expert, name).weight.data = torch.from_numpy(sh[name]).clone()
    hid = torch.from_numpy(gen.normal_f16(C["seed"] * 1000 + 902, (C["B"], C["S"], H), 1.0))
    with torch.no_grad():
        logits = torch.nn.functional.linear(hid.reshape(-1, H).float(), rw)
        _assert_tie_free(torch.sigmoid(logits), k, "glm fixture")
        ti, tw = layer.router(hid)
        y = layer(hid)
    out["router_w"] = rw.numpy()
    out["h"] = _bits(hid)
    out["idx"] = ti.numpy().astype(np.int32)
    out["w"] = _bits(tw)
    out["out"] = _bits(y)
    out["last_selected"] = np.array(layer.get_last_selected_experts(), dtype=np.int32)
    mgr.shutdown()
    np.savez_compressed(os.path.join(HERE, "glm_moe_layer.npz"), **out)


# ----------------------------------------------------------------------------- store format
def store_format_fixture(pw, cfg, store) -> None:
    """Legacy files written by pack_mixtral_experts and the single blob that
    pack_to_single_blob makes of them, for seeded 2-layer x 2-expert weights.
    pack_mixtral_experts reads a checkpoint through model.loader and sizes
    itself by MixtralConfig(); both are swapped for the call: a loader that
    yields the seeded experts, and a config with the fixture's dimensions."""
    C = STORE_CASE
    L, E, H, I, g = C["L"], C["E"], C["H"], C["I"], C["g"]

    class _SeededLoader:
        def __init__(self, model_path, config, device, dtype):
            self.config = config

        def iter_experts(self):
            for li in range(L):
                for e in range(E):
                    yield li, e, {k: torch.from_numpy(v) for k, v in
                                  gen.expert_weights(C["seed"], e, H, I, layer=li).items()}

    base = cfg.MixtralConfig

    class _SmallMixtral(base):
        def __init__(self):
            super().__init__()
            self.num_layers, self.num_experts = L, E
            self.hidden_dim, self.intermediate_dim = H, I

    stub = types.ModuleType("hydranet.model.loader")
    stub.MixtralWeightLoader = _SeededLoader
    prev = sys.modules.get("hydranet.model.loader")
    sys.modules["hydranet.model.loader"] = stub
    cfg.MixtralConfig = _SmallMixtral
    tmp = tempfile.mkdtemp()
    try:
        legacy = Path(tmp) / "legacy"
        meta = pw.pack_mixtral_experts("unused", str(legacy), pw.QuantConfig(group_size=g))
        blob_dir = Path(tmp) / "blob"
        store.pack_to_single_blob(legacy, blob_dir, _SmallMixtral(), group_size=g)
        dst = os.path.join(HERE, "store_format")
        os.makedirs(dst, exist_ok=True)
        digests = {}
        for f in sorted(legacy.glob("expert_L*_E*.bin")):
            digests[f.name] = hashlib.sha256(f.read_bytes()).hexdigest()
        with open(os.path.join(dst, "legacy_files.json"), "w") as f:
            json.dump({"case": C, "sha256": digests}, f, indent=1, sort_keys=True)
        shutil.copy(legacy / "metadata.json", os.path.join(dst, "metadata.json"))
        shutil.copy(blob_dir / "experts.bin", os.path.join(dst, "experts.bin"))
        shutil.copy(blob_dir / "experts.idx", os.path.join(dst, "experts.idx"))
        assert meta["format_version"] == "1.0"
    finally:
        cfg.MixtralConfig = base
        if prev is None:
            del sys.modules["hydranet.model.loader"]
        else:
            sys.modules["hydranet.model.loader"] = prev
        shutil.rmtree(tmp, ignore_errors=True)


def only_grouped_router(root: str) -> None:
    _map_reference(root)
    cfg = importlib.import_module("hydranet.config")
    glm4 = importlib.import_module("hydranet.model.glm4")
    grouped_router_fixture(glm4, cfg)


if __name__ == "__main__":
    _root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    if len(sys.argv) > 2 and sys.argv[2] == "grouped_router":
        only_grouped_router(_root)
    else:
        main(_root)
