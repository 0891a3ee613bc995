"""GPU test of config C5 at its full size: the Mixtral-8x7B-shaped decoder
(32 layers, H 4096, 32 query / 8 KV heads, head_dim 128, vocab 32000, every
expert INT4 g128 resident), 64 sequences of 512 seeded random prompt tokens.

Checks that do not need a CPU model of the whole network (too slow at this
size):
  * prefill is deterministic (two caches, logits bit for bit);
  * the replayed decode graphs (GraphDecoder) match eager decode steps fed the
    same tokens, within 3e-2 + 1e-2 |ref| on fp16 logits, and greedy decoding
    repeats its tokens;
  * at one eager decode step, the hidden states entering the MoE blocks of
    two layers and their outputs: each output equals the oracle's dispatch
    (torch_ref.moe_dispatch: per-expert dequantise + F.linear + fp16
    index_add_, model/mixtral.py:283-368) of those 64 rows over the routing
    the layer used, within the expert-MLP bar 1e-2 + 2e-3 |ref|; at the
    reference's decode default (top-1, TopKMode.DECODE) and at FORCED_TOP2
    (config.py:15-19)."""
import pytest
import torch

from oracle import torch_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
B, P = 64, 512


@pytest.fixture(scope="module")
def c5():
    from hydranet_amd.model.decoder import MixtralDecoderConfig, build_synthetic_decoder
    cfg = MixtralDecoderConfig(max_position_embeddings=P + 16)
    print(f"[c5] building the 32-layer decoder", flush=True)
    model = build_synthetic_decoder(cfg, DEV, decode_top_k=1, seed=5)
    ids = torch.randint(0, cfg.vocab_size, (B, P), device=DEV,
                        generator=torch.Generator(device=DEV).manual_seed(512))
    yield cfg, model, ids
    del model
    torch.cuda.empty_cache()


def _close(got, ref, atol, rtol, what):
    err = (got.float() - ref.float()).abs()
    bound = atol + rtol * ref.float().abs()
    assert torch.isfinite(got).all(), what
    assert bool((err <= bound).all()), f"{what}: {int((err > bound).sum())} off, max {err.max()}"


def test_c5_prefill_deterministic_graph_matches_eager(c5):
    from hydranet_amd.model.decoder import GraphDecoder
    cfg, model, ids = c5
    c_eager, c_graph = model.new_cache(B, P + 8), model.new_cache(B, P + 8)
    print("[c5] prefill x2", flush=True)
    l1 = model(ids, c_eager)
    l2 = model(ids, c_graph)
    assert torch.equal(l1, l2)
    tok = l1[:, -1].argmax(-1, keepdim=True)
    gd = GraphDecoder(model, c_graph, tok)
    for step in range(4):
        eager = model(tok, c_eager)
        gd.step()
        _close(gd.logits, eager, 3e-2, 1e-2, f"decode step {step}")
        tok = eager[:, -1].argmax(-1, keepdim=True)
        gd.tok.copy_(tok)
    # greedy decoding repeats itself (fresh caches)
    a = model.generate_greedy(ids[:8], 4)
    b = model.generate_greedy(ids[:8], 4)
    assert torch.equal(a, b) and a.shape == (8, 4)


@pytest.mark.parametrize("top_k", [1, 2])
def test_c5_moe_blocks_match_oracle_dispatch(c5, top_k):
    from hydranet_amd.preprocess.synthetic import slot_to_cpu
    cfg, model, ids = c5
    cache = model.new_cache(B, P + 2)
    tok = model(ids, cache)[:, -1].argmax(-1, keepdim=True)
    picked = (3, 30)
    seen = {}

    def hook(li):
        def fn(mod, args, out):
            seen[li] = (args[0].detach().reshape(B, -1).clone(), out.detach().reshape(B, -1)
                        .clone(), tuple(t.clone() for t in mod.last_routing))
        return fn

    hs = [model.layers[li].moe.register_forward_hook(hook(li)) for li in picked]
    # the MoE blocks' own forward (the folded launch, which the last test
    # compares with it, does not run the module's hooks)
    model.fold_moe_norm = False
    try:
        print(f"[c5] decode step, top-{top_k}", flush=True)
        model(tok, cache, top_k=top_k)
    finally:
        model.fold_moe_norm = True
        for h in hs:
            h.remove()
    for li in picked:
        x, y, (idx, w) = seen[li]
        assert idx.shape == (B, top_k)
        experts = {e: slot_to_cpu(s) for e, s in
                   enumerate(model.layers[li].moe.experts.table.slots)}
        ref = torch_ref.moe_dispatch(x.cpu(), idx.long().cpu(), w.cpu(), experts, 128)
        _close(y.cpu(), ref, 1e-2, 2e-3, f"layer {li} top-{top_k}")


@pytest.mark.parametrize("top_k", [1, 2])
def test_c5_folded_moe_norm_is_bit_identical(c5, top_k):
    """A decode step with the MoE block's residual add and the next RMSNorm
    inside its last launch (hn_unpermute_add_rmsnorm) gives the same logits,
    bit for bit, as the step with the unpermute and the norm as two
    launches: at top-1 after the decode layer (routing in the gate/up
    kernel), at top-2 (128 routed rows) after the routing launch and the
    experts' split down projection."""
    from hydranet_amd.model.moe import decode_layer_fits, experts_split_fits
    cfg, model, ids = c5
    moe = model.layers[0].moe
    table = moe.experts.static_table(DEV)
    fused = decode_layer_fits(B, moe.num_experts, top_k, table, moe.router.gate.weight, True)
    assert fused == (top_k == 1)
    assert fused or experts_split_fits(B, top_k, table), "the folded launch does not apply"
    cache = model.new_cache(B, P + 2)
    tok = model(ids[:, :P], cache)[:, -1].argmax(-1, keepdim=True)
    pos = torch.full((1,), cache.cur_len, dtype=torch.int64, device=DEV)
    print(f"[c5] folded vs unfolded decode step, top-{top_k}", flush=True)
    with torch.no_grad():
        model.fold_moe_norm = True
        a = model.step(tok, pos, cache, cache.cur_len + 1, None, top_k)
        model.fold_moe_norm = False
        b = model.step(tok, pos, cache, cache.cur_len + 1, None, top_k)
        model.fold_moe_norm = True
    torch.cuda.synchronize()
    assert torch.isfinite(a).all()
    assert torch.equal(a, b)
