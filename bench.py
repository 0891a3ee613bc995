#!/usr/bin/env python3
"""Benchmark of the MI355X INT4 expert-MLP hot path (one GPU).

    python bench.py [--steps K] [--warmup W] [--workload c1|c2|c3|c4|c5|...] [--tokens T]

Prints ONE JSON line.  A "step" is one pass of the hot path over one batch of
synthetic input already resident in HBM:

  c2  (default, the headline) one Mixtral MoE layer at decode, T = 1, 4, 16
      (value: T = 16): route + grouped gate/up + down + unpermute.  The default
      line also carries C1 ("c1": one expert at T = 1 against the 0.70 target),
      C3 ("c3"), C4 ("c4", TFLOP/s with its own MFMA roofline), the C5
      decoder (decoder_tokens_per_s) and the expert-miss load path ("h2d");
      --skip-c34 / --skip-c5 / --skip-h2d leave those out
  c1  one Mixtral expert SwiGLU (H 4096, I 14336, INT4 g128), T tokens (default 1)
  c3  one GLM-4.5-Air MoE layer at decode (T = 32, 128 experts, shared expert)
  c4  one Mixtral MoE layer at prefill (2048 tokens, Zipf-skewed routing)
  c5  the whole Mixtral-8x7B-shaped decoder: 64 x 512-token prompts, greedy
      decode (tokens/s over the decode forwards)
  c1phase / c2phase / c4phase: only the kernels of a counter run (rocprofv3 --pmc)

Weights are seeded N(0, 0.02) fp16 packed to INT4 by the GPU packer.  Steps
rotate over enough distinct experts (>= 0.7 GB) that weights stream from HBM,
not from the 256 MB Infinity Cache.  Steps are replayed from a HIP graph.

roofline: the dominant kernel's algorithmic bytes (flops) per launch divided by
its average duration, timed with HIP events on the stream the kernel runs on
(c2: after a warm-up pass of whole layers, 48 back-to-back launches of the
routing + gate/up kernel over the rotating layers between two events; the
down kernel likewise).  roofline.read_probe: the same bytes read by a plain
streaming read (hn_hbm_read_probe, timed the same way) and the kernel's time
as a fraction of it.
cpu_baseline: the torch-CPU restatement of the reference's
dequantise-then-matmul path (oracle/torch_ref.py) on this host: the headline
C2 layer at T = 16 (value) and T = 1, 4 (per_T), and one C1 expert ("c1").
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

import torch

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
METRIC = ("INT4 expert-MLP HBM GB/s (% of peak); Mixtral-shape decode tokens/sec, 1 GPU")


def _log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def _chunk(k: int, cap: int = 50) -> int:
    for c in range(min(cap, k), 0, -1):
        if k % c == 0:
            return c
    return 1


def _graph(fn, reps: int):
    """Capture `reps` calls of fn into one HIP graph; None if capture fails."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()  # warm allocator on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    try:
        with torch.cuda.graph(g):
            for _ in range(reps):
                fn()
    except Exception as exc:  # pragma: no cover - reported in the JSON
        _log("graph capture failed:", exc)
        return None
    return g


def _warm_replay(g) -> None:
    """One untimed replay of a freshly captured graph (its first replay carries
    one-time setup), then a device sync; part of the warm-up."""
    if g is not None:
        g.replay()
    torch.cuda.synchronize()


def _time_graph(g: torch.cuda.CUDAGraph, replays: int) -> float:
    """Average ms per replay, with events on the current stream."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    g.replay()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) / replays


# ----------------------------------------------------------------------------- C1
def bench_c1(args):
    from hydranet_amd import _lib
    from hydranet_amd.preprocess.synthetic import make_expert_slot, normal_f16, expert_seed
    from hydranet_amd.kernels import expert_mlp_int4_fused

    H, I, g, T = 4096, 14336, 128, args.tokens
    n_exp = 8  # 8 x 90.8 MB rotate: 727 MB > 256 MB Infinity Cache
    slots = [make_expert_slot(expert_seed(0, e), H, I, g, slot_idx=e) for e in range(n_exp)]
    x = normal_f16((T, H), 1234, std=1.0)
    blob = slots[0].layout.total_size
    bytes_step = blob + 2 * T * H * 2  # the expert's blob + x + y

    outs = [torch.empty(T, H, dtype=torch.float16, device="cuda") for _ in range(n_exp)]
    hws = [torch.empty(T, I, dtype=torch.float16, device="cuda") for _ in range(n_exp)]
    work = _lib.skinny_workspace(2, T, H, I, 0, "cuda")
    state = {"i": 0}

    def step():
        e = state["i"] % n_exp
        state["i"] += 1
        sl = slots[e]
        _lib.call("hn_expert_mlp_int4", _lib.ptr(x), *[_lib.ptr(t) for t in (
            sl.gate_packed, sl.gate_scales, sl.up_packed, sl.up_scales, sl.down_packed,
            sl.down_scales)], _lib.ptr(outs[e]), T, H, I, g, _lib.ptr(hws[e]), _lib.ptr(work),
            work.numel(), _lib.stream())

    # parity of the product entry point vs the CPU oracle on expert 0
    y_gpu = expert_mlp_int4_fused(x, slots[0].gate_packed, slots[0].gate_scales,
                                  slots[0].up_packed, slots[0].up_scales, slots[0].down_packed,
                                  slots[0].down_scales, g)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    chunk = _chunk(args.steps)
    state["i"] = 0
    gr = _graph(step, chunk)
    _warm_replay(gr)
    t0 = time.perf_counter()
    if gr is not None:
        for _ in range(args.steps // chunk):
            gr.replay()
    else:
        for _ in range(args.steps):
            step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms = dt * 1e3 / args.steps

    # dominant kernel: gate+up+SiLU (two thirds of the bytes); also time down
    reps = 16

    def gate_up_only():
        e = state["i"] % n_exp
        state["i"] += 1
        sl = slots[e]
        _lib.call("hn_int4_gate_up_silu", _lib.ptr(x), H, _lib.ptr(sl.gate_packed),
                  _lib.ptr(sl.gate_scales), _lib.ptr(sl.up_packed), _lib.ptr(sl.up_scales),
                  H // 2, H // g, _lib.ptr(hws[e]), I, T, I, H, g, _lib.ptr(work), work.numel(),
                  _lib.stream())

    def down_only():
        e = state["i"] % n_exp
        state["i"] += 1
        sl = slots[e]
        _lib.call("hn_int4_linear", _lib.ptr(hws[e]), I, _lib.ptr(sl.down_packed), I // 2,
                  _lib.ptr(sl.down_scales), I // g, _lib.ptr(outs[e]), H, T, H, I, g,
                  _lib.ptr(work), work.numel(), _lib.stream())

    kt = {}
    for name, fn in (("gate_up_silu", gate_up_only), ("down", down_only)):
        gk = _graph(fn, reps)
        kt[name] = _time_graph(gk, 10) / reps if gk is not None else float("nan")
    gu_bytes = 2 * (slots[0].layout.gate_packed_size + slots[0].layout.gate_scales_size) + \
        T * H * 2 + T * I * 2
    dn_bytes = slots[0].layout.down_packed_size + slots[0].layout.down_scales_size + \
        T * I * 2 + T * H * 2
    achieved = gu_bytes / (kt["gate_up_silu"] * 1e-3) / 1e9
    result = {
        "metric": METRIC,
        "value": round(bytes_step / (ms * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "tokens_per_s": round(T / (ms * 1e-3), 1),
        "ms_per_step": round(ms, 5),
        "dtype": "fp16",
        "config": {"workload": f"C1: one Mixtral expert SwiGLU 4096->14336->4096, INT4 g128, "
                               f"T={T}", "tokens": T, "hidden": H, "intermediate": I,
                   "group_size": g, "experts_rotated": n_exp, "bytes_per_step": bytes_step,
                   "graph": gr is not None},
        "roofline": {"bound": "hbm",
                     "kernel": ("stream_kernel (gate+up+SiLU, persistent)" if args.decode_path == 0
                                else "skinny_kernel (gate+up+SiLU, split-K)"),
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "bytes_per_launch": gu_bytes, "avg_us": round(kt["gate_up_silu"] * 1e3, 3),
                     "down_avg_us": round(kt["down"] * 1e3, 3),
                     "down_gbs": round(dn_bytes / (kt["down"] * 1e-3) / 1e9, 1),
                     "expert_frac": round(bytes_step / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
    }
    return result, (slots[0], x, y_gpu, g)


# ----------------------------------------------------------------------------- C2
def bench_c2(args, T: int, n_layers: int = 4, phases: bool = False):
    """One Mixtral MoE layer at decode: router + permute + grouped SwiGLU + unpermute.
    Steps rotate over n_layers layers of 8 experts (2.9 GB for 4 layers)."""
    from hydranet_amd import _lib
    from hydranet_amd.model.moe import MixtralMoELayer, ExpertTable
    from hydranet_amd.model.router import mixtral_route
    from hydranet_amd.preprocess.synthetic import make_expert_slot, normal_f16, expert_seed

    H, I, g, E = 4096, 14336, 128, 8
    layers = []
    for L in range(n_layers):
        slots = [make_expert_slot(expert_seed(L, e), H, I, g, slot_idx=e) for e in range(E)]
        layer = MixtralMoELayer(H, E, 2, layer_idx=L, slots=slots).cuda()
        layer.router.gate.weight.data = normal_f16((E, H), 7000 + L)
        layers.append(layer)
    x = normal_f16((1, T, H), 1234 + T, std=1.0)
    blob = layers[0].experts.table.slots[0].layout.total_size
    # algorithmic bytes per layer step: unique experts' blobs + gate + x + y
    step_bytes = []
    for layer in layers:
        idx, _, _ = mixtral_route(x.view(T, H), layer.router.gate.weight, 2)
        uniq = int(torch.unique(idx).numel())
        step_bytes.append(uniq * blob + E * H * 2 + 2 * T * H * 2)
    state = {"i": 0}

    def step():
        layer = layers[state["i"] % n_layers]
        state["i"] += 1
        layer(x, top_k=2)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    chunk = _chunk(args.steps)
    state["i"] = 0
    gr = _graph(step, chunk)
    _warm_replay(gr)
    t0 = time.perf_counter()
    if gr is not None:
        for _ in range(args.steps // chunk):
            gr.replay()
    else:
        for _ in range(args.steps):
            step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    total_bytes = sum(step_bytes[i % n_layers] for i in range(args.steps))
    gbs = total_bytes / (ms * 1e-3 * args.steps) / 1e9
    res = {"tokens": T, "ms_per_step": round(ms, 5), "GB_s": round(gbs, 1),
           "frac": round(gbs / HBM_PEAK_GBS, 4), "tokens_per_s": round(T / (ms * 1e-3), 1),
           "avg_unique_experts": sum((b - E * H * 2 - 4 * T * H) // blob for b in step_bytes)
           / n_layers, "graph": gr is not None}
    if phases and args.decode_path == 0:
        res["phases"] = time_decode_phases(layers, x.view(T, H), T, H, I, g, E)
    # for the CPU baseline and its parity check: layer 0's output on this input
    res["_ctx"] = (layers[0], x.view(T, H), layers[0](x, top_k=2).view(T, H))
    return res


def time_decode_phases(layers, x, T, H, I, g, E, reps: int = 12):
    """The two expert phases of the decode layer over the rotating layers:
    routing + gate/up (one launch, hn_moe_route_gate_up) and the down
    projection in four K slices (hn_grouped_decode_phase_int4 phase 1), each
    timed as a run of back-to-back launches after a warm-up pass of whole
    layers.  Bytes per launch: the active experts' packed weights and scales
    plus activations in and out (and the fp16 gate for the routing; the down
    phase writes four fp32 K-slice partials)."""
    from hydranet_amd import _lib
    from hydranet_amd.model.moe import Routed
    k = 2
    n = T * k
    xx = _lib.aligned_rows(x)
    gates = [_lib.aligned_rows(l.router.gate.weight.to(torch.float16)) for l in layers]
    rts = [Routed(T, k, E, 0, "cuda") for _ in layers]
    h_ws = torch.empty(n, I, dtype=torch.float16, device="cuda")
    out = torch.empty(T, H, dtype=torch.float16, device="cuda")
    work = _lib.skinny_workspace(3, n, H, I, E, "cuda")
    lay = layers[0].experts.table.slots[0].layout
    gu = 2 * (lay.gate_packed_size + lay.gate_scales_size)
    dn = lay.down_packed_size + lay.down_scales_size
    sp = _lib.stream()

    def route_gate_up(li):
        r, tb = rts[li], layers[li].experts.table
        _lib.call("hn_moe_route_gate_up", _lib.ptr(xx), H, _lib.ptr(gates[li]), H, None, T, E, k,
                  _lib.ptr(tb.dev), H, I, g, 1e-9, 1.0, None, _lib.ptr(r.idx), _lib.ptr(r.w),
                  _lib.ptr(r.offsets), _lib.ptr(r.perm), _lib.ptr(r.inv), _lib.ptr(r.active),
                  _lib.ptr(r.n_active), None, _lib.ptr(h_ws), sp)

    def down(li):
        r, tb = rts[li], layers[li].experts.table
        _lib.call("hn_grouped_decode_phase_int4", 1, _lib.ptr(h_ws), _lib.ptr(tb.dev),
                  _lib.ptr(r.active), _lib.ptr(r.n_active), _lib.ptr(r.offsets), E, T, n, H, I, g,
                  _lib.ptr(h_ws), _lib.ptr(work), work.numel(), sp)

    def unpermute(li):
        # same launch shape as the layer's unpermute (fp16 rows of h_ws as y)
        r = rts[li]
        _lib.call("hn_moe_unpermute", _lib.ptr(h_ws), I, _lib.ptr(r.inv), _lib.ptr(r.idx),
                  _lib.ptr(r.w), T, k, None, H, _lib.ptr(out), H, H, sp)

    n_it = 4 * reps
    for it in range(4):  # warm-up: every layer's routing outputs in place
        route_gate_up(it % 4); down(it % 4); unpermute(it % 4)
    torch.cuda.synchronize()
    # each phase as n_it back-to-back launches over the rotating layers between
    # two events on the launch stream (the host enqueues faster than a launch
    # runs, so the average is the kernel's duration plus the queue's gap, not
    # the per-launch dispatch an event pair around each eager launch adds)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    ev[0].record()
    for it in range(n_it):
        route_gate_up(it % len(layers))
    ev[1].record()
    ev[2].record()
    for it in range(n_it):
        down(it % len(layers))
    ev[3].record()
    torch.cuda.synchronize()
    nact = [int(r.n_active.item()) for r in rts]
    t_gu = ev[0].elapsed_time(ev[1]) / n_it * 1e3
    t_dn = ev[2].elapsed_time(ev[3]) / n_it * 1e3
    res = {}
    avg_act = sum(nact) / len(nact)
    for name, us, nbytes in (("route_gate_up_silu", t_gu,
                              avg_act * gu + T * H * 2 + E * H * 2 + n * I * 2),
                             ("down_4slices", t_dn, avg_act * dn + n * I * 2 + 4 * n * H * 4)):
        res[name] = {"avg_us": round(us, 3), "bytes_per_launch": int(nbytes),
                     "GB_s": round(nbytes / (us * 1e-6) / 1e9, 1)}
    res["active_experts"] = avg_act
    return res


# ----------------------------------------------------------------------------- C3
def bench_c3(args, T: int = 32, n_layers: int = 2):
    """One GLM-4.5-Air MoE layer at decode: 128 INT4 experts (4096->1408->4096, g128),
    fp16 shared expert, fp32 sigmoid router with a seeded U(-0.1, 0.1) selection bias,
    top-8, T = 32 tokens.  Steps rotate over n_layers layers (2.3 GB for 2).
    Algorithmic bytes: the unique experts' blobs (from the actual routing) + the
    shared expert + the fp32 router weight + x in + y out."""
    from hydranet_amd.model.moe import GLM4MoELayer
    from hydranet_amd.preprocess.synthetic import make_expert_slot, normal_f16, expert_seed

    H, I, g, E, k = 4096, 1408, 128, 128, 8
    layers = []
    for L in range(n_layers):
        slots = [make_expert_slot(expert_seed(L, e), H, I, g, slot_idx=e) for e in range(E)]
        layer = GLM4MoELayer(H, I, E, k, layer_idx=L, slots=slots).cuda().half()
        if args.fused_routing is not None:
            layer.fused_routing = bool(args.fused_routing)
        if args.shared_side_stream is not None:
            layer.shared_side_stream = bool(args.shared_side_stream)
        gen = torch.Generator(device="cuda").manual_seed(9000 + L)
        layer.router.weight.data = (torch.randn(E, H, generator=gen, device="cuda") * 0.02).float()
        layer.router.selection_bias = torch.rand(E, generator=gen, device="cuda") * 0.2 - 0.1
        for j, lin in enumerate((layer.shared_expert.gate_proj, layer.shared_expert.up_proj,
                                 layer.shared_expert.down_proj)):
            lin.weight.data = normal_f16(tuple(lin.weight.shape), 9100 + 10 * L + j)
        layer.eval()
        layers.append(layer)
    x = normal_f16((1, T, H), 3232, std=1.0)
    blob = layers[0].experts.table.slots[0].layout.total_size
    shared_bytes = 3 * H * I * 2
    step_bytes, uniq = [], []
    with torch.no_grad():
        for layer in layers:
            idx, _ = layer.router(x)
            u = int(torch.unique(idx).numel())
            uniq.append(u)
            step_bytes.append(u * blob + shared_bytes + E * H * 4 + 2 * T * H * 2)
    state = {"i": 0}

    def step():
        layer = layers[state["i"] % n_layers]
        state["i"] += 1
        with torch.no_grad():
            layer(x)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    chunk = _chunk(args.steps)
    state["i"] = 0
    gr = _graph(step, chunk)
    _warm_replay(gr)
    t0 = time.perf_counter()
    if gr is not None:
        for _ in range(args.steps // chunk):
            gr.replay()
    else:
        for _ in range(args.steps):
            step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    total_bytes = sum(step_bytes[i % n_layers] for i in range(args.steps))
    gbs = total_bytes / (ms * 1e-3 * args.steps) / 1e9
    return {"workload": "C3: one GLM-4.5-Air MoE layer at decode, T=32 (128 experts "
                        "4096->1408->4096 INT4 g128 + fp16 shared expert, sigmoid top-8 with "
                        "seeded selection bias); router + route + grouped SwiGLU + unpermute",
            "tokens": T, "ms_per_step": round(ms, 5), "GB_s": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "tokens_per_s": round(T / (ms * 1e-3), 1),
            "avg_unique_experts": sum(uniq) / len(uniq), "layers_rotated": n_layers,
            "graph": gr is not None}


# ----------------------------------------------------------------------------- C4
def zipf_logits(T: int, E: int, seed: int, s: float = 1.1, device="cuda"):
    """Router logits N(0,1) + ln p_e with Zipf(s) expert popularity (seeded)."""
    g = torch.Generator(device=device).manual_seed(seed)
    p = torch.tensor([1.0 / (i + 1) ** s for i in range(E)], device=device)
    return torch.randn(T, E, generator=g, device=device) + (p / p.sum()).log()


def bench_c4(args):
    """One Mixtral MoE layer at prefill: 2048 tokens, top-2 of 8 experts with
    Zipf(1.1)-skewed router logits.  Step = top-k + permute + gather + grouped
    gate/up+SiLU GEMM + grouped down GEMM + unpermute.  Work: 2 (T k) 3 H I flops."""
    from hydranet_amd import _lib
    from hydranet_amd.model.moe import ExpertTable, moe_experts_forward
    from hydranet_amd.model.router import topk_from_logits
    from hydranet_amd.preprocess.synthetic import make_expert_slot, normal_f16, expert_seed

    H, I, g, E, T, k = 4096, 14336, 128, 8, 2048, 2
    slots = [make_expert_slot(expert_seed(0, e), H, I, g, slot_idx=e) for e in range(E)]
    table = ExpertTable.from_slots(slots)
    x = normal_f16((T, H), 4242, std=1.0)
    logits = zipf_logits(T, E, 2048)
    idx0, _ = topk_from_logits(logits, k, mode=0)
    sizes = torch.bincount(idx0.view(-1).long(), minlength=E).tolist()
    flops = 2.0 * T * k * 3 * H * I

    def step():
        idx, w = topk_from_logits(logits, k, mode=0)
        moe_experts_forward(x, idx, w, table)

    for _ in range(max(2, args.warmup // 4)):
        step()
    torch.cuda.synchronize()
    steps = max(5, args.steps // 10)
    gr = _graph(step, steps)
    _warm_replay(gr)
    t0 = time.perf_counter()
    if gr is not None:
        gr.replay()
    else:
        for _ in range(steps):
            step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps

    # the two grouped GEMM launches alone, on their own stream, HIP events
    dev = x.device
    st = torch.cuda.Stream()
    idx, w = topk_from_logits(logits, k, mode=0)
    n = T * k
    meta = torch.empty(3 * E + 2 + 2 * n, dtype=torch.int32, device=dev)
    offs, act, nact = meta[:E + 1], meta[E + 1:2 * E + 1], meta[2 * E + 1:2 * E + 2]
    perm, inv = meta[2 * E + 2:2 * E + 2 + n], meta[2 * E + 2 + n:]
    x_perm = torch.empty(n, H, dtype=torch.float16, device=dev)
    h_ws = torch.empty(n, I, dtype=torch.float16, device=dev)
    y_perm = torch.empty(n, H, dtype=torch.float16, device=dev)
    work = _lib.gemm_workspace(dev)
    sp = ctypes_stream(st)
    torch.cuda.synchronize()
    _lib.call("hn_moe_permute", _lib.ptr(idx), T, k, E, _lib.ptr(offs), _lib.ptr(perm),
              _lib.ptr(inv), _lib.ptr(act), _lib.ptr(nact), sp)
    _lib.call("hn_moe_gather", _lib.ptr(x), H, _lib.ptr(perm), k, _lib.ptr(offs), E,
              _lib.ptr(x_perm), H, n, H, sp)
    kt = {}
    for phase, name in ((0, "gate_up_silu"), (1, "down")):
        def launch():
            _lib.call("hn_grouped_expert_phase_int4", phase, _lib.ptr(x_perm), _lib.ptr(table.dev),
                      _lib.ptr(act), _lib.ptr(nact), _lib.ptr(offs), E, n, H, I, g,
                      _lib.ptr(h_ws), _lib.ptr(y_perm), _lib.ptr(work), work.numel(), sp)
        for _ in range(2):
            launch()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        reps = 10
        e0.record(st)
        for _ in range(reps):
            launch()
        e1.record(st)
        e1.synchronize()
        kt[name] = e0.elapsed_time(e1) / reps
    gu_flops = 2.0 * n * 2 * H * I
    dn_flops = 2.0 * n * H * I
    ach = gu_flops / (kt["gate_up_silu"] * 1e-3) / 1e12
    return {"workload": "C4: one Mixtral MoE layer at prefill, 2048 tokens x 4096, top-2 of 8 "
                        "experts (4096->14336->4096 INT4 g128), Zipf(1.1)-skewed routing; "
                        "top-k + permute + gather + grouped gate/up GEMM + grouped down GEMM + "
                        "unpermute",
            "ms_per_step": round(ms, 4), "TFLOP_s": round(flops / (ms * 1e-3) / 1e12, 1),
            "frac": round(flops / (ms * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
            "tokens_per_s": round(T / (ms * 1e-3), 1), "group_sizes": sizes,
            "graph": gr is not None,
            "roofline": {"bound": "mfma", "kernel": "gemm_kernel<grouped, gate+up+SiLU>",
                         "achieved": round(ach, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(ach / MFMA_F16_PEAK_TFLOPS, 4),
                         "traffic": None, "flops_per_launch": gu_flops,
                         "avg_us": round(kt["gate_up_silu"] * 1e3, 2),
                         "down_avg_us": round(kt["down"] * 1e3, 2),
                         "down_TFLOP_s": round(dn_flops / (kt["down"] * 1e-3) / 1e12, 1)}}


def ctypes_stream(st):
    import ctypes
    return ctypes.c_void_p(st.cuda_stream)


def cpu_baseline_c1(ctx, budget_s: float):
    """Torch-CPU restatement of the reference's dequantise-then-matmul path,
    timed on this host.  TEST INFRASTRUCTURE (oracle) used only as the baseline."""
    from oracle import torch_ref
    from hydranet_amd.preprocess.synthetic import slot_to_cpu
    slot, x, y_gpu, g = ctx
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    e = slot_to_cpu(slot)
    xc = x.cpu()
    times = []
    y = None
    t_start = time.perf_counter()
    for i in range(64):
        t0 = time.perf_counter()
        y = torch_ref.expert_mlp(xc, *e, group_size=g)
        times.append(time.perf_counter() - t0)
        if i >= 3 and time.perf_counter() - t_start > budget_s:
            break
    runs = times[3:] if len(times) > 4 else times
    med = statistics.median(runs)
    err = (y_gpu.cpu().float() - y.float()).abs()
    ok = bool((err <= 1e-2 + 2e-3 * y.float().abs()).all())
    bytes_step = slot.layout.total_size + 2 * x.numel() * 2
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": round(bytes_step / med / 1e9, 3), "unit": "GB/s",
            "ms_per_step": round(med * 1e3, 2), "cores": torch.get_num_threads(), "kind": "port",
            "cpu": cpu_model,
            "sample": f"{len(runs)} timed calls (3 warm-up) of one C1 expert, median; "
                      f"dequant included per call"}, {"max_abs_err": float(err.max()),
                                                     "ok": ok}


def cpu_baseline_c2(ctxs, budget_s: float):
    """The headline workload (C2: one Mixtral MoE layer at decode) through the
    torch-CPU restatement of the reference's path (oracle/torch_ref.py:
    TopKRouter.forward + MixtralMoELayer.forward's fp16 dequantise-then-F.linear
    per expert + fp16 index_add_, model/router.py:96-120, model/mixtral.py:283-368),
    on this host, for T = 1, 4, 16.  Per call every routed expert is dequantised
    again (the reference clears its fp16 cache per layer, model/mixtral.py:583-584).
    TEST INFRASTRUCTURE (oracle) used only as the reported baseline; its output is
    also checked against the GPU layer's."""
    from oracle import torch_ref
    from hydranet_amd.preprocess.synthetic import slot_to_cpu
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    layer0 = ctxs["T16"][0]
    experts = {e: slot_to_cpu(s) for e, s in enumerate(layer0.experts.table.slots)}
    gate = layer0.router.gate.weight.detach().to(torch.float16).cpu()
    blob = layer0.experts.table.slots[0].layout.total_size
    E, H = gate.shape
    per_t, worst = {}, 0.0
    share = budget_s / len(ctxs)
    for name, (layer, x, y_gpu) in ctxs.items():
        xc = x.cpu()
        T = xc.shape[0]
        times, y = [], None
        t_start = time.perf_counter()
        for i in range(40):
            t0 = time.perf_counter()
            idx, w, _ = torch_ref.mixtral_router(xc, gate, 2)
            y = torch_ref.moe_dispatch(xc, idx, w, experts, 128)
            times.append(time.perf_counter() - t0)
            if i >= 4 and time.perf_counter() - t_start > share:
                break
        runs = times[3:]
        med = statistics.median(runs)
        uniq = int(torch.unique(idx).numel())
        nbytes = uniq * blob + E * H * 2 + 2 * T * H * 2
        err = (y_gpu.cpu().float() - y.float()).abs()
        ok = bool((err <= 1e-2 + 2e-3 * y.float().abs()).all())
        worst = max(worst, float(err.max()))
        per_t[name] = {"ms_per_step": round(med * 1e3, 2),
                       "GB_s": round(nbytes / med / 1e9, 3), "unique_experts": uniq,
                       "timed_calls": len(runs), "parity_ok": ok}
    head = per_t["T16"]
    return {"value": head["GB_s"], "unit": "GB/s", "ms_per_step": head["ms_per_step"],
            "cores": torch.get_num_threads(), "kind": "port", "cpu": _cpu_model(),
            "sample": "C2 (one Mixtral MoE layer at decode, layer 0 of the GPU run, same input) "
                      "at T = 16 (value) and T = 1 / 4: per T at least 2 warm-up + 2 timed "
                      "calls within " + f"{share:.0f} s, median; every routed expert dequantised "
                      "per call", "per_T": per_t, "max_abs_err_vs_gpu": worst}


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def c1phase(args):
    """Counter run: 20 launches each of the C1 gate/up+SiLU and down stream
    kernels (one Mixtral expert, T = 1, rotating over 8 experts), then 20 copies
    of 512 MiB (the copy calibrates FETCH_SIZE / WRITE_SIZE in bytes)."""
    from hydranet_amd import _lib
    from hydranet_amd.preprocess.synthetic import make_expert_slot, normal_f16, expert_seed
    H, I, g, T = 4096, 14336, 128, 1
    slots = [make_expert_slot(expert_seed(0, e), H, I, g, slot_idx=e) for e in range(8)]
    x = normal_f16((T, H), 1234, std=1.0)
    h = torch.empty(T, I, dtype=torch.float16, device="cuda")
    y = torch.empty(T, H, dtype=torch.float16, device="cuda")
    work = _lib.skinny_workspace(2, T, H, I, 0, "cuda")
    for r in range(20):
        sl = slots[r % 8]
        _lib.call("hn_int4_gate_up_silu", _lib.ptr(x), H, _lib.ptr(sl.gate_packed),
                  _lib.ptr(sl.gate_scales), _lib.ptr(sl.up_packed), _lib.ptr(sl.up_scales),
                  H // 2, H // g, _lib.ptr(h), I, T, I, H, g, _lib.ptr(work), work.numel(),
                  _lib.stream())
    for r in range(20):
        sl = slots[r % 8]
        _lib.call("hn_int4_linear", _lib.ptr(h), I, _lib.ptr(sl.down_packed), I // 2,
                  _lib.ptr(sl.down_scales), I // g, _lib.ptr(y), H, T, H, I, g, _lib.ptr(work),
                  work.numel(), _lib.stream())
    src = torch.empty(256 << 20, dtype=torch.float16, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(20):
        dst.copy_(src)
    torch.cuda.synchronize()
    lay = slots[0].layout
    print(json.dumps({"workload": "c1phase",
                      "gate_up_bytes_per_launch": 2 * (lay.gate_packed_size + lay.gate_scales_size)
                      + T * H * 2 + T * I * 2,
                      "down_bytes_per_launch": lay.down_packed_size + lay.down_scales_size
                      + T * I * 2 + T * H * 2, "copy_bytes": src.numel() * 2}), flush=True)


def bench_copy(args):
    """Reference rates for the 8 TB/s peak: torch's own device copy (read +
    write) and fp32 sum (read) of 1 and 4 GiB fp16 tensors, best of 10 by HIP
    events on the current stream; then read_probe at the expert kernels'
    bytes per launch."""
    out = {}
    for gib in (1, 4):
        n = gib * (1 << 30) // 2
        a = torch.randn(n, dtype=torch.float16, device="cuda")
        b = torch.empty_like(a)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for name, fn, nbytes in (("copy", lambda: b.copy_(a), 4 * n),
                                 ("sum", lambda: a.sum(dtype=torch.float32), 2 * n)):
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            best = float("inf")
            for _ in range(10):
                e0.record()
                fn()
                e1.record()
                torch.cuda.synchronize()
                best = min(best, e0.elapsed_time(e1))
            out[f"{name}_{gib}GiB"] = {"us": round(best * 1e3, 1),
                                       "GB_s": round(nbytes / best / 1e6, 1)}
        del a, b
        torch.cuda.empty_cache()
    # C1 down, C1 gate/up, C2 T=16 down, C2 T=16 gate/up (algorithmic bytes)
    out.update(read_probe({"read_30MB": 30_314_496, "read_61MB": 60_592_128,
                           "read_245MB": 245_235_712, "read_486MB": 485_556_224}))
    return out


def read_probe(targets: dict) -> dict:
    """hn_hbm_read_probe (a plain streaming read, 2048 workgroups) at each
    target's bytes per launch (rounded down to a multiple of 32 KiB): 48
    back-to-back launches, each over the next chunk of a 4 GiB buffer (no
    reuse from the 256 MB Infinity Cache), between two HIP events on the
    launch stream, after 8 untimed launches."""
    from hydranet_amd import _lib
    buf = torch.ones(4 << 30, dtype=torch.uint8, device="cuda")
    nwg = 2048
    sink = torch.zeros(nwg, dtype=torch.float32, device="cuda")
    st = _lib.stream()
    out = {}
    for name, target in targets.items():
        chunk = target // (nwg * 16) * nwg * 16
        nchunks = buf.numel() // chunk
        base = buf.data_ptr()

        def launch(i):
            _lib.call("hn_hbm_read_probe", base + (i % nchunks) * chunk, chunk, nwg,
                      _lib.ptr(sink), st)

        for i in range(8):
            launch(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(48):
            launch(i + 8)
        e1.record()
        e1.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / 48
        out[name] = {"bytes": chunk, "us": round(us, 2), "GB_s": round(chunk / us / 1e3, 1)}
    del buf, sink
    torch.cuda.empty_cache()
    return out


def bench_h2d(args):
    """Expert-miss path of the residency layer, one Mixtral expert = one 90.8 MB
    blob (a18): (1) pinned staging -> HBM, GpuExpertSlot.load_from_pinned on a
    copy stream (the host link alone, HIP events on that stream); (2) the whole
    PackedExpertStore.load_to_gpu_slot from an experts.bin on local disk (one
    read into the pinned staging ring -> one H2D copy per expert; the next
    expert's read overlaps the previous copy), page cache warm, host
    clock.  Eight experts, five passes each; every slab is compared with its
    blob byte for byte afterwards."""
    import shutil
    import tempfile
    import numpy as np
    from hydranet_amd.cache.blob_layout import BlobLayout
    from hydranet_amd.cache.packed_expert_store import GpuExpertSlot, PackedExpertStore
    from hydranet_amd.preprocess import pack_store as ps
    H, I, g, E, reps = 4096, 14336, 128, 8, 5
    lay = BlobLayout.from_dims(H, I, g)
    n = lay.total_size
    gen = np.random.default_rng(7)
    blobs = [gen.integers(0, 256, n, dtype=np.uint8) for _ in range(E)]
    pinned = [torch.from_numpy(b).pin_memory() for b in blobs]
    slots = [GpuExpertSlot(e, H, I, g, "cuda") for e in range(E)]
    cs = torch.cuda.Stream()

    def exact():
        return all(bool(torch.equal(slots[e].slab.cpu(), torch.from_numpy(blobs[e])))
                   for e in range(E))

    def load_pinned():
        for e in range(E):
            slots[e].load_from_pinned(pinned[e], lay, 0, e, stream=cs)

    load_pinned()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(cs)
    for _ in range(reps):
        load_pinned()
    e1.record(cs)
    e1.synchronize()
    us_pinned = e0.elapsed_time(e1) * 1e3 / (reps * E)
    ok = exact()
    for sl in slots:
        sl.slab.zero_()
    tmp = tempfile.mkdtemp(prefix="hn_h2d_")
    try:
        ps.write_packed_store(tmp, ((0, e, blobs[e]) for e in range(E)), 1, E, H, I, g,
                              model_type="mixtral")
        st = PackedExpertStore(os.path.join(tmp, "experts.idx"), device="cuda")
        for e in range(E):  # warms the page cache
            st.load_to_gpu_slot(0, e, slots[e])
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            for e in range(E):
                st.load_to_gpu_slot(0, e, slots[e])
        torch.cuda.synchronize()
        us_store = (time.perf_counter() - t0) * 1e6 / (reps * E)
        ok = ok and exact()
        st.close()
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return {"workload": "h2d: one Mixtral expert blob (4096 -> 14336 -> 4096 INT4 g128) per "
                        "load, 8 experts x 5 passes",
            "bytes_per_expert": n, "us_per_expert": round(us_pinned, 1),
            "GB_s": round(n / us_pinned / 1e3, 2),
            "store_path": {"us_per_expert": round(us_store, 1),
                           "GB_s": round(n / us_store / 1e3, 2),
                           "path": "experts.bin -> pinned staging (8 MiB preadv pieces on eight threads) -> "
                                   "H2D, page cache warm"},
            "bit_exact": ok}


def c2phase(args):
    """Counter run: 20 launches of the C2 T=16 routing + gate/up stream kernel (the
    roofline kernel), then 20 copies of 512 MiB (the copy calibrates FETCH_SIZE /
    WRITE_SIZE in bytes)."""
    from hydranet_amd import _lib
    from hydranet_amd.model.moe import ExpertTable, Routed
    from hydranet_amd.preprocess.synthetic import make_expert_slot, normal_f16, expert_seed
    H, I, g, E, T, k = 4096, 14336, 128, 8, 16, 2
    slots = [make_expert_slot(expert_seed(0, e), H, I, g, slot_idx=e) for e in range(E)]
    table = ExpertTable.from_slots(slots)
    gate = normal_f16((E, H), 7000)
    x = normal_f16((T, H), 1234 + T, std=1.0)
    r = Routed(T, k, E, 0, "cuda")
    n = T * k
    h_ws = torch.empty(n, I, dtype=torch.float16, device="cuda")
    for _ in range(20):
        _lib.call("hn_moe_route_gate_up", _lib.ptr(x), H, _lib.ptr(gate), H, None, T, E, k,
                  _lib.ptr(table.dev), H, I, g, 1e-9, 1.0, None, _lib.ptr(r.idx), _lib.ptr(r.w),
                  _lib.ptr(r.offsets), _lib.ptr(r.perm), _lib.ptr(r.inv), _lib.ptr(r.active),
                  _lib.ptr(r.n_active), None, _lib.ptr(h_ws), _lib.stream())
    src = torch.empty(256 << 20, dtype=torch.float16, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(20):
        dst.copy_(src)
    torch.cuda.synchronize()
    lay = slots[0].layout
    na = int(r.n_active.item())
    print(json.dumps({"workload": "c2phase", "active_experts": na,
                      "route_gate_up_bytes_per_launch": na * 2 * (
                          lay.gate_packed_size + lay.gate_scales_size) + T * H * 2 + E * H * 2
                      + n * I * 2, "copy_bytes": src.numel() * 2}), flush=True)


def c4phase(args):
    """Counter run: the C4 layer's grouped gate/up and down GEMM launches (three
    each, with the stream-K workspace), for rocprofv3 --pmc MFMA counters."""
    from hydranet_amd import _lib
    from hydranet_amd.model.moe import ExpertTable
    from hydranet_amd.model.router import topk_from_logits
    from hydranet_amd.preprocess.synthetic import make_expert_slot, normal_f16, expert_seed
    H, I, g, E, T, k = 4096, 14336, 128, 8, 2048, 2
    slots = [make_expert_slot(expert_seed(0, e), H, I, g, slot_idx=e) for e in range(E)]
    table = ExpertTable.from_slots(slots)
    x = normal_f16((T, H), 4242, std=1.0)
    idx, _ = topk_from_logits(zipf_logits(T, E, 2048), k, mode=0)
    n = T * k
    dev = x.device
    meta = torch.empty(3 * E + 2 + 2 * n, dtype=torch.int32, device=dev)
    offs, act, nact = meta[:E + 1], meta[E + 1:2 * E + 1], meta[2 * E + 1:2 * E + 2]
    perm, inv = meta[2 * E + 2:2 * E + 2 + n], meta[2 * E + 2 + n:]
    x_perm = torch.empty(n, H, dtype=torch.float16, device=dev)
    h_ws = torch.empty(n, I, dtype=torch.float16, device=dev)
    y_perm = torch.empty(n, H, dtype=torch.float16, device=dev)
    work = _lib.gemm_workspace(dev)
    sp = _lib.stream()
    _lib.call("hn_moe_permute", _lib.ptr(idx), T, k, E, _lib.ptr(offs), _lib.ptr(perm),
              _lib.ptr(inv), _lib.ptr(act), _lib.ptr(nact), sp)
    _lib.call("hn_moe_gather", _lib.ptr(x), H, _lib.ptr(perm), k, _lib.ptr(offs), E,
              _lib.ptr(x_perm), H, n, H, sp)
    for phase in (0, 1):
        for _ in range(3):
            _lib.call("hn_grouped_expert_phase_int4", phase, _lib.ptr(x_perm),
                      _lib.ptr(table.dev), _lib.ptr(act), _lib.ptr(nact), _lib.ptr(offs), E, n,
                      H, I, g, _lib.ptr(h_ws), _lib.ptr(y_perm), _lib.ptr(work), work.numel(), sp)
    torch.cuda.synchronize()
    print(json.dumps({"workload": "c4phase", "gate_up_flops": 2.0 * n * 2 * H * I,
                      "down_flops": 2.0 * n * H * I}), flush=True)


# ----------------------------------------------------------------------------- C5
def bench_c5(args):
    """Full Mixtral-8x7B-shaped decoder (32 layers, H 4096, 32 Q / 8 KV heads,
    head_dim 128, vocab 32000), random init N(0, 0.02) fp16, norms 1, all 256
    experts INT4 g128 resident in HBM.  64 sequences x 512 seeded random prompt
    ids, greedy decode of `--decode-tokens` tokens (top-2 routing at prefill,
    top-1 at decode).  The decode step is captured once as a HIP graph
    (GraphDecoder: attention over the whole cache with later positions masked)
    and replayed.  Timed: the decode forwards after `--warmup-decode` untimed
    ones; tokens/s = 64 x timed forwards / time.  bytes_per_step counts
    every expert of every layer once (64 tokens at top-1 leave an expert of a
    layer unused with probability (7/8)^64), the dense weights, the LM head and
    the KV cache read at the step's context length.  "top2": the same decode
    with top-2 routing (the reference's FORCED_TOP2 mode, config.py:15-19),
    from a second prefill, over min(64, --decode-tokens) tokens."""
    from hydranet_amd.model.decoder import (GraphDecoder, MixtralDecoderConfig,
                                            build_synthetic_decoder)

    B, P, N = 64, 512, args.decode_tokens
    cfg = MixtralDecoderConfig(max_position_embeddings=P + N)
    t0 = time.perf_counter()
    model = build_synthetic_decoder(cfg, "cuda", decode_top_k=1, seed=5)
    if args.attn_decode is not None:
        for layer in model.layers:
            layer.self_attn.decode_kernel = bool(args.attn_decode)
    torch.cuda.synchronize()
    _log("c5 built in", round(time.perf_counter() - t0, 1), "s")
    H, I, L = cfg.hidden_dim, cfg.intermediate_dim, cfg.num_layers
    blob = model.layers[0].moe.experts.table.slots[0].layout.total_size
    nh, nkv, hd = cfg.num_attention_heads, cfg.num_kv_heads, cfg.head_dim
    dense = (2 * H * nh * hd + 2 * H * nkv * hd) * 2 + cfg.num_experts * H * 2
    kv_per_pos = B * L * nkv * hd * 2 * 2
    ids = torch.randint(0, cfg.vocab_size, (B, P), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(512))
    cache = model.new_cache(B, P + N)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    logits = model(ids, cache)
    tok = logits[:, -1].argmax(-1, keepdim=True)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    del logits
    W = min(args.warmup_decode, N - 2)
    t0 = time.perf_counter()
    gd = GraphDecoder(model, cache, tok)  # the decode step, captured once
    torch.cuda.synchronize()
    capture_s = time.perf_counter() - t0
    for _ in range(W):
        gd.step()
    torch.cuda.synchronize()
    n = N - 1 - W
    ctx0 = cache.cur_len
    out = torch.empty((B, n), dtype=torch.int64, device="cuda")
    t0 = time.perf_counter()
    for i in range(n):
        out[:, i:i + 1].copy_(gd.step())
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    total_bytes = sum(L * (cfg.num_experts * blob + dense) + cfg.vocab_size * H * 2
                      + kv_per_pos * (ctx0 + i + 1) for i in range(n))
    gbs = total_bytes / dt / 1e9
    toks = out
    # the same decode at top-2 (FORCED_TOP2): fresh cache and prefill
    del gd, cache
    N2 = min(64, N)
    cache2 = model.new_cache(B, P + N2)
    tok2 = model(ids, cache2)[:, -1].argmax(-1, keepdim=True)
    model.decode_top_k = 2
    gd2 = GraphDecoder(model, cache2, tok2)
    for _ in range(min(W, N2 - 2)):
        gd2.step()
    torch.cuda.synchronize()
    n2 = N2 - 1 - min(W, N2 - 2)
    t0 = time.perf_counter()
    for i in range(n2):
        gd2.step()
    torch.cuda.synchronize()
    dt2 = time.perf_counter() - t0
    model.decode_top_k = 1
    del gd2, cache2
    return {"workload": "C5: Mixtral-8x7B-shaped decoder (32 layers, H 4096, 32/8 heads, "
                        "head_dim 128, vocab 32000, 8 INT4 g128 experts per layer resident), "
                        "64 x 512-token random prompts, greedy decode (top-1 routing)",
            "batch": B, "prompt": P, "decode_tokens": N, "timed_forwards": n,
            "ms_per_step": round(dt * 1e3 / n, 4), "tokens_per_s": round(B * n / dt, 1),
            "prefill_s": round(prefill_s, 3), "graph_capture_s": round(capture_s, 3),
            "prefill_tokens_per_s": round(B * P / prefill_s, 1),
            "GB_s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
            "bytes_per_step_avg": int(total_bytes / n),
            "distinct_last_tokens": int(torch.unique(toks[:, -1]).numel()),
            "top2": {"routing": "top-2 at decode (FORCED_TOP2)", "decode_tokens": N2,
                     "timed_forwards": n2, "ms_per_step": round(dt2 * 1e3 / n2, 4),
                     "tokens_per_s": round(B * n2 / dt2, 1)}}


# HBM bytes per launch of the roofline kernel (routing + grouped gate/up stream
# kernel, C2 T=16, 8 active experts): FETCH_SIZE + WRITE_SIZE from two rocprofv3
# --pmc passes over `bench.py --workload c2phase`, each scaled by the same
# counter on a 512 MiB copy.  Commands, raw counter values and scale factors:
# profiles/route_gate_up_c2_t16_traffic.md.  Re-measure after a kernel change.
ROUTE_GATE_UP_C2_T16_TRAFFIC = 487_504_833


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="c2",
                    choices=["c1", "c2", "c3", "c4", "c5", "c1phase", "c2phase", "c4phase",
                             "h2d", "copy"],
                    help="c2phase: only the C2 T=16 routing + gate/up kernel and a 512 MiB copy "
                         "(the two kernels whose rocprofv3 counters give roofline.traffic); "
                         "c4phase: only the C4 grouped GEMM launches (MFMA counters); "
                         "h2d: the expert-miss load path (pinned -> HBM, and from a store "
                         "on disk); copy: torch's device copy and sum rates (HBM reference)")
    ap.add_argument("--tokens", type=int, default=1)
    ap.add_argument("--shared-side-stream", type=int, default=None, choices=[0, 1],
                    help="c3: the shared expert on a second stream (1) or first on the "
                         "layer's stream (0); default: the layer's")
    ap.add_argument("--attn-decode", type=int, default=None, choices=[0, 1],
                    help="c5: decode attention in one launch (1, hn_attn_decode) or the two "
                         "products with the softmax between (0); default: the model's")
    ap.add_argument("--fused-routing", type=int, default=None, choices=[0, 1],
                    help="c3: routing inside the gate/up kernel (1) or its own launch (0); "
                         "default: the layer's")
    ap.add_argument("--decode-tokens", type=int, default=256, help="c5: tokens generated")
    ap.add_argument("--warmup-decode", type=int, default=3, help="c5: untimed decode forwards")
    ap.add_argument("--skip-h2d", action="store_true",
                    help="c2: leave out the expert-miss load path (workload h2d)")
    ap.add_argument("--skip-c5", action="store_true",
                    help="c2: leave out the whole-decoder tokens/s run (workload c5)")
    ap.add_argument("--skip-c34", action="store_true",
                    help="c2: leave out the GLM layer (c3) and prefill (c4) lines")
    ap.add_argument("--cpu-budget", type=float, default=24.0,
                    help="seconds of CPU-baseline work (C2 at T = 1, 4, 16; C1 gets a quarter)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--decode-path", type=int, default=0, choices=[0, 1],
                    help="0: streaming kernels where they apply (default); 1: split-K only")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU only; the INT4 expert path is "
                                   "benchmarked per GPU (with expert parallelism each GPU "
                                   "runs this same grouped path on its own experts)",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    torch.cuda.set_device(0)
    from hydranet_amd import _lib
    _lib.set_decode_path(args.decode_path)
    _log("workload", args.workload, "steps", args.steps, "warmup", args.warmup)
    if args.workload == "c1phase":
        c1phase(args)
        return
    if args.workload == "c2phase":
        c2phase(args)
        return
    if args.workload == "c4phase":
        c4phase(args)
        return
    if args.workload == "h2d":
        r = bench_h2d(args)
        _log("h2d", r)
        print(json.dumps({"metric": "expert H2D load GB/s (residency miss path, 1 GPU)",
                          "value": r["GB_s"], "unit": "GB/s", "n_gpus": 1,
                          "higher_is_better": True, "dtype": "u8", "data": "synthetic",
                          "config": r}), flush=True)
        return
    if args.workload == "copy":
        r = bench_copy(args)
        _log("copy", r)
        print(json.dumps({"metric": "torch device copy GB/s (read + write, HBM reference, 1 GPU)",
                          "value": r["copy_4GiB"]["GB_s"], "unit": "GB/s", "n_gpus": 1,
                          "higher_is_better": True, "dtype": "fp16", "data": "synthetic",
                          "config": r}), flush=True)
        return
    if args.workload == "c3":
        c3 = bench_c3(args)
        _log("c3", c3)
        print(json.dumps({"metric": "INT4 expert-MLP HBM GB/s (GLM-4.5-Air MoE layer decode, "
                                    "1 GPU)", "value": c3["GB_s"], "unit": "GB/s", "n_gpus": 1,
                          "ms_per_step": c3["ms_per_step"], "higher_is_better": True,
                          "dtype": "fp16", "data": "synthetic", "config": c3}), flush=True)
        return
    if args.workload == "c5":
        c5 = bench_c5(args)
        _log("c5", c5)
        print(json.dumps({"metric": "Mixtral-shape decode tokens/sec, 1 GPU", "value":
                          c5["tokens_per_s"], "unit": "tokens/s", "n_gpus": 1,
                          "ms_per_step": c5["ms_per_step"], "higher_is_better": True,
                          "dtype": "fp16", "data": "synthetic", "config": c5}), flush=True)
        return
    if args.workload == "c4":
        c4 = bench_c4(args)
        _log("c4", c4)
        print(json.dumps({"metric": "INT4 expert-MLP prefill TFLOP/s (MoE layer, 1 GPU)",
                          "value": c4["TFLOP_s"], "unit": "TFLOP/s", "n_gpus": 1,
                          "ms_per_step": c4["ms_per_step"], "higher_is_better": True,
                          "dtype": "fp16", "data": "synthetic", "config": c4}), flush=True)
        return
    res, ctx = bench_c1(args)
    _log("c1 done", res["value"], res["unit"])
    c1 = {"GB_s": res["value"], "frac": res["roofline"]["expert_frac"], "target_frac": 0.70,
          "us_per_expert": round(res["ms_per_step"] * 1e3, 2),
          "tokens_per_s": res["tokens_per_s"],
          "kernels": {"gate_up_silu_us": res["roofline"]["avg_us"],
                      "down_us": res["roofline"]["down_avg_us"]}}
    cpu = None
    cpu_c1 = None
    if not args.no_cpu:
        cpu_c1, parity = cpu_baseline_c1(ctx, args.cpu_budget / 4)
        res["parity"] = parity
    if args.workload == "c2":
        sweep, ctxs = {}, {}
        for T in (1, 4, 16):
            sweep[f"T{T}"] = bench_c2(args, T, phases=(T == 16))
            ctxs[f"T{T}"] = sweep[f"T{T}"].pop("_ctx")
            _log("c2", T, sweep[f"T{T}"])
        head = sweep["T16"]
        ph = head.pop("phases", None)
        if ph is not None:
            # roofline of the dominant kernel of the headline workload: the grouped
            # gate/up + SiLU stream kernel over the active experts at T = 16
            gu = ph["route_gate_up_silu"]
            res["c1_roofline"] = res.pop("roofline")
            res["roofline"] = {
                "bound": "hbm",
                "kernel": "stream_kernel<grouped, gate+up+SiLU, routing in the prologue> (C2, T=16)",
                "achieved": gu["GB_s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(gu["GB_s"] / HBM_PEAK_GBS, 4), "traffic": None,
                "traffic_source": None,
                "bytes_per_launch": gu["bytes_per_launch"], "avg_us": gu["avg_us"],
                "down": ph["down_4slices"], "active_experts": ph["active_experts"]}
            # the same bytes read by a plain streaming read: what a launch that
            # only reads them reaches (context for frac, whose peak is nominal)
            rp = read_probe({"gate_up": gu["bytes_per_launch"],
                             "down": ph["down_4slices"]["bytes_per_launch"]})
            res["roofline"]["read_probe"] = {
                **rp["gate_up"], "kernel_over_read": round(rp["gate_up"]["us"] / gu["avg_us"], 3)}
            res["roofline"]["down"]["read_probe"] = {
                **rp["down"],
                "kernel_over_read": round(rp["down"]["us"] / ph["down_4slices"]["avg_us"], 3)}
            if ph["active_experts"] == 8:
                res["roofline"]["traffic"] = ROUTE_GATE_UP_C2_T16_TRAFFIC
                res["roofline"]["traffic_source"] = (
                    "constant from profiles/route_gate_up_c2_t16_traffic.md (rocprofv3 "
                    "FETCH_SIZE + WRITE_SIZE of bench.py --workload c2phase, scaled by a 512 MiB "
                    "copy); not measured in this run")
        if not args.no_cpu:
            cpu = cpu_baseline_c2(ctxs, args.cpu_budget)
            cpu["c1"] = cpu_c1
            _log("cpu baseline", cpu)
        del ctxs
        res["metric"] = METRIC
        res["value"] = head["GB_s"]
        res["ms_per_step"] = head["ms_per_step"]
        res["tokens_per_s"] = head["tokens_per_s"]
        res["config"] = {"workload": "C2: one Mixtral MoE layer at decode (8 experts "
                                     "4096->14336->4096 INT4 g128, softmax top-2), T=16 tokens; "
                                     "router + permute + grouped SwiGLU + unpermute",
                         "tokens": 16, "experts": 8, "top_k": 2, "layers_rotated": 4,
                         "sweep": sweep, "c1_single_expert_T1": c1,
                         "graph": head["graph"]}
        res["c1"] = c1
        if not args.skip_c34:
            torch.cuda.empty_cache()
            c3 = bench_c3(args)
            _log("c3", c3)
            res["c3"] = c3
            torch.cuda.empty_cache()
            c4 = bench_c4(args)
            _log("c4", c4)
            res["c4"] = c4
        if not args.skip_c5:
            # the metric's second half: whole-decoder decode tokens/s (workload c5)
            torch.cuda.empty_cache()
            c5 = bench_c5(args)
            _log("c5", c5)
            res["decoder_tokens_per_s"] = c5["tokens_per_s"]
            res["decoder_tokens_per_s_top2"] = c5["top2"]["tokens_per_s"]
            res["config"]["c5_decoder"] = c5
        if not args.skip_h2d:
            # the residency layer's expert-miss load path (pinned -> HBM, and a
            # store on disk -> HBM), beside the resident-path numbers
            torch.cuda.empty_cache()
            h2d = bench_h2d(args)
            _log("h2d", h2d)
            res["h2d"] = h2d
    else:
        cpu = cpu_c1
    out = {"metric": res.pop("metric"), "value": res.pop("value"), "unit": res.pop("unit"),
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": res.pop("ms_per_step"), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": res.pop("dtype"), "data": "synthetic",
           "config": res.pop("config"), "roofline": res.pop("roofline"), "cpu_baseline": cpu}
    out.update(res)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
