"""hn_expert_mlp_int4_noalloc (scratch in a static device array) against
hn_expert_mlp_int4 (caller-provided buffers): the same kernels, so the same
bits, on two calls in a row, the second smaller; and the limits rejected
before any GPU work."""
import ctypes

import pytest
import torch


def _expert(H, I, seed):
    from hydranet_amd.preprocess.synthetic import make_expert_slot
    return make_expert_slot(seed, H, I, 128)


def _args(slot):
    from hydranet_amd import _lib
    return [_lib.ptr(getattr(slot, n)) for n in ("gate_packed", "gate_scales", "up_packed",
                                                  "up_scales", "down_packed", "down_scales")]


def test_noalloc_rejects_sizes_beyond_its_scratch():
    from hydranet_amd import _lib
    for T, H, I in ((17, 4096, 14336), (16, 8192, 65536), (-1, 4096, 14336)):
        with pytest.raises(RuntimeError, match="noalloc"):
            _lib.call("hn_expert_mlp_int4_noalloc", None, None, None, None, None, None, None,
                      None, T, H, I, 128, None)


@pytest.mark.gpu
def test_noalloc_matches_expert_mlp_int4():
    from hydranet_amd import _lib
    dev = "cuda:0"
    cases = [(16, 4096, 14336, 11), (3, 4096, 1408, 12)]  # second call smaller
    outs = []
    for T, H, I, seed in cases:
        print(f"[noalloc] T={T} H={H} I={I}", flush=True)
        slot = _expert(H, I, seed)
        x = (torch.randn(T, H, generator=torch.Generator().manual_seed(seed)) * 1.0).half().to(dev)
        ref = torch.empty(T, H, dtype=torch.float16, device=dev)
        h_ws = torch.empty(T, I, dtype=torch.float16, device=dev)
        work = _lib.skinny_workspace(2, T, H, I, 0, dev)
        _lib.call("hn_expert_mlp_int4", _lib.ptr(x), *_args(slot), _lib.ptr(ref), T, H, I, 128,
                  _lib.ptr(h_ws), _lib.ptr(work), work.numel(), _lib.stream())
        got = torch.full((T, H), float("nan"), dtype=torch.float16, device=dev)
        _lib.call("hn_expert_mlp_int4_noalloc", _lib.ptr(x), *_args(slot), _lib.ptr(got), T, H,
                  I, 128, _lib.stream())
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        assert torch.equal(got, ref), (T, H, I)
        outs.append(got)
    # the split-K family uses the workspace's counters and partials
    _lib.set_decode_path(1)
    try:
        T, H, I, seed = 8, 4096, 14336, 13
        slot = _expert(H, I, seed)
        x = torch.randn(T, H, generator=torch.Generator().manual_seed(seed)).half().to(dev)
        ref = torch.empty(T, H, dtype=torch.float16, device=dev)
        h_ws = torch.empty(T, I, dtype=torch.float16, device=dev)
        work = _lib.skinny_workspace(2, T, H, I, 0, dev)
        for _ in range(2):
            _lib.call("hn_expert_mlp_int4", _lib.ptr(x), *_args(slot), _lib.ptr(ref), T, H, I,
                      128, _lib.ptr(h_ws), _lib.ptr(work), work.numel(), _lib.stream())
            got = torch.empty(T, H, dtype=torch.float16, device=dev)
            _lib.call("hn_expert_mlp_int4_noalloc", _lib.ptr(x), *_args(slot), _lib.ptr(got), T,
                      H, I, 128, _lib.stream())
            torch.cuda.synchronize()
            assert torch.equal(got, ref)
    finally:
        _lib.set_decode_path(0)


_CAPTURE_CHILD = r"""
import sys, torch
sys.path.insert(0, {root!r})
from hydranet_amd import _lib
from hydranet_amd.preprocess.synthetic import make_expert_slot
dev = "cuda:0"
T, H, I = 4, 4096, 14336
slot = make_expert_slot(21, H, I, 128)
args = [_lib.ptr(getattr(slot, n)) for n in ("gate_packed", "gate_scales", "up_packed",
                                             "up_scales", "down_packed", "down_scales")]
x = torch.randn(T, H, generator=torch.Generator().manual_seed(22)).half().to(dev)
ref = torch.empty(T, H, dtype=torch.float16, device=dev)
h_ws = torch.empty(T, I, dtype=torch.float16, device=dev)
work = _lib.skinny_workspace(2, T, H, I, 0, dev)
_lib.call("hn_expert_mlp_int4", _lib.ptr(x), *args, _lib.ptr(ref), T, H, I, 128,
          _lib.ptr(h_ws), _lib.ptr(work), work.numel(), _lib.stream())
torch.cuda.synchronize()
out = torch.zeros(T, H, dtype=torch.float16, device=dev)
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    # the process's first noalloc call: symbol lookup and counter clear under capture
    _lib.call("hn_expert_mlp_int4_noalloc", _lib.ptr(x), *args, _lib.ptr(out), T, H, I, 128,
              _lib.stream())
torch.cuda.synchronize()
for rep in range(3):
    out.fill_(float("nan"))
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, ref), ("replay", rep)
    # eager work between replays (the same kernels through caller buffers)
    _lib.call("hn_expert_mlp_int4", _lib.ptr(x), *args, _lib.ptr(ref), T, H, I, 128,
              _lib.ptr(h_ws), _lib.ptr(work), work.numel(), _lib.stream())
    torch.cuda.synchronize()
print("capture ok", flush=True)
"""


@pytest.mark.gpu
def test_noalloc_first_call_under_graph_capture():
    """A fresh process makes its first hn_expert_mlp_int4_noalloc call inside a
    graph capture (the scratch lookup and the counter-clearing kernel are
    recorded then); three replays, with eager calls between them, equal the
    eager hn_expert_mlp_int4 bit for bit."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("[noalloc capture] child process", flush=True)
    r = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD.format(root=root)],
                       capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    assert "capture ok" in r.stdout
