"""GPU tests of the split reductions' last-arriver counters (tagged 64-bit
words, hn_arrive in csrc/hn_common.h) on the two kernels that use them: the
skinny GEMV's split-K (decode family 1, activations too large for one
workgroup's LDS) and the prefill GEMM's stream-K.

A counter left dirty by a launch stopped part-way is simulated from the host:
the test writes a count of 3 (tag 0, the value an untagged counter would keep)
into every counter word of the workspace.  The next launch reclaims each word
it uses with its own tag, so its result equals the clean workspace's bit for
bit, and it leaves the words it used at zero.  A captured graph replays with
its capture-time tag: replays, with eager launches of the same shape between
them, equal the eager result."""
import pytest
import torch

from hydranet_amd import _lib
from hydranet_amd.kernels import int4_gemm as g

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
SKINNY_CTR_WORDS = (2 << 20) // 8   # the skinny workspace's counter region
GEMM_CTR_WORDS = 1 << 16            # the stream-K workspace's counter region


def _operands(M, N, K, seed):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    w = torch.randn(N, K, device=DEV, dtype=torch.float16, generator=gen) * 0.02
    q, s = g.quantize_int4(w, 128)
    x = torch.randn(M, K, device=DEV, dtype=torch.float16, generator=gen)
    return x, q, s


def _dirty(ws, words):
    ctr = ws[:words * 8].view(torch.int64)
    ctr.fill_(3)
    return ctr


@pytest.fixture
def family1():
    _lib.set_decode_path(1)
    yield
    _lib.set_decode_path(0)


def test_skinny_split_k_heals_dirty_counters(family1):
    M, N, K = 64, 1024, 14336
    print(f"[ctr] skinny split-K M={M} N={N} K={K}", flush=True)
    x, q, s = _operands(M, N, K, 1)
    clean = g.int4_linear(x, q, s, 128)
    ws = _lib.skinny_workspace(0, M, N, K, 0, x.device)
    ctr = _dirty(ws, SKINNY_CTR_WORDS)
    again = g.int4_linear(x, q, s, 128)
    torch.cuda.synchronize()
    assert torch.equal(again, clean)
    tiles = N // 16
    assert int(ctr[:tiles].abs().sum()) == 0, "a launch leaves its counters at zero"
    assert bool((ctr[tiles:] == 3).all()), "counters the launch did not use are untouched"
    ref = x.float() @ g.dequantize_int4(q, s, 128).float().t()
    assert bool(((clean.float() - ref).abs() <= 1e-2 + 2e-3 * ref.abs()).all())


def _gate_up(x, gq, gs, uq, us, ws):
    M, H = x.shape
    I = gq.shape[0]
    h = torch.empty(M, I, device=DEV, dtype=torch.float16)
    _lib.call("hn_int4_gate_up_silu", _lib.ptr(x), H, _lib.ptr(gq), _lib.ptr(gs), _lib.ptr(uq),
              _lib.ptr(us), gq.stride(0), gs.stride(0), _lib.ptr(h), I, M, I, H, 128,
              _lib.ptr(ws), ws.numel(), _lib.stream(x.device))
    return h


def test_skinny_gate_up_split_k_heals_dirty_counters(family1):
    M, I, H = 48, 512, 14336
    print(f"[ctr] skinny gate/up split-K M={M} I={I} H={H}", flush=True)
    x, gq, gs = _operands(M, I, H, 2)
    _, uq, us = _operands(1, I, H, 3)
    ws = _lib.skinny_workspace(1, M, I, H, 0, x.device)
    clean = _gate_up(x, gq, gs, uq, us, ws)
    _dirty(ws, SKINNY_CTR_WORDS)
    again = _gate_up(x, gq, gs, uq, us, ws)
    torch.cuda.synchronize()
    assert torch.equal(again, clean)
    deq = lambda q_, s_: g.dequantize_int4(q_, s_, 128).float().t()
    gr, ur = (x.float() @ deq(gq, gs)).half().float(), (x.float() @ deq(uq, us)).half().float()
    ref = torch.nn.functional.silu(gr).half().float() * ur
    assert bool(((clean.float() - ref).abs() <= 1e-2 + 2e-3 * ref.abs()).all())


def test_stream_k_heals_dirty_counters():
    M, N, K = 512, 1024, 4096
    print(f"[ctr] stream-K M={M} N={N} K={K}", flush=True)
    x, q, s = _operands(M, N, K, 4)
    clean = g.int4_linear(x, q, s, 128)
    ws = _lib.gemm_workspace(x.device)
    ctr = _dirty(ws, GEMM_CTR_WORDS)
    again = g.int4_linear(x, q, s, 128)
    torch.cuda.synchronize()
    assert torch.equal(again, clean)
    assert int((ctr == 3).sum()) < GEMM_CTR_WORDS, "the launch used (and reset) counters"
    ref = x.float() @ g.dequantize_int4(q, s, 128).float().t()
    assert bool(((clean.float() - ref).abs() <= 1e-2 + 2e-3 * ref.abs()).all())


@pytest.mark.parametrize("M,K", [(64, 14336), (512, 4096)])
def test_split_reductions_replay_in_a_graph(M, K, family1):
    N = 1024
    print(f"[ctr] graph replay M={M} N={N} K={K}", flush=True)
    x, q, s = _operands(M, N, K, 5)
    eager = g.int4_linear(x, q, s, 128)
    out = torch.empty_like(eager)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        g.int4_linear(x, q, s, 128)   # warm-up on the capture stream
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            out.copy_(g.int4_linear(x, q, s, 128))
    torch.cuda.current_stream().wait_stream(stream)
    for rep in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep}"
        assert torch.equal(g.int4_linear(x, q, s, 128), eager)
