"""HIP graph capture of one forward + backward step of the fused scan.

The C ABI runs on the caller's stream, allocates nothing itself (the wrapper allocates with torch, which
draws from the graph's private pool during capture), makes no host synchronisation and records no memset,
so a step can be captured. The test captures one step with `torch.cuda.graph`, then replays it three times.
Before each replay, eager kernels write new inputs into the captured tensors, followed by a synchronisation.
Every output of every replay is compared bit for bit with an eager step on the same inputs: the kernels are
deterministic, so a replay that reads stale inputs, skips a node or races shows as a difference.
"""
from __future__ import annotations

import math

import pytest
import torch

from conftest import gpu_available

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not gpu_available(), reason="needs an MI355X (HIP device)")]

BF = torch.bfloat16


def _fill(t, g, dev):
    """New values for the captured inputs, drawn with eager kernels into the same storage."""
    b, L, H, P = t["x"].shape
    G, N = t["B"].shape[2:]
    kw = dict(generator=g, device=dev, dtype=torch.float32)
    t["x"].copy_(torch.randn(b, L, H, P, **kw))
    t["dt"].copy_(torch.nn.functional.softplus(torch.randn(b, L, H, **kw) - 4.0).clamp(1e-3, 0.1))
    t["A"].copy_(-torch.exp(torch.rand(H, **kw) * math.log(16.0)))
    t["B"].copy_(torch.randn(b, L, G, N, **kw) / math.sqrt(N))
    t["C"].copy_(torch.randn(b, L, G, N, **kw) / math.sqrt(N))
    t["D"].copy_(torch.randn(H, **kw))
    t["z"].copy_(torch.randn(b, L, H, P, **kw))
    t["w"].copy_(1.0 + 0.1 * torch.randn(H * P, **kw))
    t["init"].copy_(0.1 * torch.randn(b, H, P, N, **kw))
    t["dy"].copy_(torch.randn(b, L, H, P, **kw))
    t["dfinal"].copy_(torch.randn(b, H, P, N, **kw))


def test_graph_replays_match_eager():
    from kernels import _capi as C_
    from kernels import ssd_scan as S

    dev = torch.device("cuda", 0)
    b, L, H, P, G, N, Q = 2, 1024, 8, 64, 2, 64, 256
    t = {
        "x": torch.empty(b, L, H, P, device=dev, dtype=BF), "dt": torch.empty(b, L, H, device=dev),
        "A": torch.empty(H, device=dev), "B": torch.empty(b, L, G, N, device=dev, dtype=BF),
        "C": torch.empty(b, L, G, N, device=dev, dtype=BF), "D": torch.empty(H, device=dev),
        "z": torch.empty(b, L, H, P, device=dev, dtype=BF), "w": torch.empty(H * P, device=dev),
        "init": torch.empty(b, H, P, N, device=dev), "dy": torch.empty(b, L, H, P, device=dev, dtype=BF),
        "dfinal": torch.empty(b, H, P, N, device=dev),
    }
    g = torch.Generator(device=dev).manual_seed(11)
    cfg = S._Cfg(chunk=Q, a_mode=C_.SSD_A_PER_HEAD, nseq=b, varlen=False, state_code=C_.SSD_DTYPE_F32,
                 want_acs=False, eps=1e-6)

    def step(inp):
        y, final, _, saved = S._forward(cfg, inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], inp["z"],
                                        inp["w"], inp["init"], None)
        grads = S._backward(cfg, saved, inp["x"], inp["dt"], inp["A"], inp["B"], inp["C"], inp["D"], inp["z"],
                            inp["w"], inp["init"], None, inp["dy"], inp["dfinal"])
        out = {"y": y, "final": final}
        out.update({"d" + k: v for k, v in grads.items() if v is not None})
        return out

    _fill(t, g, dev)
    side = torch.cuda.Stream()  # default priority
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step(t)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step(t)
    torch.cuda.synchronize()
    assert len(captured) >= 10, sorted(captured)

    for rep in range(3):
        _fill(t, g, dev)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eager = step({k: v.clone() for k, v in t.items()})
        torch.cuda.synchronize()
        assert sorted(eager) == sorted(captured)
        for k in eager:
            assert torch.isfinite(eager[k].float()).all(), (rep, k)
            assert torch.equal(captured[k], eager[k]), (rep, k, (captured[k].float() - eager[k].float()).abs().max())
