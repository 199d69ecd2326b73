"""Seeded synthetic inputs with the distributions the benchmark configs name.

x, dy ~ N(0,1); dt = clamp(softplus(N(0,1) - 4), 1e-3, 0.1); A = -exp(U(0, ln 16));
B, C ~ N(0,1)/sqrt(N); D ~ N(0,1); z ~ N(0,1); init ~ N(0, 0.1^2); dfinal ~ N(0,1).
Drawn in that fixed order from one torch.Generator, in fp32 on ``device``.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F


@dataclass
class SsdShape:
    batch: int
    seqlen: int
    nheads: int
    headdim: int
    ngroups: int
    dstate: int
    chunk: int
    cu_seqlens: list = field(default=None)

    @property
    def nseq(self):
        return self.batch if self.cu_seqlens is None else len(self.cu_seqlens) - 1


# The benchmark configurations (config 3's sequence lengths are drawn by
# varlen_lengths below).
CONFIG0 = SsdShape(1, 512, 4, 32, 1, 32, 64)
CONFIG1 = SsdShape(8, 2048, 24, 64, 1, 128, 256)
CONFIG2 = SsdShape(4, 8192, 64, 64, 1, 128, 256)


def varlen_lengths(total, lo=512, hi=8192, seed=3):
    """Lengths ~ U{lo..hi} drawn until their sum reaches ``total``; the last one
    is trimmed so they sum to exactly ``total``."""
    g = torch.Generator().manual_seed(seed)
    lens, acc = [], 0
    while acc < total:
        v = int(torch.randint(lo, hi + 1, (1,), generator=g))
        v = min(v, total - acc)
        lens.append(v)
        acc += v
    return lens


def config3_shape():
    lens = varlen_lengths(65536)
    cu = [0]
    for v in lens:
        cu.append(cu[-1] + v)
    return SsdShape(1, 65536, 32, 64, 8, 64, 256, cu_seqlens=cu)


def make_inputs(shape: SsdShape, seed=0, device="cpu", with_z=False, with_init=False,
                with_dfinal=False):
    g = torch.Generator(device=device).manual_seed(seed)
    b, L, H, P, G, N = (shape.batch, shape.seqlen, shape.nheads, shape.headdim,
                        shape.ngroups, shape.dstate)
    kw = dict(generator=g, device=device, dtype=torch.float32)
    out = {}
    out["x"] = torch.randn(b, L, H, P, **kw)
    out["dt"] = F.softplus(torch.randn(b, L, H, **kw) - 4.0).clamp(1e-3, 0.1)
    out["A"] = -torch.exp(torch.rand(H, **kw) * math.log(16.0))
    out["B"] = torch.randn(b, L, G, N, **kw) / math.sqrt(N)
    out["C"] = torch.randn(b, L, G, N, **kw) / math.sqrt(N)
    out["D"] = torch.randn(H, **kw)
    out["dy"] = torch.randn(b, L, H, P, **kw)
    if with_z:
        out["z"] = torch.randn(b, L, H, P, **kw)
    if with_init:
        out["init"] = torch.randn(shape.nseq, H, P, N, **kw) * 0.1
    if with_dfinal:
        out["dfinal"] = torch.randn(shape.nseq, H, P, N, **kw)
    return out


def make_reference_test_inputs(b, seqlen, n_heads, d_head, d_state, seed=0, dtype=torch.float32):
    """The reference test's input recipe (r2/dhammic-ai/tests/kernels/test_ssd_scan.py:31-39),
    drawn here on CPU: x*0.5, A = -U*0.1 per token, B and C * 0.5."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(b, seqlen, n_heads, d_head, generator=g, dtype=dtype) * 0.5
    A = -torch.rand(b, seqlen, n_heads, generator=g, dtype=dtype) * 0.1
    B = torch.randn(b, seqlen, n_heads, d_state, generator=g, dtype=dtype) * 0.5
    C = torch.randn(b, seqlen, n_heads, d_state, generator=g, dtype=dtype) * 0.5
    return x, A, B, C
