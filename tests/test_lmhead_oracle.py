"""CPU checks of the LM-head oracle (oracle/lmhead.py) against torch's cross_entropy (an
independent routine) and the reference's clamp and ignore rules."""
from __future__ import annotations

import torch
import torch.nn.functional as F

from oracle.lmhead import lmhead_xent


def _inputs(M=40, V=97, D=24, seed=0):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(M, D, generator=g, dtype=torch.float64)
    w = torch.randn(V, D, generator=g, dtype=torch.float64) / D ** 0.5
    t = torch.randint(0, V, (M,), generator=g)
    return h, w, t


def test_matches_cross_entropy_with_ignored_rows():
    h, w, t = _inputs()
    t[::7] = -100
    hl, wl = h.clone().requires_grad_(True), w.clone().requires_grad_(True)
    loss = lmhead_xent(hl, wl, t)
    loss.backward()
    h2, w2 = h.clone().requires_grad_(True), w.clone().requires_grad_(True)
    ref = F.cross_entropy(h2 @ w2.t(), t, ignore_index=-100)
    ref.backward()
    assert torch.allclose(loss, ref, rtol=1e-12)
    assert torch.allclose(hl.grad, h2.grad, rtol=1e-10, atol=1e-14)
    assert torch.allclose(wl.grad, w2.grad, rtol=1e-10, atol=1e-14)


def test_out_of_range_target_reads_logit_zero_and_all_ignored_gives_zero():
    h, w, t = _inputs(seed=1)
    t_bad = t.clone()
    t_bad[3] = w.shape[0] + 5                 # not ignored, out of range: the reference's clamp
    t_zero = t.clone()
    t_zero[3] = 0
    assert torch.allclose(lmhead_xent(h, w, t_bad), lmhead_xent(h, w, t_zero), rtol=1e-14)
    assert lmhead_xent(h, w, torch.full_like(t, -100)).item() == 0.0


def test_gradcheck():
    h, w, t = _inputs(M=5, V=7, D=3, seed=2)
    t[1] = -100
    assert torch.autograd.gradcheck(lambda a, b: lmhead_xent(a, b, t),
                                    (h.requires_grad_(True), w.requires_grad_(True)))
