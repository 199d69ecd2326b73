"""CPU checks of the front-end oracle (oracle/frontend.py): the trapezoidal forward against its
identities and the reference's own closed-form backward (trapezoidal.py:28-52) against autograd;
the rotary embedding's group properties; the in-projection split's views."""
from __future__ import annotations

import math

import torch

from oracle.frontend import inproj_split, rope, trapezoidal, trapezoidal_grads_closed_form


def _trapz_inputs(seed=0, rows=37, H=5):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)  # noqa: E731
    return r(rows, H), r(rows, H), 0.1 * r(H), r(H).clamp(-4, 1)


def test_trapezoidal_identities():
    dt_raw, lam_raw, bias, alog = _trapz_inputs()
    dt, dA, beta, gamma = trapezoidal(dt_raw, lam_raw, bias, alog)
    lam = torch.sigmoid(lam_raw)
    assert (dt > 0).all()
    assert torch.allclose(dt, torch.log1p(torch.exp(dt_raw + bias)), rtol=1e-12)
    assert torch.allclose(dA, -dt * torch.exp(alog), rtol=1e-12)
    # beta exp(-dA) + gamma = dt: the two weights of the rule split dt by lam
    assert torch.allclose(beta * torch.exp(-dA) + gamma, dt, rtol=1e-12)
    assert torch.allclose(gamma, lam * dt, rtol=1e-12)


def test_trapezoidal_closed_form_backward_matches_autograd():
    ins = [t.requires_grad_(True) for t in _trapz_inputs(seed=1)]
    outs = trapezoidal(*ins)
    g = torch.Generator().manual_seed(2)
    gs = [torch.randn(o.shape, generator=g, dtype=torch.float64) for o in outs]
    auto = torch.autograd.grad(outs, ins, gs)
    closed = trapezoidal_grads_closed_form(*[t.detach() for t in ins], *gs)
    for a, c in zip(auto, closed):
        assert torch.allclose(a, c, rtol=1e-10, atol=1e-12)
    # planted slip: the beta path's (1 + dA) factor dropped from d(dt) changes d_dt_raw
    lam = torch.sigmoid(ins[1].detach())
    dt, dA, _, _ = [o.detach() for o in outs]
    slip = gs[2] * (1 - lam) * torch.exp(dA) * dA * torch.sigmoid(ins[0].detach() + ins[2].detach())
    assert slip.abs().max() > 1e-3


def test_trapezoidal_gradcheck():
    ins = [t.requires_grad_(True) for t in _trapz_inputs(seed=3, rows=6, H=3)]
    assert torch.autograd.gradcheck(lambda *t: trapezoidal(*t), ins)


def test_rope_group_properties():
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 7, 3, 8, generator=g, dtype=torch.float64)
    a = torch.randn(2, 7, 3, 4, generator=g, dtype=torch.float64)
    b = torch.randn(2, 7, 3, 4, generator=g, dtype=torch.float64)
    assert torch.allclose(rope(x, torch.zeros_like(a)), x)
    assert torch.allclose(rope(rope(x, a), b), rope(x, a + b))           # rotations compose
    assert torch.allclose(rope(rope(x, a), -a), x)                        # and invert
    pn = lambda t: t[..., 0::2] ** 2 + t[..., 1::2] ** 2  # noqa: E731
    assert torch.allclose(pn(rope(x, a)), pn(x))                         # pair norms kept
    q = rope(x, torch.full_like(a, math.pi / 2))                          # a quarter turn: (x1, x2) -> (-x2, x1)
    assert torch.allclose(q[..., 0::2], -x[..., 1::2]) and torch.allclose(q[..., 1::2], x[..., 0::2])
    shared = a[:, :, :1]
    assert torch.allclose(rope(x, shared), rope(x, shared.expand_as(a)))  # shared angles broadcast over heads
    x.requires_grad_(True)
    a.requires_grad_(True)
    assert torch.autograd.gradcheck(rope, (x[:1, :2], a[:1, :2]))


def test_inproj_split_views():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 3, 6, generator=g, dtype=torch.float64)
    w = torch.randn(11, 6, generator=g, dtype=torch.float64)
    parts = inproj_split(x, w, [4, 4, 2, 1])
    assert [p.shape[-1] for p in parts] == [4, 4, 2, 1]
    assert torch.allclose(torch.cat(parts, -1), x @ w.t())
