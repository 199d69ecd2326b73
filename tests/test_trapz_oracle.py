"""CPU checks of the trapezoidal two-SSD oracle (oracle/trapezoidal.py) and of the identity the
native single-scan form rests on.

* two_call_ssd (the reference block's two chunked calls with the cache) against
  two_path_sequential (two fp64 token recurrences, the beta path's decay detached unless
  exact): outputs and every gradient, in both gradient settings, on a ragged length.
* The cache really drops the beta path's decay gradient: the two settings' dA differ, and only
  dA does.
* The fold: SSD((gamma + rho) x, a, B, C) - rho (C.B) x with rho[t] = beta[t+1] exp(-a[t+1])
  equals the pair exactly (what csrc/ssd_trapz.hip computes).
"""
from __future__ import annotations

import pytest
import torch

from oracle.ssd_sequential import ssd_sequential
from oracle.trapezoidal import two_call_ssd, two_path_sequential


def _inputs(b=2, T=40, H=2, P=3, N=4, seed=0):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)  # noqa: E731
    x = r(b, T, H, P)
    dt = torch.nn.functional.softplus(r(b, T, H) - 1.0)
    A = -torch.exp(torch.empty(H, dtype=torch.float64).uniform_(-2.0, 0.0, generator=g))
    lam = torch.sigmoid(r(b, T, H))
    dA = dt * A
    gamma = lam * dt                              # trapezoidal.py:7-13
    beta = (1.0 - lam) * dt * torch.exp(dA)
    B, C = r(b, T, H, N), r(b, T, H, N)
    return x, dA, gamma, beta, B, C


def _grads(fn, ins, seed=1):
    leaves = [t.detach().clone().requires_grad_(True) for t in ins]
    y = fn(*leaves)
    dy = torch.randn(y.shape, generator=torch.Generator().manual_seed(seed), dtype=y.dtype)
    gs = torch.autograd.grad(y, leaves, dy, allow_unused=True)
    return y.detach(), [torch.zeros_like(l) if gi is None else gi for l, gi in zip(leaves, gs)]


@pytest.mark.parametrize("exact", [False, True], ids=["drop_beta_dA", "exact_dA"])
def test_two_calls_equal_two_recurrences(exact):
    ins = _inputs()
    y1, g1 = _grads(lambda *t: two_call_ssd(*t, chunk_size=16, exact_beta_dA=exact), ins)
    y2, g2 = _grads(lambda *t: two_path_sequential(*t, exact_beta_dA=exact), ins)
    # the chunked calls keep the reference's acausal e^-20 entries: <= 2.1e-9 * sum |terms| per output
    assert torch.allclose(y1, y2, rtol=0, atol=1e-6)
    for name, a, b in zip(("x", "dA", "gamma", "beta", "B", "C"), g1, g2):
        assert (a - b).abs().max() <= 1e-7 * b.abs().max(), name


def test_cache_drops_only_the_beta_decay_gradient():
    ins = _inputs(seed=3)
    _, g_drop = _grads(lambda *t: two_call_ssd(*t, chunk_size=16), ins)
    _, g_exact = _grads(lambda *t: two_call_ssd(*t, chunk_size=16, exact_beta_dA=True), ins)
    for name, a, b in zip(("x", "dA", "gamma", "beta", "B", "C"), g_drop, g_exact):
        d = (a - b).abs().max().item()
        if name == "dA":
            assert d > 1e-3 * b.abs().max().item(), "the beta path's decay gradient was not dropped"
        else:
            assert d < 1e-12 * max(1.0, b.abs().max().item()), name


def test_fold_into_one_scan():
    """The pair = SSD((gamma + rho) x) - rho (C.B) x, rho[t] = beta[t+1] exp(-a[t+1]), rho[T-1] = 0."""
    x, dA, gamma, beta, B, C = _inputs(T=33, seed=5)
    rho = torch.zeros_like(gamma)
    rho[:, :-1] = beta[:, 1:] * torch.exp(-dA[:, 1:])
    y_one, _ = ssd_sequential(x * (gamma + rho).unsqueeze(-1), dA, B, C)
    y_one = y_one - (rho * (B * C).sum(-1)).unsqueeze(-1) * x
    y_pair = two_path_sequential(x, dA, gamma, beta, B, C)
    assert torch.allclose(y_one, y_pair, rtol=0, atol=1e-11)
    # planted slip: rho without the exp(-a) factor breaks it
    rho_bad = torch.zeros_like(gamma)
    rho_bad[:, :-1] = beta[:, 1:]
    y_bad, _ = ssd_sequential(x * (gamma + rho_bad).unsqueeze(-1), dA, B, C)
    y_bad = y_bad - (rho_bad * (B * C).sum(-1)).unsqueeze(-1) * x
    assert (y_bad - y_pair).abs().max() > 1e-3


def test_packed_sequences_restart_the_shift():
    x, dA, gamma, beta, B, C = _inputs(b=1, T=45, seed=7)
    cu = [0, 17, 17, 45]
    y = two_call_ssd(x, dA, gamma, beta, B, C, 16, cu_seqlens=cu)
    parts = [two_path_sequential(x[:, s:e], dA[:, s:e], gamma[:, s:e], beta[:, s:e], B[:, s:e], C[:, s:e])
             for s, e in zip(cu[:-1], cu[1:]) if e > s]
    assert torch.allclose(y, torch.cat(parts, dim=1), rtol=0, atol=1e-6)
