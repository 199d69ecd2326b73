"""The block front end's reference math (test infrastructure only).

* ``trapezoidal`` restates r2/dhammic-ai/src/kernels/trapezoidal.py:3-13 (forward) with the
  wrapper's casts (dt_bias and A_log to the input dtype, :236-237); its gradient is plain autograd.
  ``trapezoidal_grads_closed_form`` restates the reference's own derivation (:28-52) separately, so
  each pins the other.
* ``rope`` restates the eager rotation of rope.py:4-10 (pairs (2k, 2k+1) of the last axis).
* ``inproj_split`` is ``nn.Linear(bias=False)`` followed by ``torch.split`` (inproj_split.py:8-14).

Arithmetic in the dtype of the arguments given (fp64 for pinning).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def trapezoidal(dt_raw, lam_raw, dt_bias, A_log):
    """(dt, dA, beta, gamma) of the trapezoidal rule; dt_bias and A_log cast to dt_raw's dtype."""
    bias = dt_bias.to(dt_raw.dtype)
    alog = A_log.to(dt_raw.dtype)
    dt = F.softplus(dt_raw + bias)
    lam = torch.sigmoid(lam_raw)
    A = -torch.exp(alog)
    dA = dt * A
    return dt, dA, (1.0 - lam) * dt * torch.exp(dA), lam * dt


def trapezoidal_grads_closed_form(dt_raw, lam_raw, dt_bias, A_log, g_dt, g_dA, g_beta, g_gamma):
    """The reference's backward derivation (trapezoidal.py:28-52): (d_dt_raw, d_lam_raw, d_dt_bias, d_A_log)."""
    s = dt_raw + dt_bias
    dt = F.softplus(s)
    sig_s = torch.sigmoid(s)
    lam = torch.sigmoid(lam_raw)
    A = -torch.exp(A_log)
    dA = dt * A
    alpha = torch.exp(dA)
    g_dt_total = g_dt + g_dA * A + g_beta * (1 - lam) * alpha * (1 + dA) + g_gamma * lam
    g_lam = -g_beta * dt * alpha + g_gamma * dt
    g_A = g_dA * dt + g_beta * (1 - lam) * dt * dt * alpha
    d_dt_raw = g_dt_total * sig_s
    d_lam_raw = g_lam * lam * (1 - lam)
    H = dt_raw.shape[-1]
    return d_dt_raw, d_lam_raw, d_dt_raw.reshape(-1, H).sum(0), (g_A * A).reshape(-1, H).sum(0)


def rope(x, angles):
    """Rotate the pairs (x[..., 2k], x[..., 2k+1]) by angles[..., k] (broadcast over heads if shared)."""
    x1, x2 = x[..., 0::2], x[..., 1::2]
    c, s = torch.cos(angles), torch.sin(angles)
    return torch.stack([c * x1 - s * x2, s * x1 + c * x2], dim=-1).flatten(-2)


def inproj_split(x, weight, split_sizes):
    return torch.split(F.linear(x, weight), list(split_sizes), dim=-1)
