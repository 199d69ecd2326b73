"""The LM head + cross-entropy the fused kernel computes (test infrastructure only).

Restates r2/dhammic-ai/src/kernels/lmhead_xent.py:1-45 and its forward kernel (:75-140):
logits = hidden weight^T in the dtype given (the reference multiplies in fp32), logZ per row,
the target logit with the clamp of :101-103 (a target that is not ignore_index but outside
[0, V) reads logit 0), and the mean of (logZ - target_logit) over the non-ignored rows
(:300-302, at least one row in the divisor). Gradients by autograd.
"""
from __future__ import annotations

import torch


def lmhead_xent(hidden, weight, targets, ignore_index=-100):
    D = hidden.shape[-1]
    h = hidden.reshape(-1, D)
    t = targets.reshape(-1)
    V = weight.shape[0]
    logits = h @ weight.t()
    valid = t != ignore_index
    te = torch.where(valid & (t >= 0) & (t < V), t, torch.zeros_like(t))
    logZ = torch.logsumexp(logits, dim=-1)
    tl = logits.gather(1, te.unsqueeze(1)).squeeze(1)
    m = valid.to(logits.dtype)
    return ((logZ - tl) * m).sum() / m.sum().clamp_min(1.0)
