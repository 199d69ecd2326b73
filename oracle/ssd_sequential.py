"""Brute-force token-by-token SSD recurrence (test infrastructure only).

The exact operator without chunking or clamps:
    h_t = exp(a_t) * h_{t-1} + X_t (outer) B_t,    y_t = h_t @ C_t
which is what stream/ces/ssd_reference/extract.py:13-63 and
stream/ces/ces-ssm/src/lib.rs:255-299 compute (there with P = 1 and the
discretisation dt = softplus(dt + dt_bias), X = dt * x, a = dt * A).

Differentiable (plain autograd through the loop), so it also serves as an
independent check of the chunked oracle's backward on small shapes.
"""
from __future__ import annotations

import math

import torch


def ssd_sequential(X, a, B, C, initial_states=None):
    """X (b,T,h,p), a (b,T,h), B/C (b,T,h,n), initial_states (b,h,p,n) or None.

    Returns (Y (b,T,h,p), final_state (b,h,p,n)).
    """
    b, T, h, p = X.shape
    n = B.shape[-1]
    state = (torch.zeros(b, h, p, n, dtype=X.dtype) if initial_states is None
             else initial_states)
    ys = []
    for t in range(T):
        state = torch.exp(a[:, t])[..., None, None] * state \
            + X[:, t].unsqueeze(-1) * B[:, t].unsqueeze(-2)
        ys.append(torch.einsum("bhpn,bhn->bhp", state, C[:, t]))
    return torch.stack(ys, dim=1), state


def softplus_scalar(v):
    return math.log(math.exp(v) + 1.0)


def ces_scalar_reference(x, a, b, c, dt, d, dt_bias, batch, seq_len, n_heads, d_state):
    """Pure-Python scalar loop with the ces-ssm test's exact iteration order
    (lib.rs:255-299): flat row-major lists in, flat list y (batch,seq,heads) out."""
    out = [0.0] * (batch * seq_len * n_heads)
    state = [0.0] * (batch * n_heads * d_state)
    for t in range(seq_len):
        for bi in range(batch):
            for hh in range(n_heads):
                idx = (bi * seq_len + t) * n_heads + hh
                step = dt[idx] + (dt_bias[hh] if dt_bias is not None else 0.0)
                step = softplus_scalar(step)
                decay = math.exp(step * a[hh])
                xv = x[idx]
                acc = 0.0
                for k in range(d_state):
                    i_btn = idx * d_state + k
                    i_bhn = (bi * n_heads + hh) * d_state + k
                    state[i_bhn] = decay * state[i_bhn] + step * b[i_btn] * xv
                    acc += c[i_btn] * state[i_bhn]
                out[idx] = acc + d[hh] * xv
    return out
