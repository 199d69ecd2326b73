"""The extended SSD operator, defined by composition (test infrastructure only).

No single reference function computes this; it is the composition the
caller performs around the reference op (r2/dhammic-ai/src/mamba_base_engine.py:
152-191: zero-pad to a chunk multiple :154-165, SSD :170, ``+ D*x`` :187,
``norm(y) * silu(z)`` :191 with FusedRMSNormModule eps 1e-6,
r2/dhammic-ai/src/kernels/rmsnorm.py:222-235) plus the Mamba-2 discretisation
(X = dt*x, a = dt*A_h) and grouped B/C (head h reads group h // (H/G)).

Packed variable-length input is defined as the SSD run per sequence
[cu[i], cu[i+1]) with that sequence's own initial and final state; each
sequence is zero-padded on the right to a chunk multiple, which is exact
(padded tokens have X = 0 and a = 0).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .ssd_chunked import ssd_forward_impl


def gated_rmsnorm(y, z, weight, eps):
    """out = y * rsqrt(mean(y^2 over the last dim) + eps) * weight * silu(z)."""
    r = torch.rsqrt(y.pow(2).mean(dim=-1, keepdim=True) + eps)
    return y * r * weight * F.silu(z)


def _ssd_one(X, a, Bh, Ch, chunk, init):
    T = X.shape[1]
    pad = (chunk - T % chunk) % chunk
    if pad:
        X = F.pad(X, (0, 0, 0, 0, 0, pad))
        a = F.pad(a, (0, 0, 0, pad))
        Bh = F.pad(Bh, (0, 0, 0, 0, 0, pad))
        Ch = F.pad(Ch, (0, 0, 0, 0, 0, pad))
    Y, final, _ = ssd_forward_impl(X, a, Bh, Ch, chunk,
                                   None if init is None else init.unsqueeze(1))
    return Y[:, :T], final


def ssd_combined(x, dt, A, B, C, chunk_size, D=None, z=None, norm_weight=None,
                 norm_eps=1e-6, initial_states=None, cu_seqlens=None):
    """x (b,L,H,P), dt (b,L,H) (already positive), A (H,), B/C (b,L,G,N),
    D (H,), z (b,L,H,P), norm_weight (H*P,), initial_states (nseq,H,P,N),
    cu_seqlens (nseq+1,) ints with b == 1.

    Returns (out (b,L,H,P), final_states (nseq,H,P,N)); nseq = b without
    cu_seqlens.
    """
    b, L, H, P = x.shape
    G = B.shape[2]
    assert H % G == 0
    X = x * dt.unsqueeze(-1)
    a = dt * A.view(1, 1, H)
    Bh = B.repeat_interleave(H // G, dim=2)
    Ch = C.repeat_interleave(H // G, dim=2)
    if cu_seqlens is None:
        Y, final = _ssd_one(X, a, Bh, Ch, chunk_size, initial_states)
    else:
        assert b == 1
        cu = [int(v) for v in cu_seqlens]
        ys, finals = [], []
        for i in range(len(cu) - 1):
            s, e = cu[i], cu[i + 1]
            init = None if initial_states is None else initial_states[i:i + 1]
            y_i, f_i = _ssd_one(X[:, s:e], a[:, s:e], Bh[:, s:e], Ch[:, s:e], chunk_size, init)
            ys.append(y_i)
            finals.append(f_i)
        Y = torch.cat(ys, dim=1)
        final = torch.cat(finals, dim=0)
    if D is not None:
        Y = Y + x * D.view(1, 1, H, 1)
    if z is not None:
        w = norm_weight if norm_weight is not None else torch.ones(H * P, dtype=Y.dtype, device=Y.device)
        Y = gated_rmsnorm(Y.reshape(b, L, H * P), z.reshape(b, L, H * P), w, norm_eps)
        Y = Y.reshape(b, L, H, P)
    return Y, final
