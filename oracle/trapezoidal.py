"""The trapezoidal block's two SSD calls (test infrastructure only).

``two_call_ssd`` restates the SSD section of ``Mamba3Block._forward_impl``
(r2/dhammic-ai/src/mamba_base_engine.py:152-191) over ``ssd_chunked.fused_ssd_scan``:
zero-pad to a chunk multiple (:154-165), the gamma call on ``x * gamma`` (:170-173), the
one-token shift of B and x (:175-176), the beta call on ``x_prev * beta`` with ``B_prev``
reusing the gamma call's cache (:177-181), the sum cut back to T (:183), ``+ x * D`` (:187) and
``norm(y) * silu(z)`` (:190-191; RMSNorm eps 1e-6, rmsnorm.py:222-235). With
``exact_beta_dA`` the beta call takes no cache, so its decay also feeds dA (the complete
gradient; the reference's cached call drops it, ssd_scan.py:476-533). ``cu_seqlens`` runs the
block per packed sequence (the reference has no packed form; this is its definition here).

``two_path_sequential`` is the same operator as two token-by-token recurrences in fp64 (no
chunks, no clamps): h_g[t] = e^a[t] h_g[t-1] + gamma[t] x[t] B[t]^T and
h_b[t] = e^a[t] h_b[t-1] + beta[t] x[t-1] B[t-1]^T, y[t] = C[t] (h_g[t] + h_b[t]). Without
``exact_beta_dA`` the beta path's decay is detached, which is what the cache does. It pins
``two_call_ssd`` independently of the chunked formulation.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .ssd_chunked import fused_ssd_scan
from .ssd_extended import gated_rmsnorm


def _shift(t):
    """t[:, s] -> t[:, s - 1] along the token axis, zero at s = 0 (mamba_base_engine.py:175-176)."""
    return F.pad(t[:, :-1], (0, 0) * (t.dim() - 2) + (1, 0))


def _block(x, dA, gamma, beta, B, C, chunk, exact_beta_dA, storage):
    T = x.shape[1]
    pad = (chunk - T % chunk) % chunk
    if pad:
        x = F.pad(x, (0, 0, 0, 0, 0, pad))
        dA = F.pad(dA, (0, 0, 0, pad))
        B = F.pad(B, (0, 0, 0, 0, 0, pad))
        C = F.pad(C, (0, 0, 0, 0, 0, pad))
        gamma = F.pad(gamma, (0, 0, 0, pad))
        beta = F.pad(beta, (0, 0, 0, pad))
    y_g, _, cache = fused_ssd_scan(x * gamma.unsqueeze(-1), dA, B, C, chunk, storage=storage)
    y_b, _, _ = fused_ssd_scan(_shift(x) * beta.unsqueeze(-1), dA, _shift(B), C, chunk,
                               cache=None if exact_beta_dA else cache, storage=storage)
    return (y_g + y_b)[:, :T]


def two_call_ssd(x, dA, gamma, beta, B, C, chunk_size, D=None, z=None, norm_weight=None, norm_eps=1e-6,
                 exact_beta_dA=False, cu_seqlens=None, storage=None):
    """x (b,T,H,P); dA, gamma, beta (b,T,H); B, C (b,T,G,N) (head h reads group h // (H/G));
    D (H,); z (b,T,H,P); norm_weight (H*P,). Returns y (b,T,H,P)."""
    b, T, H, P = x.shape
    G = B.shape[2]
    Bh = B.repeat_interleave(H // G, dim=2)
    Ch = C.repeat_interleave(H // G, dim=2)
    if cu_seqlens is None:
        y = _block(x, dA, gamma, beta, Bh, Ch, int(chunk_size), exact_beta_dA, storage)
    else:
        cu = [int(v) for v in cu_seqlens]
        y = torch.cat([_block(x[:, s:e], dA[:, s:e], gamma[:, s:e], beta[:, s:e], Bh[:, s:e], Ch[:, s:e],
                              int(chunk_size), exact_beta_dA, storage)
                       for s, e in zip(cu[:-1], cu[1:]) if e > s], dim=1)
    if D is not None:
        y = y + x * D.view(1, 1, H, 1)
    if z is not None:
        w = norm_weight if norm_weight is not None else torch.ones(H * P, dtype=y.dtype, device=y.device)
        y = gated_rmsnorm(y.reshape(b, T, H * P), z.reshape(b, T, H * P), w, norm_eps).reshape(b, T, H, P)
    return y


def two_path_sequential(x, dA, gamma, beta, B, C, exact_beta_dA=False):
    """The pair of recurrences (no chunks, no clamps), y (b,T,H,P); B, C per head (b,T,H,N)."""
    b, T, H, P = x.shape
    N = B.shape[-1]
    hg = torch.zeros(b, H, P, N, dtype=x.dtype)
    hb = torch.zeros(b, H, P, N, dtype=x.dtype)
    a_b = dA if exact_beta_dA else dA.detach()
    ys = []
    for t in range(T):
        hg = torch.exp(dA[:, t])[..., None, None] * hg + (gamma[:, t, :, None] * x[:, t]).unsqueeze(-1) * \
            B[:, t].unsqueeze(-2)
        hb = torch.exp(a_b[:, t])[..., None, None] * hb
        if t > 0:
            hb = hb + (beta[:, t, :, None] * x[:, t - 1]).unsqueeze(-1) * B[:, t - 1].unsqueeze(-2)
        ys.append(torch.einsum("bhpn,bhn->bhp", hg + hb, C[:, t]))
    return torch.stack(ys, dim=1)
