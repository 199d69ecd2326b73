"""CPU restatement of the reference's chunked SSD path (test infrastructure only).

Follows r2/dhammic-ai/src/kernels/ssd_scan.py, written from its text:

* ``segsum``      — :61-72 (spec), :78-120 (forward), :123-198 (backward)
* ``exp_clamp``   — :201-214 (forward), :217-232 (backward)
* ``ssd_forward_impl`` — :330-421 (A_cumsum, L, Y_diag, states, decay_chunk,
  recurrence in matrix form, Y_off, cache dict)
* ``fused_ssd_scan`` — :539-583 with the ``FusedSSDScan`` contract of
  :427-533 (forward under no_grad, backward = re-run forward with grad +
  autograd.grad, cache path returns no gradient for A).

Everything runs on CPU tensors in whatever floating dtype the inputs carry
(fp64 for pinning, fp32 for the CPU baseline). The reference's quirks are kept
on purpose: every decay exponent clamped to [-20, 20], the -1e4 fill above the
diagonal (which the clamp turns into e^-20, an acausal leak), strict clamp
masks in the backward, inclusive per-chunk cumsum.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

CLAMP_MIN = -20.0
CLAMP_MAX = 20.0
OFF_DIAG_FILL = -1e4


class _Segsum(torch.autograd.Function):
    """y[..., i, j] = clamp(sum_{k=j+1..i} x[..., k], -20, 20) for i >= j, else clamp(-1e4).

    ssd_scan.py:61-72, :99-116. The sum starts at j+1 (the diagonal is 0).
    Backward (ssd_scan.py:131-194): dx[t] = sum_{j<t} sum_{i>=t} dy[i, j]
    restricted to entries whose forward value lies strictly inside (-20, 20).
    """

    @staticmethod
    def forward(ctx, x):
        T = x.shape[-1]
        idx = torch.arange(T, device=x.device)
        strict_lower = (idx[:, None] > idx[None, :]).to(x.dtype)  # [i, j] = 1 iff i > j
        # column j accumulates x[k] for k = j+1..i down the rows i
        contrib = x.unsqueeze(-1) * strict_lower                  # [..., i, j] = x[i] if i > j
        y = torch.cumsum(contrib, dim=-2)
        upper = idx[:, None] < idx[None, :]
        y = torch.where(upper, torch.full_like(y, OFF_DIAG_FILL), y)
        y = y.clamp(CLAMP_MIN, CLAMP_MAX)
        ctx.save_for_backward(y)
        return y

    @staticmethod
    def backward(ctx, dy):
        (y,) = ctx.saved_tensors
        T = y.shape[-1]
        idx = torch.arange(T, device=y.device)
        inside = (y > CLAMP_MIN) & (y < CLAMP_MAX)
        lower_incl = idx[:, None] >= idx[None, :]
        g = torch.where(inside & lower_incl, dy, torch.zeros_like(dy))
        # dx[t] = sum_{i >= t} sum_{j < t} g[i, j]
        # R[i, t] = sum_{j < t} g[i, j]  (exclusive prefix over columns)
        R = torch.cumsum(g, dim=-1) - g
        # dx[t] = sum_{i >= t} R[i, t]  (suffix over rows)
        suffix = torch.flip(torch.cumsum(torch.flip(R, dims=[-2]), dim=-2), dims=[-2])
        dx = torch.diagonal(suffix, dim1=-2, dim2=-1)
        return dx


class _ExpClamp(torch.autograd.Function):
    """y = exp(clamp(x, -20, 20)); dx = dy * y * 1(-20 < x < 20) (ssd_scan.py:201-232)."""

    @staticmethod
    def forward(ctx, x):
        y = torch.exp(x.clamp(CLAMP_MIN, CLAMP_MAX))
        ctx.save_for_backward(x, y)
        return y

    @staticmethod
    def backward(ctx, dy):
        x, y = ctx.saved_tensors
        inside = (x > CLAMP_MIN) & (x < CLAMP_MAX)
        return torch.where(inside, dy * y, torch.zeros_like(dy))


def segsum(x):
    return _Segsum.apply(x)


def exp_clamp(x):
    return _ExpClamp.apply(x)


def ssd_forward_impl(x, A, B, C, chunk_size, initial_states=None,
                     L_cache=None, decay_chunk_cache=None, A_cumsum_cache=None, storage=None):
    """Chunked SSD forward, ssd_scan.py:330-421.

    x (b,T,h,p), A (b,T,h), B/C (b,T,h,n); T % chunk_size == 0 (asserted, :348).
    Returns (Y (b,T,h,p), final_state (b,h,p,n), {L, decay_chunk, A_cumsum}).

    ``storage`` (e.g. torch.bfloat16) emulates the reference run on inputs of that
    dtype while computing in the inputs' (wider) dtype: every intermediate the
    reference keeps as a tensor of the input dtype (A_cumsum, L, decay_states,
    states, decay_chunk, new_states, state_decay_out, Y_diag, Y_off, Y) is rounded
    to ``storage``, and so is its gradient (autograd through the two casts), while
    each contraction accumulates in the wide dtype as the reference's bmm does.
    """
    def st(t):
        return t if storage is None else t.to(storage).to(t.dtype)
    assert x.shape[1] % chunk_size == 0, (
        f"sequence length {x.shape[1]} not divisible by chunk_size {chunk_size}")
    b, T = x.shape[0], x.shape[1]
    c = T // chunk_size

    def chunk(m):
        return m.reshape(b, c, chunk_size, *m.shape[2:])

    x_c, A_c, B_c, C_c = chunk(x), chunk(A), chunk(B), chunk(C)
    A_perm = A_c.permute(0, 3, 1, 2)                              # (b,h,c,l)
    A_cumsum = A_cumsum_cache if A_cumsum_cache is not None else st(torch.cumsum(A_perm, dim=-1))

    # step 1: intra-chunk diagonal blocks, L = exp(clamp(segsum(A))) (:370-385)
    L = L_cache if L_cache is not None else st(exp_clamp(st(segsum(A_perm))))
    Y_diag = st(torch.einsum("bclhn,bcshn,bhcls,bcshp->bclhp", C_c, B_c, L, x_c))

    # step 2: per-chunk states (:387-392)
    decay_states = st(exp_clamp(st(A_cumsum[..., -1:] - A_cumsum)))
    states = st(torch.einsum("bclhn,bhcl,bclhp->bchpn", B_c, decay_states, x_c))

    # step 3: inter-chunk recurrence in matrix form (:394-410)
    if initial_states is None:
        initial_states = torch.zeros_like(states[:, :1])
    states_full = torch.cat([initial_states, states], dim=1)
    if decay_chunk_cache is not None:
        decay_chunk = decay_chunk_cache
    else:
        decay_chunk = st(exp_clamp(st(segsum(F.pad(A_cumsum[..., -1], (1, 0))))))
    new_states = st(torch.einsum("bhzc,bchpn->bzhpn", decay_chunk, states_full))
    states_in, final_state = new_states[:, :-1], new_states[:, -1]

    # step 4: state -> output (:412-418)
    Y_off = st(torch.einsum("bclhn,bchpn,bhcl->bclhp", C_c, states_in, st(exp_clamp(A_cumsum))))
    Y = st(Y_diag + Y_off).reshape(b, T, *Y_diag.shape[3:])
    return Y, final_state, {"L": L, "decay_chunk": decay_chunk, "A_cumsum": A_cumsum}


def fused_ssd_scan(x, A, B, C, chunk_size, initial_states=None, cache=None, storage=None):
    """Reference public API (ssd_scan.py:539-583), plain autograd (``storage``: see
    ssd_forward_impl).

    Gradients equal the reference's checkpointed backward (:467-533): with a
    cache, A is never read, so it receives no gradient; cache tensors never
    receive gradients because the reference returns None for them (:533).
    """
    if cache is not None:
        L_in = cache.get("L")
        dc_in = cache.get("decay_chunk")
        ac_in = cache.get("A_cumsum")
        L_in = None if L_in is None else L_in.detach()
        dc_in = None if dc_in is None else dc_in.detach()
        ac_in = None if ac_in is None else ac_in.detach()
    else:
        L_in = dc_in = ac_in = None
    return ssd_forward_impl(x, A, B, C, int(chunk_size), initial_states, L_in, dc_in, ac_in, storage)


def fused_ssd_scan_fwd_bwd_baseline(x, A, B, C, chunk_size, dY, initial_states=None):
    """One forward + backward in the reference's own call pattern (:440-533).

    Forward under no_grad; backward re-runs the forward under enable_grad on
    fresh leaves and calls torch.autograd.grad. This is what the CPU baseline
    times. Returns (Y, final_state, dx, dA, dB, dC).
    """
    with torch.no_grad():
        Y, final_state, _ = ssd_forward_impl(x, A, B, C, chunk_size, initial_states)
    leaves = [t.detach().requires_grad_(True) for t in (x, A, B, C)]
    with torch.enable_grad():
        Y_r, _, _ = ssd_forward_impl(*leaves, chunk_size, initial_states)
        grads = torch.autograd.grad([Y_r], leaves, [dY])
    return (Y, final_state) + tuple(grads)
