"""Pins the CPU oracle before anything is compared against it.

Each check is chosen so that a plausible slip in the oracle (a dropped term,
an off-by-one in the segsum band, a wrong sign, a transposed operand, a lost
clamp mask) fails at least one of them:

* the reference's committed golden vectors (stream/ces/ssd_reference/
  golden_vectors, verify.py:26 tolerance 1e-5) and the ces-ssm KAT inputs
  (stream/ces/ces-ssm/src/lib.rs:309-337) against a scalar brute force;
* the chunked restatement against the sequential recurrence (different
  formulation) for Y, final_state and all gradients;
* closed forms (a = 0, X = 0, one chunk), chunk-size invariance, split/concat
  through initial_states, linearity;
* fp64 gradcheck of the custom segsum / exp-clamp backward rules, plus a
  planted mistake in a copy of the oracle that gradcheck must reject;
* the reference test's own shapes/cache contract (test_ssd_scan.py:99-131).
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ssd_chunked as oc
from oracle.ssd_extended import ssd_combined
from oracle.ssd_sequential import ces_scalar_reference, ssd_sequential
from oracle.inputs import make_reference_test_inputs

GOLDEN = Path(__file__).resolve().parent / "golden"
E20 = math.exp(-20.0)


def _rand_case(b, T, h, p, n, seed, decay=0.1, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(b, T, h, p, generator=g, dtype=dtype)
    a = -torch.rand(b, T, h, generator=g, dtype=dtype) * decay
    B = torch.randn(b, T, h, n, generator=g, dtype=dtype) * 0.5
    C = torch.randn(b, T, h, n, generator=g, dtype=dtype) * 0.5
    return X, a, B, C


def T_SUM_BOUND(X, B, C):
    """max over outputs of sum_s |C_l . B_s| |X_s| (per batch/head), times 2."""
    S = torch.einsum("blhn,bshn->bhls", C.abs(), B.abs())
    return 2 * torch.einsum("bhls,bshp->blhp", S, X.abs()).max().item()


def _golden_cases():
    return sorted((GOLDEN / "ces").glob("*.npz"))


@pytest.mark.parametrize("path", _golden_cases(), ids=lambda p: p.stem)
@pytest.mark.parametrize("dtype", [torch.float64, torch.float32])
def test_golden_vectors_chunked(path, dtype):
    d = np.load(path, allow_pickle=False)
    meta = json.loads(str(d["metadata"]))
    t = {k: torch.from_numpy(d[k]).to(dtype) for k in ("x", "A", "B", "C", "dt", "D", "dt_bias")}
    step = F.softplus(t["dt"] + t["dt_bias"].view(1, 1, -1))       # extract.py:44-45
    X = (step * t["x"]).unsqueeze(-1)                                # P = 1
    a = step * t["A"].view(1, 1, -1)
    Y, _, _ = oc.ssd_forward_impl(X, a, t["B"], t["C"], meta["chunk_len"])
    y = Y[..., 0] + t["D"].view(1, 1, -1) * t["x"]
    expect = torch.from_numpy(d["expected_y"]).double()
    err = (y.double() - expect).abs().max().item()
    if dtype == torch.float64:
        # the vectors were written in fp32 by a sequential loop: verify.py:26's 1e-5
        assert err <= 1e-5, f"{path.name}: max|dy| = {err:.3e}"
    else:
        # fp32 chunked vs fp32 sequential: two different rounding orders, |y| up to ~60
        assert err <= 1e-6 * expect.abs().max().item(), f"{path.name}: max|dy| = {err:.3e}"


@pytest.mark.parametrize("path", _golden_cases()[:3], ids=lambda p: p.stem)
def test_golden_vectors_sequential(path):
    d = np.load(path, allow_pickle=False)
    t = {k: torch.from_numpy(d[k]).double() for k in ("x", "A", "B", "C", "dt", "D", "dt_bias")}
    step = F.softplus(t["dt"] + t["dt_bias"].view(1, 1, -1))
    Y, _ = ssd_sequential((step * t["x"]).unsqueeze(-1), step * t["A"].view(1, 1, -1), t["B"], t["C"])
    y = Y[..., 0] + t["D"].view(1, 1, -1) * t["x"]
    err = (y - torch.from_numpy(d["expected_y"]).double()).abs().max().item()
    assert err <= 1e-5


def test_ces_ssm_kat():
    k = json.loads((GOLDEN / "ces_ssm_kat.json").read_text())
    bt, T, H, N = k["batch"], k["seq_len"], k["n_heads"], k["d_state"]
    expect = torch.tensor(ces_scalar_reference(k["x"], k["a"], k["b"], k["c"], k["dt"], k["d"],
                                               k["dt_bias"], bt, T, H, N), dtype=torch.float64)
    x = torch.tensor(k["x"], dtype=torch.float64).view(bt, T, H)
    dt = torch.tensor(k["dt"], dtype=torch.float64).view(bt, T, H)
    step = F.softplus(dt + torch.tensor(k["dt_bias"], dtype=torch.float64).view(1, 1, H))
    Bm = torch.tensor(k["b"], dtype=torch.float64).view(bt, T, H, N)
    Cm = torch.tensor(k["c"], dtype=torch.float64).view(bt, T, H, N)
    A = torch.tensor(k["a"], dtype=torch.float64)
    for Q in (1, 2, 4):
        Y, _, _ = oc.ssd_forward_impl((step * x).unsqueeze(-1), step * A, Bm, Cm, Q)
        y = Y[..., 0] + torch.tensor(k["d"], dtype=torch.float64) * x
        assert (y.flatten() - expect).abs().max().item() < k["tolerance"]


@pytest.mark.parametrize("Q", [1, 4, 16, 64])
def test_chunked_equals_sequential(Q):
    X, a, B, C = _rand_case(2, 64, 3, 4, 5, seed=Q)
    init = torch.randn(2, 3, 4, 5, dtype=torch.float64, generator=torch.Generator().manual_seed(9))
    Yc, fc, _ = oc.ssd_forward_impl(X, a, B, C, Q, init.unsqueeze(1))
    Ys, fs = ssd_sequential(X, a, B, C, init)
    # decays stay far above e^-20 here: only the acausal e^-20 fill differs
    bound = 10 * E20 * (X.abs().sum() * B.abs().max() * C.abs().max() * 5 + init.abs().sum())
    assert (Yc - Ys).abs().max().item() <= 1e-10 + bound.item()
    assert (fc - fs).abs().max().item() <= 1e-10 + bound.item()


def test_strong_decay_within_clamp_bound():
    """With strong decay the clamp fires on most entries; the reference values
    then differ from exact math by at most e^-20 * sum |terms|."""
    X, a, B, C = _rand_case(1, 128, 2, 4, 4, seed=3, decay=2.0)
    Yc, fc, _ = oc.ssd_forward_impl(X, a, B, C, 32)
    Ys, fs = ssd_sequential(X, a, B, C)
    terms = X.abs().sum() * B.abs().max() * C.abs().max() * 4
    assert (Yc - Ys).abs().max().item() <= 4 * E20 * terms.item()
    assert (Yc - Ys).abs().max().item() > 0  # the clamp is live in this case


def test_closed_form_zero_decay():
    """a = 0, one chunk: L = 1 on and below the diagonal, e^-20 above (the -1e4
    fill, ssd_scan.py:111-116), and the matrix-form recurrence (:403-409) also
    leaks e^-20 of the chunk's own state into its entering state, so
    Y = (C B^T * L) X + e^-20 * C st^T with st = X^T B."""
    X, _, B, C = _rand_case(1, 16, 2, 3, 4, seed=5)
    a = torch.zeros(1, 16, 2, dtype=torch.float64)
    Y, _, _ = oc.ssd_forward_impl(X, a, B, C, 16)
    Lm = torch.full((16, 16), E20, dtype=torch.float64).tril(-1).T + torch.ones(16, 16, dtype=torch.float64).tril()
    for h in range(2):
        S = C[0, :, h] @ B[0, :, h].T
        st = X[0, :, h].T @ B[0, :, h]                      # (p, n)
        ref = (S * Lm) @ X[0, :, h] + E20 * C[0, :, h] @ st.T
        assert torch.allclose(Y[0, :, h], ref, atol=1e-13, rtol=0)
        assert not torch.allclose(Y[0, :, h], (S * Lm) @ X[0, :, h], atol=1e-13, rtol=0)


def test_closed_form_zero_input():
    """X = 0 => Y_t = exp(clamp(cumsum a)) C_t . init (first chunk) and Y = 0 without init."""
    _, a, B, C = _rand_case(1, 32, 2, 3, 4, seed=6)
    X = torch.zeros(1, 32, 2, 3, dtype=torch.float64)
    Y0, f0, _ = oc.ssd_forward_impl(X, a, B, C, 8)
    assert Y0.abs().max().item() == 0.0 and f0.abs().max().item() == 0.0
    init = torch.randn(1, 2, 3, 4, dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    Y, f, _ = oc.ssd_forward_impl(X, a, B, C, 8, init.unsqueeze(1))
    cs = torch.cumsum(a[0], dim=0)                                      # (T, h)
    ref = torch.exp(cs)[..., None] * torch.einsum("thn,hpn->thp", C[0], init[0])
    assert torch.allclose(Y[0], ref, atol=1e-12, rtol=1e-10)
    assert torch.allclose(f[0], torch.exp(cs[-1])[:, None, None] * init[0], atol=1e-12)


def test_chunk_size_invariance_and_split():
    """Chunking changes only the e^-20 leak terms, bounded by e^-20 * sum|terms|."""
    X, a, B, C = _rand_case(2, 128, 2, 4, 6, seed=7)
    # per output the leak is e^-20 * sum_s |C_l.B_s X_s| (<= ~1e-7 here, |Y| ~ 10)
    tol = E20 * T_SUM_BOUND(X, B, C)
    Y64, f64, _ = oc.ssd_forward_impl(X, a, B, C, 64)
    for Q in (8, 16, 32, 128):
        Y, f, _ = oc.ssd_forward_impl(X, a, B, C, Q)
        assert (Y - Y64).abs().max().item() < tol
        assert (f - f64).abs().max().item() < tol
    Y1, f1, _ = oc.ssd_forward_impl(X[:, :64], a[:, :64], B[:, :64], C[:, :64], 32)
    Y2, f2, _ = oc.ssd_forward_impl(X[:, 64:], a[:, 64:], B[:, 64:], C[:, 64:], 32, f1.unsqueeze(1))
    assert (torch.cat([Y1, Y2], 1) - Y64).abs().max().item() < tol
    assert (f2 - f64).abs().max().item() < tol
    assert tol < 1e-6


def test_linearity_in_x():
    X, a, B, C = _rand_case(1, 64, 2, 3, 4, seed=8)
    X2 = torch.randn_like(X)
    Y1, _, _ = oc.ssd_forward_impl(X, a, B, C, 16)
    Y2, _, _ = oc.ssd_forward_impl(X2, a, B, C, 16)
    Y3, _, _ = oc.ssd_forward_impl(2.0 * X - 3.0 * X2, a, B, C, 16)
    assert (Y3 - (2 * Y1 - 3 * Y2)).abs().max().item() < 1e-11  # the leak is linear in X too


def _tiny(seed=0, decay=0.3):
    X, a, B, C = _rand_case(1, 8, 2, 2, 3, seed=seed, decay=decay)
    init = torch.randn(1, 1, 2, 2, 3, dtype=torch.float64, generator=torch.Generator().manual_seed(seed))
    return [t.requires_grad_(True) for t in (X, a, B, C, init)]


def _fn(X, a, B, C, init):
    Y, f, _ = oc.ssd_forward_impl(X, a, B, C, 4, init)
    return Y, f


def test_gradcheck_chunked_backward():
    assert torch.autograd.gradcheck(_fn, _tiny(), eps=1e-6, atol=1e-7)


def test_gradcheck_rejects_planted_segsum_slip(monkeypatch):
    """Shift the segsum band by one row in a copy of the backward: gradcheck
    must fail (shows the check has teeth for index slips)."""
    def wrong_backward(ctx, dy):
        (y,) = ctx.saved_tensors
        T = y.shape[-1]
        idx = torch.arange(T)
        g = torch.where((idx[:, None] >= idx[None, :]), dy, torch.zeros_like(dy))
        R = torch.cumsum(g, dim=-1)          # planted: inclusive instead of exclusive
        suffix = torch.flip(torch.cumsum(torch.flip(R, dims=[-2]), dim=-2), dims=[-2])
        return torch.diagonal(suffix, dim1=-2, dim2=-1)
    monkeypatch.setattr(oc._Segsum, "backward", staticmethod(wrong_backward))
    assert not torch.autograd.gradcheck(_fn, _tiny(), eps=1e-6, atol=1e-7, raise_exception=False)


def test_clamp_masks_are_strict_and_zero_outside():
    """Entries clamped at -20 carry no gradient (ssd_scan.py:192, :230)."""
    x = torch.tensor([-25.0, -20.0, -19.0, 0.0, 25.0], dtype=torch.float64, requires_grad=True)
    y = oc.exp_clamp(x)
    y.sum().backward()
    expect = torch.tensor([0.0, 0.0, math.exp(-19.0), 1.0, 0.0], dtype=torch.float64)
    assert torch.allclose(x.grad, expect)


def test_chunked_grads_match_sequential():
    X, a, B, C = _rand_case(2, 48, 2, 3, 4, seed=11)
    init = torch.randn(2, 2, 3, 4, dtype=torch.float64, generator=torch.Generator().manual_seed(2))
    dY = torch.randn_like(X)
    dF = torch.randn_like(init)
    res = []
    for chunked in (True, False):
        leaves = [t.clone().requires_grad_(True) for t in (X, a, B, C, init)]
        if chunked:
            Y, f, _ = oc.ssd_forward_impl(*leaves[:4], 16, leaves[4].unsqueeze(1))
        else:
            Y, f = ssd_sequential(*leaves)
        torch.autograd.backward([Y, f], [dY, dF])
        res.append([t.grad for t in leaves])
    for gc, gs in zip(*res):
        # e^-20 leak terms only (~4e-8 here against gradients of size ~10)
        assert (gc - gs).abs().max().item() < 1e-6 * gs.abs().max().item()


def test_reference_contract_shapes_and_cache():
    """test_ssd_scan.py:99-131: final_state (b,h,p,n); cache shapes; cache reuse."""
    b, T, h, p, n, chunk = 2, 512, 4, 32, 8, 128
    x, A, B, C = make_reference_test_inputs(b, T, h, p, n, seed=3)
    _, fs, cache = oc.fused_ssd_scan(x, A, B, C, chunk)
    c = T // chunk
    assert fs.shape == (b, h, p, n)
    assert cache["L"].shape == (b, h, c, chunk, chunk)
    assert cache["decay_chunk"].shape == (b, h, c + 1, c + 1)
    assert cache["A_cumsum"].shape == (b, h, c, chunk)
    x2, _, B2, C2 = make_reference_test_inputs(b, T, h, p, n, seed=5)
    Yf, ff, _ = oc.fused_ssd_scan(x2, A, B2, C2, chunk)
    Yr, fr, _ = oc.fused_ssd_scan(x2, A, B2, C2, chunk, cache=cache)
    assert (Yf - Yr).abs().max().item() < 1e-4 and (ff - fr).abs().max().item() < 1e-4


def test_cache_path_drops_dA():
    """With a cache the reference never reads A, so A gets no gradient
    (ssd_scan.py:364-406, :533); x, B, C still do."""
    x, A, B, C = make_reference_test_inputs(1, 64, 2, 4, 4, seed=1, dtype=torch.float64)
    _, _, cache = oc.fused_ssd_scan(x, A, B, C, 16)
    leaves = [t.clone().requires_grad_(True) for t in (x, A, B, C)]
    Y, _, _ = oc.fused_ssd_scan(*leaves, 16, cache=cache)
    Y.sum().backward()
    assert leaves[1].grad is None
    assert all(t.grad is not None for t in (leaves[0], leaves[2], leaves[3]))


def test_extended_varlen_equals_batched():
    """Varlen with equal-length sequences equals the batched layout; groups
    equal explicit per-head expansion."""
    g = torch.Generator().manual_seed(4)
    b, L, H, P, G, N = 3, 40, 4, 3, 2, 5
    x = torch.randn(b, L, H, P, generator=g, dtype=torch.float64)
    dt = torch.rand(b, L, H, generator=g, dtype=torch.float64) * 0.1 + 0.01
    A = -torch.rand(H, generator=g, dtype=torch.float64) * 4
    B = torch.randn(b, L, G, N, generator=g, dtype=torch.float64)
    C = torch.randn(b, L, G, N, generator=g, dtype=torch.float64)
    D = torch.randn(H, generator=g, dtype=torch.float64)
    init = torch.randn(b, H, P, N, generator=g, dtype=torch.float64)
    Yb, fb = ssd_combined(x, dt, A, B, C, 16, D=D, initial_states=init)
    cu = torch.tensor([0, L, 2 * L, 3 * L])
    Yv, fv = ssd_combined(x.reshape(1, b * L, H, P), dt.reshape(1, b * L, H), A,
                          B.reshape(1, b * L, G, N), C.reshape(1, b * L, G, N), 16, D=D,
                          initial_states=init, cu_seqlens=cu)
    assert (Yv.reshape(b, L, H, P) - Yb).abs().max().item() < 1e-12
    assert (fv - fb).abs().max().item() < 1e-12
    # exact operator: sequential brute force on the discretised inputs
    Ys, fs = ssd_sequential(x * dt[..., None], dt * A, B.repeat_interleave(2, 2),
                            C.repeat_interleave(2, 2), init)
    # e^-20 leak terms only
    assert (Yb - (Ys + x * D.view(1, 1, H, 1))).abs().max().item() < 1e-7
    assert (fb - fs).abs().max().item() < 1e-7


def test_extended_gated_norm_invariants():
    """Properties that fix the norm: scale invariance (eps = 0), unit RMS of the
    normalised row (w = 1, gate divided out), eps inside the square root (a
    constant row c gives c / sqrt(c^2 + eps)), reduction over the last dim only."""
    from oracle.ssd_extended import gated_rmsnorm
    g = torch.Generator().manual_seed(5)
    y = torch.randn(2, 3, 8, generator=g, dtype=torch.float64)
    z = torch.randn(2, 3, 8, generator=g, dtype=torch.float64)
    w = torch.randn(8, generator=g, dtype=torch.float64)
    assert torch.allclose(gated_rmsnorm(3.7 * y, z, w, 0.0), gated_rmsnorm(y, z, w, 0.0), atol=1e-13)
    gate = torch.nn.functional.silu(z)
    u = gated_rmsnorm(y, z, torch.ones(8, dtype=torch.float64), 0.0) / gate
    assert torch.allclose(u.pow(2).mean(-1), torch.ones(2, 3, dtype=torch.float64), atol=1e-12)
    c, eps = 0.05, 1e-3
    row = torch.full((1, 1, 8), c, dtype=torch.float64)
    one = torch.ones(8, dtype=torch.float64)
    out = gated_rmsnorm(row, torch.full_like(row, 50.0), one, eps)  # silu(50) = 50 to 1e-20
    assert torch.allclose(out, torch.full_like(row, c / math.sqrt(c * c + eps) * 50.0), rtol=1e-12)
    # rows are independent: changing one row leaves the others unchanged
    y2 = y.clone()
    y2[0, 0] *= -5.0
    assert torch.equal(gated_rmsnorm(y2, z, w, 1e-6)[1], gated_rmsnorm(y, z, w, 1e-6)[1])


def test_extended_gated_norm_backward_matches_reference_closed_form():
    """The reference documents RMSNorm's backward in closed form
    (r2/dhammic-ai/src/kernels/rmsnorm.py:15-36): with r = rsqrt(mean(x^2) + e),
    s = sum_j w_j x_j g_j, dx_i = r (w_i g_i - (x_i / D) r^2 s), dw = sum_rows x r g.
    The oracle differentiates by autograd; composing the closed form with the
    gate's product rule must give the same gradients."""
    from oracle.ssd_extended import gated_rmsnorm
    g = torch.Generator().manual_seed(6)
    D, eps = 16, 1e-6
    y = torch.randn(5, D, generator=g, dtype=torch.float64, requires_grad=True)
    z = torch.randn(5, D, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(D, generator=g, dtype=torch.float64, requires_grad=True)
    go = torch.randn(5, D, generator=g, dtype=torch.float64)
    dy, dz, dw = torch.autograd.grad(gated_rmsnorm(y, z, w, eps), (y, z, w), go)
    with torch.no_grad():
        sig = torch.sigmoid(z)
        gate = z * sig
        r = torch.rsqrt(y.pow(2).mean(-1, keepdim=True) + eps)
        gn = go * gate                                   # gradient reaching the norm's output
        s = (w * y * gn).sum(-1, keepdim=True)
        dy_ref = r * (w * gn - (y / D) * r * r * s)
        dw_ref = (y * r * gn).sum(0)
        dz_ref = go * (y * r * w) * (sig * (1 + z * (1 - sig)))
    assert torch.allclose(dy, dy_ref, atol=1e-12)
    assert torch.allclose(dw, dw_ref, atol=1e-12)
    assert torch.allclose(dz, dz_ref, atol=1e-12)


def test_storage_emulation_of_the_bf16_reference_run():
    """fused_ssd_scan(storage=bf16) on wide inputs: fp32 arithmetic with every intermediate (and its gradient)
    rounded to bf16. It must be the plain oracle when storage is the inputs' own dtype, move the results by a
    bf16-sized amount, and land within a small factor of an actual bf16 run of the oracle (CPU bf16 einsum,
    fp32 accumulation inside each contraction)."""
    x, A, B, C = make_reference_test_inputs(2, 256, 4, 16, 8, seed=5)
    x, A, B, C = [t.bfloat16().double() for t in (x, A, B, C)]
    dY = torch.randn(2, 256, 4, 16, generator=torch.Generator().manual_seed(6)).bfloat16().double()

    def run(dtype, storage):
        leaves = [t.detach().clone().to(dtype).requires_grad_(True) for t in (x, A, B, C)]
        Y, fin, _ = oc.fused_ssd_scan(*leaves, 64, storage=storage)
        Y.backward(dY.to(dtype))
        return [Y.detach().double()] + [t.grad.double() for t in leaves]

    ref = run(torch.float64, None)
    same = run(torch.float64, torch.float64)
    emu = run(torch.float32, torch.bfloat16)
    real = run(torch.bfloat16, None)
    rel = lambda a, b: ((a - b).abs().max() / b.abs().max()).item()  # noqa: E731
    for r, s_ in zip(ref, same):
        assert torch.equal(r, s_)
    for name, r, e, b in zip(("Y", "dx", "dA", "dB", "dC"), ref, emu, real):
        de, db = rel(e, r), rel(b, r)
        assert 1e-4 < de < 5e-2, (name, de)
        assert de < 4 * db + 1e-3 and db < 4 * de + 1e-3, (name, de, db)
