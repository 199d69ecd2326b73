"""GPU parity of the block front-end kernels (include/ssd_frontend.h) against oracle/frontend.py
in fp64 on the CPU, at config 4's layer shape (B=4, T=4096, H=32; RoPE on per-head B/C with N=128)
and at odd sizes: every output and every gradient, normwise (max|got - ref| / max|ref|) within
1e-5 for fp32 and 1e-2 for bf16 storage (the oracle on the same stored values)."""
from __future__ import annotations

import pytest
import torch

from conftest import gpu_available
from oracle import frontend as of
from ssd_testlib import rel_err

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not gpu_available(), reason="needs an MI355X (HIP device)")]

DEV = "cuda"
TOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2}


def _k():
    import kernels
    return kernels


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("shape", [(4, 4096, 32), (3, 37, 5)], ids=["config4", "odd"])
@pytest.mark.parametrize("used", ["all", "dt_beta"])
def test_trapezoidal(shape, dtype, used):
    g = torch.Generator().manual_seed(0)
    H = shape[-1]
    dt_raw = torch.randn(*shape, generator=g).to(dtype)
    lam_raw = torch.randn(*shape, generator=g).to(dtype)
    bias = torch.empty(H).uniform_(0.001, 0.1, generator=g)      # fp32 parameters, as in the block
    alog = torch.empty(H).uniform_(-4, -1, generator=g)
    gs = [torch.randn(*shape, generator=g).to(dtype) for _ in range(4)]
    pick = [0, 1, 2, 3] if used == "all" else [0, 2]

    leaves = [t.to(DEV).requires_grad_(True) for t in (dt_raw, lam_raw, bias, alog)]
    outs = _k().fused_trapezoidal(*leaves)
    torch.autograd.backward([outs[i] for i in pick], [gs[i].to(DEV) for i in pick])
    ref_leaves = [dt_raw.double().requires_grad_(True), lam_raw.double().requires_grad_(True),
                  bias.to(dtype).double().requires_grad_(True), alog.to(dtype).double().requires_grad_(True)]
    routs = of.trapezoidal(*ref_leaves)
    torch.autograd.backward([routs[i] for i in pick], [gs[i].double() for i in pick])
    tol = TOL[dtype]
    for name, o, r in zip(("dt", "dA", "beta", "gamma"), outs, routs):
        assert o.dtype == dtype
        assert rel_err(o, r) <= tol, f"{name}: {rel_err(o, r):.2e}"
    for name, a, b in zip(("d_dt_raw", "d_lam_raw", "d_dt_bias", "d_A_log"), leaves, ref_leaves):
        if b.grad is None:
            continue
        assert a.grad.dtype == a.dtype
        assert rel_err(a.grad, b.grad) <= tol, f"{name}: {rel_err(a.grad, b.grad):.2e}"


@pytest.mark.parametrize("dtype,adtype", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.float32),
                                          (torch.bfloat16, torch.float32)], ids=["bf16", "fp32", "bf16_x_fp32_angles"])
@pytest.mark.parametrize("per_head", [True, False], ids=["per_head", "shared"])
@pytest.mark.parametrize("shape", [(4, 4096, 32, 128), (2, 9, 3, 6)], ids=["config4", "odd"])
def test_rope(shape, per_head, dtype, adtype):
    B, T, H, D = shape
    g = torch.Generator().manual_seed(1)
    x = torch.randn(B, T, H, D, generator=g).to(dtype)
    ang = (3.0 * torch.randn(B, T, H if per_head else 1, D // 2, generator=g)).to(adtype)
    dy = torch.randn(B, T, H, D, generator=g).to(dtype)
    xl, al = x.to(DEV).requires_grad_(True), ang.to(DEV).requires_grad_(True)
    out = _k().fused_rope(xl, al)
    out.backward(dy.to(DEV))
    xr, ar = x.double().requires_grad_(True), ang.double().requires_grad_(True)
    ref = of.rope(xr, ar)
    ref.backward(dy.double())
    tol = TOL[dtype]
    assert out.dtype == dtype and al.grad.dtype == adtype
    assert rel_err(out, ref) <= tol
    assert rel_err(xl.grad, xr.grad) <= tol
    tol_a = TOL[adtype] if dtype == adtype else 1e-2  # bf16 x and dy bound the angle gradient
    assert rel_err(al.grad, ar.grad) <= tol_a


def test_inproj_split_forward_and_partial_backward():
    """The block's split (mamba_base_engine.py:63-71 sizes at config 4): views of one GEMM, and a
    backward where only some outputs are used."""
    torch.manual_seed(2)
    d_model, d_inner, N, H = 1024, 2048, 128, 32
    sizes = [d_inner, d_inner, N, N, H, H, N // 2]
    x = torch.randn(2, 64, d_model, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    w = (torch.randn(sum(sizes), d_model, device=DEV) / d_model ** 0.5).to(torch.bfloat16).requires_grad_(True)
    parts = _k().fused_inproj_split(x, w, sizes)
    assert [p.shape[-1] for p in parts] == sizes
    base = parts[0].untyped_storage().data_ptr()
    assert all(p.untyped_storage().data_ptr() == base for p in parts)  # zero-copy views of one buffer
    (parts[0].float().sum() + 2 * parts[6].float().sum()).backward()
    xr, wr = x.detach().float().requires_grad_(True), w.detach().float().requires_grad_(True)
    pr = of.inproj_split(xr, wr, sizes)
    (pr[0].sum() + 2 * pr[6].sum()).backward()
    assert rel_err(torch.cat(parts, -1), torch.cat(pr, -1)) <= 1e-2
    assert rel_err(x.grad, xr.grad) <= 1e-2 and rel_err(w.grad, wr.grad) <= 1e-2
