"""Helpers shared by the parity tests: tolerances, oracle runs, input makers."""
from __future__ import annotations

import torch

from oracle import ssd_chunked as oc
from oracle.ssd_extended import ssd_combined

# fp32 accumulation; relative error <= 1e-2 for bf16
# inputs, <= 1e-4 for fp32 inputs, measured normwise per tensor as
# max|got - ref| / max|ref|.
TOL = {torch.float32: 1e-4, torch.bfloat16: 1e-2}


def rel_err(got, ref):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    den = ref.abs().max().item()
    return (got - ref).abs().max().item() / (den if den > 0 else 1.0)


def assert_close(name, got, ref, tol):
    e = rel_err(got, ref)
    assert e <= tol, f"{name}: rel err {e:.3e} > {tol:.1e}"
    return e


def oracle_reference_api(x, A, B, C, chunk, dY, init=None, dfinal=None, cache_from=None,
                         dtype=torch.float64):
    """Reference-API oracle on CPU in `dtype`: returns Y, final and grads dict."""
    leaves = [t.detach().cpu().to(dtype).requires_grad_(True) for t in (x, A, B, C)]
    init_l = None if init is None else init.detach().cpu().to(dtype).requires_grad_(True)
    cache = None
    if cache_from is not None:
        with torch.no_grad():
            _, _, cache = oc.fused_ssd_scan(*[t.detach().cpu().to(dtype) for t in cache_from], chunk)
    Y, fin, cache_out = oc.fused_ssd_scan(*leaves, chunk, init_l, cache)
    outs, grads = [Y], [dY.detach().cpu().to(dtype)]
    if dfinal is not None:
        outs.append(fin)
        grads.append(dfinal.detach().cpu().to(dtype))
    torch.autograd.backward(outs, grads)
    g = {k: t.grad for k, t in zip(("x", "A", "B", "C"), leaves)}
    g["init"] = None if init_l is None else init_l.grad
    return Y.detach(), fin.detach(), g, cache_out


def oracle_extended(inp, chunk, dtype=torch.float64, with_z=False, with_D=True, init=None, cu=None,
                    dfinal=None, norm_weight=None):
    names = ["x", "dt", "A", "B", "C"] + (["D"] if with_D else []) + (["z"] if with_z else [])
    t = {k: inp[k].detach().cpu().to(dtype).requires_grad_(True) for k in names}
    init_l = None if init is None else init.detach().cpu().to(dtype).requires_grad_(True)
    w = None if norm_weight is None else norm_weight.detach().cpu().to(dtype).requires_grad_(True)
    out, fin = ssd_combined(t["x"], t["dt"], t["A"], t["B"], t["C"], chunk, D=t.get("D"), z=t.get("z"),
                            norm_weight=w, initial_states=init_l,
                            cu_seqlens=None if cu is None else cu.cpu())
    outs, grads = [out], [inp["dy"].detach().cpu().to(dtype)]
    if dfinal is not None:
        outs.append(fin)
        grads.append(dfinal.detach().cpu().to(dtype))
    torch.autograd.backward(outs, grads)
    g = {k: v.grad for k, v in t.items()}
    g["init"] = None if init_l is None else init_l.grad
    g["w"] = None if w is None else w.grad
    return out.detach(), fin.detach(), g
