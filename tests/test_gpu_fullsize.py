"""GPU parity at BASELINE's full shapes (configs 1, 2 and 3).

The HIP path runs through the C ABI on the full configuration. The checker is
the CPU oracle's restatement of the reference's chunked path, run here on the
GPU in fp32 (plain torch ops: cumsum, einsum, exp), on the same bf16-rounded
inputs; fp32 matrix products keep full precision (no TF32). Tolerance: the
north_star's 1e-2 normwise (max|got - ref| / max|ref|) for bf16 inputs.

Size-independent properties are checked on the kernels alone at config 2:
splitting a sequence at a chunk boundary and carrying the state across
(final_state -> initial_states forward, dinit -> dfinal backward) reproduces
the unsplit call.
"""
from __future__ import annotations

import pytest
import torch

from conftest import gpu_available
from oracle.inputs import CONFIG1, CONFIG2, SsdShape, config3_shape, make_inputs
from oracle.ssd_extended import ssd_combined
from ssd_testlib import TOL, assert_close

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not gpu_available(), reason="needs an MI355X (HIP device)")]

DEV = "cuda"
BF = torch.bfloat16


@pytest.fixture(autouse=True)
def _fp32_matmul():
    prev = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    yield
    torch.backends.cuda.matmul.allow_tf32 = prev
    torch.cuda.empty_cache()


def _k():
    import kernels
    return kernels


def _inputs(shape, seed, with_z, with_init):
    inp = make_inputs(shape, seed=seed, device=DEV, with_z=with_z, with_init=with_init,
                      with_dfinal=with_init)
    for k in ("x", "B", "C", "dy", "z"):
        if k in inp:
            inp[k] = inp[k].to(BF).float()
    return inp


def _native(inp, shape, with_z, cu, use_init):
    leaves = {k: inp[k].to(BF).requires_grad_(True) for k in ("x", "B", "C") + (("z",) if with_z else ())}
    for k in ("dt", "A", "D") + (("init",) if use_init else ()):
        leaves[k] = inp[k].clone().requires_grad_(True)
    w = torch.ones(shape.nheads * shape.headdim, device=DEV).requires_grad_(True) if with_z else None
    out, fin = _k().ssd_scan_combined(
        leaves["x"], leaves["dt"], leaves["A"], leaves["B"], leaves["C"], shape.chunk, D=leaves["D"],
        z=leaves.get("z"), norm_weight=w, initial_states=leaves.get("init"),
        cu_seqlens=None if cu is None else torch.tensor(cu, dtype=torch.int32, device=DEV),
        return_final_state=True)
    outs, grads = [out], [inp["dy"].to(BF)]
    if use_init:
        outs.append(fin)
        grads.append(inp["dfinal"])
    torch.autograd.backward(outs, grads)
    g = {k: v.grad for k, v in leaves.items()}
    if with_z:
        g["w"] = w.grad
    return out.detach(), fin.detach(), g


def _oracle_gpu(inp, shape, with_z, cu, use_init):
    names = ("x", "dt", "A", "B", "C", "D") + (("z",) if with_z else ())
    t = {k: inp[k].clone().requires_grad_(True) for k in names}
    init = inp["init"].clone().requires_grad_(True) if use_init else None
    w = torch.ones(shape.nheads * shape.headdim, device=DEV).requires_grad_(True) if with_z else None
    out, fin = ssd_combined(t["x"], t["dt"], t["A"], t["B"], t["C"], shape.chunk, D=t["D"], z=t.get("z"),
                            norm_weight=w, initial_states=init, cu_seqlens=cu)
    outs, grads = [out], [inp["dy"]]
    if use_init:
        outs.append(fin)
        grads.append(inp["dfinal"])
    torch.autograd.backward(outs, grads)
    g = {k: v.grad for k, v in t.items()}
    if use_init:
        g["init"] = init.grad
    if with_z:
        g["w"] = w.grad
    return out.detach(), fin.detach(), g


def _check(shape, seed, with_z, use_init, cu=None):
    inp = _inputs(shape, seed, with_z, use_init)
    out, fin, g = _native(inp, shape, with_z, cu, use_init)
    torch.cuda.synchronize()
    oo, fo, go = _oracle_gpu(inp, shape, with_z, cu, use_init)
    tol = TOL[BF]
    errs = {"out": assert_close("out", out, oo, tol), "final": assert_close("final", fin, fo, tol)}
    for k in go:
        errs["d" + k] = assert_close("d" + k, g[k], go[k], tol)
    print(f"{shape}: " + " ".join(f"{k}={v:.1e}" for k, v in errs.items()), flush=True)


def test_config1_full():
    """Config 1 (130M-class layer): B=8 L=2048 H=24 P=64 G=1 N=128 Q=256, bf16, + D."""
    _check(CONFIG1, seed=21, with_z=False, use_init=False)


def test_config2_full_gated():
    """Config 2 (the headline shape) with the gated RMSNorm epilogue and D."""
    _check(CONFIG2, seed=22, with_z=True, use_init=False)


def test_config3_full_varlen():
    """Config 3: 65 536 packed tokens, sequences U{512..8192}, H=32 P=64 G=8 N=64,
    per-sequence initial states, final states and their gradients."""
    shape = config3_shape()
    _check(shape, seed=23, with_z=False, use_init=True, cu=shape.cu_seqlens)


def test_config2_split_carries_state():
    """Config 2 without the norm: the second half run from the first half's final
    state equals the unsplit run, and the first half's backward fed with the
    second half's dinit as dfinal reproduces the unsplit gradients."""
    shape = CONFIG2
    inp = _inputs(shape, 24, with_z=False, with_init=False)
    L2 = shape.seqlen // 2
    k = _k()

    def run(sl, init, dfinal):
        leaves = {n: inp[n][:, sl].to(BF).contiguous().requires_grad_(True) for n in ("x", "B", "C")}
        dt = inp["dt"][:, sl].contiguous().requires_grad_(True)
        ini = None if init is None else init.clone().requires_grad_(True)
        y, f = k.ssd_scan_combined(leaves["x"], dt, inp["A"], leaves["B"], leaves["C"], shape.chunk,
                                   D=inp["D"], initial_states=ini, return_final_state=True)
        outs, grads = [y], [inp["dy"][:, sl].to(BF).contiguous()]
        if dfinal is not None:
            outs.append(f)
            grads.append(dfinal)
        torch.autograd.backward(outs, grads)
        g = {n: v.grad for n, v in leaves.items()}
        g["dt"] = dt.grad
        g["init"] = None if ini is None else ini.grad
        return y.detach(), f.detach(), g

    y, f, g = run(slice(None), None, None)
    y1, f1, _ = run(slice(0, L2), None, None)
    y2, f2, g2 = run(slice(L2, None), f1, None)
    _, _, g1 = run(slice(0, L2), None, g2["init"])
    tol = TOL[BF]
    assert_close("y first half", y1, y[:, :L2], tol)
    assert_close("y second half", y2, y[:, L2:], tol)
    assert_close("final", f2, f, tol)
    for n in ("x", "B", "C", "dt"):
        assert_close(f"d{n} first half", g1[n], g[n][:, :L2], tol)
        assert_close(f"d{n} second half", g2[n], g[n][:, L2:], tol)
