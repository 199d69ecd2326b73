"""The block front end that produces the SSD scan's inputs, on MI355X.

Drop-ins for the reference's front-end ops (same names, arguments, shapes, dtypes and
return conventions):

* ``fused_trapezoidal(dt_raw, lam_raw, dt_bias, A_log) -> (dt, dA, beta, gamma)`` and
  ``FusedTrapezoidal`` (r2/dhammic-ai/src/kernels/trapezoidal.py:214-331): HIP kernels
  ``ssd_trapezoidal_fwd`` / ``ssd_trapezoidal_bwd`` (include/ssd_frontend.h).
* ``fused_rope(x, angles)`` and ``FusedRoPE`` (rope.py:228-321): ``ssd_rope_fwd`` /
  ``ssd_rope_bwd``; angles per head (B, T, H, D/2) or shared (B, T, 1, D/2).
* ``fused_inproj_split(x, weight, split_sizes)``, ``FusedInProjSplit`` and
  ``FusedInProjSplitModule`` (inproj_split.py:48-286): one library GEMM (torch's, hipBLASLt on
  ROCm) whose outputs are zero-copy column views, the reference's "single_gemm" strategy; the
  backward is two GEMMs over the concatenated gradient. The reference's "multi_gemm" strategy and
  its start-up micro-benchmark only choose between call patterns with the same values; both names
  run the single GEMM here.

All device work of the first two runs in libssd_mi355x.so on the current torch stream. There is no
CPU fallback: CPU tensors raise AssertionError as in the reference (trapezoidal.py:217-219,
rope.py:208).
"""
from __future__ import annotations

from typing import List, Tuple

import torch
import torch.nn as nn
from torch import Tensor

from . import _capi as C_
from .ssd_scan import _code, _p, _stream

__all__ = ["fused_trapezoidal", "FusedTrapezoidal", "fused_rope", "FusedRoPE", "fused_inproj_split",
           "FusedInProjSplit", "FusedInProjSplitModule"]


class FusedTrapezoidal(torch.autograd.Function):
    """(dt, dA, beta, gamma) = trapezoidal coefficients (trapezoidal.py:3-13); dt_bias and A_log are
    cast to the input dtype first, as the reference does (:236-237)."""

    @staticmethod
    def forward(ctx, dt_raw: Tensor, lam_raw: Tensor, dt_bias: Tensor, A_log: Tensor):
        assert dt_raw.is_cuda and lam_raw.is_cuda and dt_bias.is_cuda and A_log.is_cuda, (
            "FusedTrapezoidal requires CUDA tensors")
        assert dt_raw.shape == lam_raw.shape, f"dt_raw {dt_raw.shape} vs lam_raw {lam_raw.shape}"
        assert dt_raw.dim() >= 1, "expected at least (..., H) tensor"
        H = dt_raw.shape[-1]
        assert dt_bias.dim() == 1 and dt_bias.shape[0] == H, f"dt_bias shape {dt_bias.shape} mismatches H={H}"
        assert A_log.dim() == 1 and A_log.shape[0] == H, f"A_log shape {A_log.shape} mismatches H={H}"
        dtype = dt_raw.dtype
        code = _code(dtype, "dt_raw")
        x = dt_raw.contiguous()
        lam = lam_raw.to(dtype).contiguous()
        bias = dt_bias.detach().contiguous().to(dtype)
        alog = A_log.detach().contiguous().to(dtype)
        rows = x.numel() // H
        outs = [torch.empty_like(x) for _ in range(4)]
        lib = C_.load()
        dev = x.device
        with torch.cuda.device(dev):
            st = lib.ssd_trapezoidal_fwd(code, rows, H, _p(x), _p(lam), _p(bias), _p(alog), *[_p(o) for o in outs],
                                         _stream(dev))
        C_.check(st, "ssd_trapezoidal_fwd")
        ctx.save_for_backward(x, lam, bias, alog)
        ctx.param_dtypes = (dt_bias.dtype, A_log.dtype)
        ctx.set_materialize_grads(False)
        return tuple(outs)

    @staticmethod
    def backward(ctx, g_dt, g_dA, g_beta, g_gamma):
        x, lam, bias, alog = ctx.saved_tensors
        H = x.shape[-1]
        rows = x.numel() // H
        dtype = x.dtype
        gs = [None if g is None else g.to(dtype).contiguous() for g in (g_dt, g_dA, g_beta, g_gamma)]
        d_x, d_lam = torch.empty_like(x), torch.empty_like(lam)
        d_bias = torch.empty(H, dtype=torch.float32, device=x.device)
        d_alog = torch.empty(H, dtype=torch.float32, device=x.device)
        lib = C_.load()
        ws = torch.empty(lib.ssd_trapezoidal_bwd_workspace(rows, H), dtype=torch.uint8, device=x.device)
        with torch.cuda.device(x.device):
            st = lib.ssd_trapezoidal_bwd(_code(dtype, "dt_raw"), rows, H, _p(x), _p(lam), _p(bias), _p(alog),
                                         *[_p(g) for g in gs], _p(d_x), _p(d_lam), _p(d_bias), _p(d_alog), _p(ws),
                                         ws.numel(), _stream(x.device))
        C_.check(st, "ssd_trapezoidal_bwd")
        return d_x, d_lam, d_bias.to(ctx.param_dtypes[0]), d_alog.to(ctx.param_dtypes[1])


def fused_trapezoidal(dt_raw: Tensor, lam_raw: Tensor, dt_bias: Tensor, A_log: Tensor):
    """Trapezoidal-discretisation coefficients (dt, dA, beta, gamma), each shaped and typed like dt_raw."""
    return FusedTrapezoidal.apply(dt_raw, lam_raw, dt_bias, A_log)


class FusedRoPE(torch.autograd.Function):
    """Data-dependent rotary embedding (rope.py:4-10) with per-head or shared angles."""

    @staticmethod
    def forward(ctx, x: Tensor, angles: Tensor) -> Tensor:
        assert x.is_cuda and angles.is_cuda, "fused_rope requires CUDA tensors"
        assert x.dim() == 4 and angles.dim() == 4, \
            f"expected x.dim()==4, angles.dim()==4, got {x.dim()}, {angles.dim()}"
        B, T, H, D = x.shape
        assert D % 2 == 0, f"x last dim must be even, got {D}"
        half = D // 2
        aB, aT, aH, aDh = angles.shape
        assert aB == B and aT == T and aDh == half, \
            f"angles shape {tuple(angles.shape)} mismatch (B,T,{{1|H}},D/2)=({B},{T},{{1|{H}}},{half})"
        assert aH == 1 or aH == H, f"angles H dim must be 1 (broadcast) or {H} (per-head), got {aH}"
        xc, ac = x.contiguous(), angles.contiguous()
        out = torch.empty_like(xc)
        lib = C_.load()
        with torch.cuda.device(x.device):
            st = lib.ssd_rope_fwd(_code(x.dtype, "x"), _code(angles.dtype, "angles"), B, T, H, half, int(aH == H),
                                  _p(xc), _p(ac), _p(out), _stream(x.device))
        C_.check(st, "ssd_rope_fwd")
        ctx.save_for_backward(xc, ac)
        return out

    @staticmethod
    def backward(ctx, dy: Tensor):
        xc, ac = ctx.saved_tensors
        B, T, H, D = xc.shape
        dyc = dy.to(xc.dtype).contiguous()
        dx = torch.empty_like(xc)
        dang = torch.empty_like(ac)
        lib = C_.load()
        with torch.cuda.device(xc.device):
            st = lib.ssd_rope_bwd(_code(xc.dtype, "x"), _code(ac.dtype, "angles"), B, T, H, D // 2,
                                  int(ac.shape[2] == H), _p(xc), _p(ac), _p(dyc), _p(dx), _p(dang),
                                  _stream(xc.device))
        C_.check(st, "ssd_rope_bwd")
        return dx, dang


def fused_rope(x: Tensor, angles: Tensor) -> Tensor:
    """x (B, T, H, D) rotated pairwise by angles (B, T, H or 1, D/2); same shape and dtype as x."""
    return FusedRoPE.apply(x, angles)


class FusedInProjSplit(torch.autograd.Function):
    """proj = x W^T as one GEMM; the outputs are column views of it (inproj_split.py:48-84)."""

    @staticmethod
    def forward(ctx, x: Tensor, weight: Tensor, split_sizes: Tuple[int, ...]):
        proj = torch.nn.functional.linear(x, weight)
        ctx.save_for_backward(x, weight)
        ctx.split_sizes = split_sizes
        return tuple(proj.split(list(split_sizes), dim=-1))

    @staticmethod
    def backward(ctx, *grad_outs: Tensor):
        x, weight = ctx.saved_tensors
        g = torch.cat([torch.zeros(*x.shape[:-1], s, dtype=x.dtype, device=x.device) if go is None else go
                       for go, s in zip(grad_outs, ctx.split_sizes)], dim=-1)
        g2 = g.reshape(-1, g.shape[-1])
        grad_x = (g2 @ weight).reshape(x.shape)
        grad_w = g2.t() @ x.reshape(-1, x.shape[-1])
        return grad_x, grad_w, None


def fused_inproj_split(x: Tensor, weight: Tensor, split_sizes: List[int], *, strategy: str = "single_gemm"
                       ) -> Tuple[Tensor, ...]:
    """``nn.Linear(d_model, sum(split_sizes), bias=False)`` then ``torch.split`` as one op."""
    if x.shape[-1] != weight.shape[1]:
        raise ValueError(f"x.shape[-1]={x.shape[-1]} must equal weight.shape[1]={weight.shape[1]}")
    if sum(split_sizes) != weight.shape[0]:
        raise ValueError(f"sum(split_sizes)={sum(split_sizes)} must equal weight.shape[0]={weight.shape[0]}")
    if strategy not in ("single_gemm", "multi_gemm"):
        raise ValueError(f"unknown strategy={strategy!r}")
    return FusedInProjSplit.apply(x, weight, tuple(int(s) for s in split_sizes))


class FusedInProjSplitModule(nn.Module):
    """Drop-in for ``nn.Linear`` + ``torch.split`` (inproj_split.py:224-286)."""

    def __init__(self, d_model: int, split_sizes: List[int], *, dtype: torch.dtype = torch.bfloat16,
                 device=None, probe_shape=None, bench_iters: int = 30) -> None:
        super().__init__()
        self.d_model = int(d_model)
        self.split_sizes = tuple(int(s) for s in split_sizes)
        self.total = sum(self.split_sizes)
        self.weight = nn.Parameter(torch.empty(self.total, self.d_model, dtype=dtype, device=device))
        nn.init.kaiming_uniform_(self.weight, a=5 ** 0.5)
        self.strategy = "single_gemm"

    def forward(self, x: Tensor) -> Tuple[Tensor, ...]:
        return fused_inproj_split(x, self.weight, list(self.split_sizes), strategy=self.strategy)

    def extra_repr(self) -> str:
        return f"d_model={self.d_model}, split_sizes={list(self.split_sizes)}, strategy={self.strategy}"
