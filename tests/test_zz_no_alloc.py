"""ssd_fwd_noalloc (the forward entry point that allocates nothing) against ssd_fwd.

Called through the C ABI on two calls in a row, the second with a smaller
input, each compared bit for bit with ssd_fwd on caller-allocated workspaces
(the same kernels run on both paths, so the outputs must be identical).
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from conftest import gpu_available
from oracle.inputs import SsdShape, make_inputs, make_reference_test_inputs

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not gpu_available(), reason="needs an MI355X (HIP device)")]

DEV = "cuda"


def _noalloc(cfg, x, dt, A, B, C, D, z, w, init, cu):
    """ssd_fwd_noalloc with the same descriptor and output layout as kernels.ssd_scan._forward."""
    from kernels import _capi as C_
    from kernels import ssd_scan as ks
    lib = C_.load()
    desc = ks._desc(cfg, x, B, dt, D, z, init)
    b, T, H, P = x.shape
    N = B.shape[3]
    y = torch.empty_like(x)
    sdt = torch.float32 if cfg.state_code == C_.SSD_DTYPE_F32 else torch.bfloat16
    final = torch.empty((cfg.nseq, H, P, N), dtype=sdt, device=x.device)
    acs = torch.empty((b, H, T // cfg.chunk, cfg.chunk), dtype=x.dtype, device=x.device) if cfg.want_acs else None
    p = ks._p
    args = C_.SsdFwdArgs(p(x), p(dt), p(A), p(B), p(C), p(D), p(z), p(w), p(init), p(cu), p(y), p(final), p(acs),
                         None)
    with torch.cuda.device(x.device):
        st = lib.ssd_fwd_noalloc(ctypes.byref(desc), ctypes.byref(args), ks._stream(x.device))
    C_.check(st, "ssd_fwd_noalloc")
    return y, final, acs


def _extended_case():
    from kernels import _capi as C_
    from kernels import ssd_scan as ks
    shape = SsdShape(2, 1024, 8, 64, 2, 128, 256)
    inp = make_inputs(shape, seed=61, with_z=True, with_init=True)
    t = {k: v.to(DEV) for k, v in inp.items()}
    x, B, C, z = (t[k].bfloat16() for k in ("x", "B", "C", "z"))
    w = torch.ones(shape.nheads * shape.headdim, device=DEV)
    cfg = ks._Cfg(chunk=shape.chunk, a_mode=C_.SSD_A_PER_HEAD, nseq=shape.batch, varlen=False,
                  state_code=C_.SSD_DTYPE_F32, want_acs=False, eps=1e-6)
    return cfg, (x, t["dt"], t["A"], B, C, t["D"], z, w, t["init"], None)


def _reference_api_case():
    from kernels import _capi as C_
    from kernels import ssd_scan as ks
    x, A, B, C = [v.to(DEV) for v in make_reference_test_inputs(1, 256, 4, 16, 8, seed=62)]
    cfg = ks._Cfg(chunk=64, a_mode=C_.SSD_A_PER_TOKEN, nseq=1, varlen=False, state_code=C_.SSD_DTYPE_F32,
                  want_acs=True, eps=0.0)
    return cfg, (x, None, A, B, C, None, None, None, None, None)


def test_noalloc_forward_matches_ssd_fwd_on_two_calls():
    from kernels import ssd_scan as ks
    for name, case in (("bf16 extended, B=2 L=1024 H=8 P=64 N=128", _extended_case),
                       ("fp32 reference API, B=1 L=256 H=4 P=16 N=8 (smaller)", _reference_api_case)):
        print("case:", name, flush=True)
        cfg, inputs = case()
        y0, f0, a0, _ = ks._forward(cfg, *inputs)
        y1, f1, a1 = _noalloc(cfg, *inputs)
        torch.cuda.synchronize()
        assert torch.equal(y1, y0), name
        assert torch.equal(f1, f0), name
        if cfg.want_acs:
            assert torch.equal(a1, a0), name
