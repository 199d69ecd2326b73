"""A Mamba-3-style language model for the model-level parity tests (test scaffolding only).

BASELINE config 4 is a full random-init training step of a 24-layer Mamba-3-style LM (d_model 1024, expand 2,
H = 32, P = 64, N = 128, vocab 50 304, B = 4, L = 4096) with the native SSD kernel swapped in, loss and
per-layer gradients compared with the reference. This file restates, in plain PyTorch, the model around the
SSD so that the comparison runs the reference's own composition:

* ``Mamba3Block`` follows ``r2/dhammic-ai/src/mamba_base_engine.py:34-192``: one in-projection split into
  (z, x, B, C, dt_raw, lam_raw, theta) (:63-71, :124), the trapezoidal coefficients (:128-130), RMSNorm on B and
  C (:133-134, eps 1e-6), per-head data-dependent RoPE of B/C with learnable per-head biases (:136-149),
  padding to the chunk (:154-165), the two SSD calls of the trapezoidal rule, the second reusing the first
  call's cache (:170-181), their sum (:183), ``+ D x`` (:187) and the gated output norm (eps 1e-6) and
  projection (:190-192).
* ``Layer`` follows ``MambaBlock`` (``src/citta_vithi_pipeline.py:159-190``): pre-norm residual layers with
  RMSNorm eps 1e-5 (:168-169) and a SwiGLU MLP of width int(2.5 d) (:175); the model ends in a final RMSNorm,
  eps 1e-5 (:290).
* The loss is the tied LM head and token cross-entropy of ``train.py:126-136`` with
  ``src/kernels/lmhead_xent.py:367-396``: logits = hidden W_embed^T accumulated in fp32, mean over the
  non-ignored targets (the fused kernel's chunking over the vocabulary does not change the value).
* ``trapezoidal`` follows ``src/kernels/trapezoidal.py:1-52``; ``rope`` follows ``src/kernels/rope.py:1-25``;
  ``rmsnorm`` follows ``src/kernels/rmsnorm.py:222-235`` (fp32 statistics, output in the input dtype).
* ``set_native`` switches the blocks to the native composition (``Mamba3Block.forward_native``: in-projection
  split, trapezoidal coefficients, RoPE, one trapezoidal scan with D and the gated norm fused, then out_proj)
  and optionally the loss to the fused LM head, for the tests that check that composition against this one.

The SSD function is a parameter with the reference's public signature
``ssd(x, A, B, C, chunk_size, initial_states=None, cache=None) -> (Y, final_state, cache)``, so the same model
runs on the native drop-in or on the oracle's restatement of the reference SSD.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F
import torch.utils.checkpoint


def rmsnorm(x, weight, eps=1e-6):
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * weight.float()).to(x.dtype)


class RMSNorm(nn.Module):
    def __init__(self, d, eps=1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(d))
        self.eps = eps

    def forward(self, x):
        return rmsnorm(x, self.weight, self.eps)


def trapezoidal(dt_raw, lam_raw, dt_bias, A_log):
    """(dt, dA, beta, gamma) in the dtype of dt_raw, computed in fp32 as the reference kernel does: the
    parameters cast to the input dtype first (trapezoidal.py:241-242), softplus as
    max(s, 0) + log(1 + exp(-|s|)) (:108-110)."""
    s = dt_raw.float() + dt_bias.to(dt_raw.dtype).float()
    dt = torch.clamp_min(s, 0.0) + torch.log(1.0 + torch.exp(-s.abs()))
    lam = 1.0 / (1.0 + torch.exp(-lam_raw.float()))
    A = -torch.exp(A_log.to(dt_raw.dtype).float())
    dA = dt * A
    beta = (1.0 - lam) * dt * torch.exp(dA)
    gamma = lam * dt
    return tuple(t.to(dt_raw.dtype) for t in (dt, dA, beta, gamma))


def rope(x, angles):
    """Rotate (even, odd) pairs of the last axis of x by angles (..., D/2); fp32 inside, x's dtype out."""
    xf, a = x.float(), angles.float()
    x1, x2 = xf[..., 0::2], xf[..., 1::2]
    c, s = torch.cos(a), torch.sin(a)
    return torch.stack([c * x1 - s * x2, s * x1 + c * x2], dim=-1).flatten(-2).to(x.dtype)


class Mamba3Block(nn.Module):
    def __init__(self, ssd, d_model, d_state, expand, n_heads, chunk_size, dtype=torch.bfloat16):
        super().__init__()
        self.ssd = ssd
        self.d_inner = d_model * expand
        self.n_heads = n_heads
        self.d_head = self.d_inner // n_heads
        self.d_state = d_state
        self.chunk_size = chunk_size
        self.split_sizes = [self.d_inner, self.d_inner, d_state, d_state, n_heads, n_heads, d_state // 2]
        self.in_proj = nn.Linear(d_model, sum(self.split_sizes), bias=False, dtype=dtype)
        self.A_log = nn.Parameter(torch.empty(n_heads).uniform_(-4, -1))
        self.D = nn.Parameter(torch.ones(n_heads))
        self.dt_bias = nn.Parameter(torch.empty(n_heads).uniform_(0.001, 0.1))
        self.B_norm = RMSNorm(d_state)
        self.C_norm = RMSNorm(d_state)
        self.B_bias = nn.Parameter(torch.ones(n_heads, d_state))
        self.C_bias = nn.Parameter(torch.ones(n_heads, d_state))
        self.out_proj = nn.Linear(self.d_inner, d_model, bias=False, dtype=dtype)
        self.norm = RMSNorm(self.d_inner)
        self.native = False

    def forward(self, x):
        if self.native:
            return self.forward_native(x)
        b, T, _ = x.shape
        x = x.to(self.in_proj.weight.dtype)
        z, x_ssm, B_proj, C_proj, dt_raw, lam_raw, theta = torch.split(self.in_proj(x), self.split_sizes, dim=-1)
        dt, dA, beta, gamma = trapezoidal(dt_raw, lam_raw, self.dt_bias, self.A_log)
        B_proj = self.B_norm(B_proj)
        C_proj = self.C_norm(C_proj)
        cum_angles = -torch.cumsum(dt.unsqueeze(-1) * theta.unsqueeze(2), dim=1)
        dtype = x_ssm.dtype
        B_h = rope(B_proj.unsqueeze(2) + self.B_bias, cum_angles).to(dtype)
        C_h = rope(C_proj.unsqueeze(2) + self.C_bias, cum_angles).to(dtype)
        x_heads = x_ssm.reshape(b, T, self.n_heads, self.d_head)
        pad = (self.chunk_size - T % self.chunk_size) % self.chunk_size
        x_p = F.pad(x_heads, (0, 0, 0, 0, 0, pad))
        dA_p = F.pad(dA, (0, 0, 0, pad))
        B_p = F.pad(B_h, (0, 0, 0, 0, 0, pad))
        C_p = F.pad(C_h, (0, 0, 0, 0, 0, pad))
        gamma_p = F.pad(gamma, (0, 0, 0, pad))
        beta_p = F.pad(beta, (0, 0, 0, pad))
        y_gamma, _, cache = self.ssd(x_p * gamma_p.unsqueeze(-1), dA_p, B_p, C_p, self.chunk_size)
        B_prev = F.pad(B_p[:, :-1], (0, 0, 0, 0, 1, 0))
        x_prev = F.pad(x_p[:, :-1], (0, 0, 0, 0, 1, 0))
        y_beta, _, _ = self.ssd(x_prev * beta_p.unsqueeze(-1), dA_p, B_prev, C_p, self.chunk_size, cache=cache)
        y = (y_gamma + y_beta)[:, :T]
        y = y + x_heads * self.D.to(dtype).view(1, 1, -1, 1)
        y = self.norm(y.reshape(b, T, -1)) * F.silu(z)
        return self.out_proj(y)

    def forward_native(self, x):
        """The same block on the native kernels: the in-projection split, the trapezoidal coefficients
        and the RoPE of B/C as HIP kernels, then one trapezoidal scan with + D x and the gated output
        norm in its last phase (no padding: the last chunk is partial), feeding out_proj."""
        import kernels
        b, T, _ = x.shape
        x = x.to(self.in_proj.weight.dtype)
        z, x_ssm, B_proj, C_proj, dt_raw, lam_raw, theta = kernels.fused_inproj_split(x, self.in_proj.weight,
                                                                                     self.split_sizes)
        dt, dA, beta, gamma = kernels.fused_trapezoidal(dt_raw, lam_raw, self.dt_bias, self.A_log)
        B_proj = self.B_norm(B_proj)
        C_proj = self.C_norm(C_proj)
        cum_angles = -torch.cumsum(dt.unsqueeze(-1) * theta.unsqueeze(2), dim=1)
        dtype = x_ssm.dtype
        # rotated in fp32 and rounded after, as the reference does (the bias gradients sum every token's
        # gradient with heavy cancellation, so a rounding before the rotation shows in them)
        ang = cum_angles.float()
        B_h = kernels.fused_rope(B_proj.unsqueeze(2) + self.B_bias, ang).to(dtype)
        C_h = kernels.fused_rope(C_proj.unsqueeze(2) + self.C_bias, ang).to(dtype)
        x_heads = x_ssm.reshape(b, T, self.n_heads, self.d_head)
        y = kernels.fused_trapezoidal_ssd_scan(x_heads, dA, gamma, beta, B_h, C_h, self.chunk_size, D=self.D, z=z,
                                               norm_weight=self.norm.weight, norm_eps=self.norm.eps)
        return self.out_proj(y.reshape(b, T, -1))


class SwiGLU(nn.Module):
    def __init__(self, d_model, hidden, dtype=torch.bfloat16):
        super().__init__()
        self.w_gate = nn.Linear(d_model, hidden, bias=False, dtype=dtype)
        self.w_up = nn.Linear(d_model, hidden, bias=False, dtype=dtype)
        self.w_down = nn.Linear(hidden, d_model, bias=False, dtype=dtype)

    def forward(self, x):
        return self.w_down(F.silu(self.w_gate(x)) * self.w_up(x))


class Layer(nn.Module):
    def __init__(self, ssd, d_model, d_state, expand, n_heads, chunk_size, mlp_hidden=None, dtype=torch.bfloat16):
        super().__init__()
        self.norm1 = RMSNorm(d_model, eps=1e-5)
        self.mixer = Mamba3Block(ssd, d_model, d_state, expand, n_heads, chunk_size, dtype=dtype)
        self.norm2 = RMSNorm(d_model, eps=1e-5)
        self.mlp = SwiGLU(d_model, mlp_hidden or int(d_model * 2.5), dtype=dtype)

    def forward(self, h):
        h = h + self.mixer(self.norm1(h))
        return h + self.mlp(self.norm2(h))


class Mamba3LM(nn.Module):
    """Embedding, ``n_layers`` layers, final RMSNorm, LM head tied to the embedding. ``checkpoint``
    recomputes each layer's forward in the backward (both SSD variants alike), bounding the memory of a
    24-layer step."""

    def __init__(self, ssd, vocab, d_model, n_layers, d_state, expand, n_heads, chunk_size, mlp_hidden=None,
                 dtype=torch.bfloat16, checkpoint=False):
        super().__init__()
        self.embed = nn.Embedding(vocab, d_model, dtype=dtype)
        nn.init.normal_(self.embed.weight, std=1.0 / d_model ** 0.5)
        self.layers = nn.ModuleList(
            [Layer(ssd, d_model, d_state, expand, n_heads, chunk_size, mlp_hidden, dtype) for _ in range(n_layers)])
        self.norm_f = RMSNorm(d_model, eps=1e-5)
        self.checkpoint = checkpoint
        self.native_head = False

    def loss(self, tokens, targets, ignore_index=-100):
        h = self.embed(tokens)
        for layer in self.layers:
            if self.checkpoint:
                h = torch.utils.checkpoint.checkpoint(layer, h, use_reentrant=False)
            else:
                h = layer(h)
        hidden = self.norm_f(h)
        if self.native_head:
            import kernels
            return kernels.fused_lmhead_xent(hidden, self.embed.weight, targets, ignore_index)
        logits = hidden.float() @ self.embed.weight.float().t()
        return F.cross_entropy(logits.reshape(-1, logits.shape[-1]), targets.reshape(-1), ignore_index=ignore_index)


def set_ssd(model, ssd):
    for layer in model.layers:
        layer.mixer.ssd = ssd


def set_native(model, blocks, head=False):
    """Run the blocks on the native kernels end to end (Mamba3Block.forward_native) and, with ``head``,
    the loss on the fused LM head (bf16 only)."""
    for layer in model.layers:
        layer.mixer.native = blocks
    model.native_head = head
