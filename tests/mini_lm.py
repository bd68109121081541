"""A two-layer language model with the reference model's attention block, for full-model parity tests.

It mirrors the parts of ref: tnlm/model.py that touch attention: q1/k1 (and q2/k2 for the two-pair kinds) and v
projections viewed as (B, H, T, d) with `.transpose(1, 2)` (so v reaches the operator as a strided view), RoPE on
q/k from the position within document (ref: tnlm/attention.py:12-19,41-51), per-head `b` / `coef` parameters,
row power 1 for offset_square and 1/2 otherwise (ref: tnlm/model.py:54-56), the fast-path context of
ref: tnlm/model.py:205-227, and a bilinear MLP. backend="reference" runs the dense restatement of
ref: tnlm/attention.py:54-77 with autograd; backend="hip" goes through tensor_train_ing_amd.model_glue.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from tensor_train_ing_amd import model_glue

TWO_PAIRS = ("signed_product", "lower_degree_mix")


def doc_positions(doc: torch.Tensor) -> torch.Tensor:
    B, T = doc.shape
    ar = torch.arange(T, device=doc.device).expand(B, T)
    start = torch.ones_like(doc, dtype=torch.bool)
    start[:, 1:] = doc[:, 1:] != doc[:, :-1]
    return ar - torch.where(start, ar, torch.zeros_like(ar)).cummax(-1).values


def rope(x, cos, sin):
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat([x1 * cos - x2 * sin, x1 * sin + x2 * cos], dim=-1)


def dense_attention(kind, q1, k1, q2, k2, v, C, coef, b, degree):
    """P = C * A(S1, S2), y = P v; S = q k^T / sqrt(dk); mask and row scale after the polynomial."""
    sm = q1.shape[-1] ** -0.5
    S1 = q1 @ k1.transpose(-1, -2) * sm
    if kind == "signed_product":
        A = S1 * (q2 @ k2.transpose(-1, -2) * sm)
    elif kind == "lower_degree_mix":
        S2 = q2 @ k2.transpose(-1, -2) * sm
        c = coef[None, :, :, None, None]
        A = c[:, :, 0] + c[:, :, 1] * S1 + c[:, :, 2] * S2 + c[:, :, 3] * S1 * S2
    elif kind == "offset_square":
        A = (S1 + b[None, :, None, None]) ** 2
    else:
        A = S1 ** degree
    return (C * A).to(v.dtype) @ v


class Block(nn.Module):
    def __init__(self, kind, mlp, d_model, heads, d_key, d_value, d_mlp, degree):
        super().__init__()
        self.kind, self.degree, self.H, self.dk, self.dv = kind, degree, heads, d_key, d_value
        self.n1, self.n2 = nn.RMSNorm(d_model), nn.RMSNorm(d_model)
        self.q1, self.k1 = nn.Linear(d_model, heads * d_key, bias=False), nn.Linear(d_model, heads * d_key, bias=False)
        if kind in TWO_PAIRS:
            self.q2, self.k2 = (nn.Linear(d_model, heads * d_key, bias=False) for _ in range(2))
        self.v = nn.Linear(d_model, heads * d_value, bias=False)
        self.o = nn.Linear(heads * d_value, d_model, bias=False)
        if kind == "offset_square":
            self.b = nn.Parameter(torch.full((heads,), 0.5))
        if kind == "lower_degree_mix":
            self.coef = nn.Parameter(torch.tensor([[0.1, 0.2, -0.3, 1.0]]).repeat(heads, 1))
        self.row_power = 1.0 if kind == "offset_square" else 0.5
        bias = mlp == "affine_bilinear"
        self.l, self.r = nn.Linear(d_model, d_mlp, bias=bias), nn.Linear(d_model, d_mlp, bias=bias)
        self.d = nn.Linear(d_mlp, d_model, bias=bias)

    def _heads(self, x, lin, dh):
        B, T, _ = x.shape
        return lin(x).view(B, T, self.H, dh).transpose(1, 2)

    def attention(self, x, ctx):
        cos, sin = ctx["rope"]
        fused = ctx["backend"] != "reference"  # the HIP operator rotates q/k itself (rope=)
        rot = (lambda t: t) if fused else (lambda t: rope(t, cos, sin))  # noqa: E731
        q1 = rot(self._heads(x, self.q1, self.dk))
        k1 = rot(self._heads(x, self.k1, self.dk))
        q2 = k2 = None
        if self.kind in TWO_PAIRS:
            q2 = rot(self._heads(x, self.q2, self.dk))
            k2 = rot(self._heads(x, self.k2, self.dk))
        v = self._heads(x, self.v, self.dv)
        coef, b = getattr(self, "coef", None), getattr(self, "b", None)
        if ctx["backend"] == "reference":
            y = dense_attention(self.kind, q1, k1, q2, k2, v, ctx["C"][self.row_power], coef, b, self.degree)
        else:
            y = model_glue.attention(self.kind, q1, k1, q2, k2, v, ctx, self.row_power, coef=coef, b=b,
                                     degree=self.degree if self.kind == "power" else None, rope=ctx["rope"])
        B, H, T, dv = y.shape
        return self.o(y.transpose(1, 2).reshape(B, T, H * dv))

    def forward(self, x, ctx):
        x = x + self.attention(self.n1(x), ctx)
        h = self.n2(x)
        return x + self.d(self.l(h) * self.r(h))


class MiniLM(nn.Module):
    def __init__(self, kind, mlp="bilinear", layers=2, d_model=128, heads=2, d_key=64, d_value=64, d_mlp=96,
                 vocab_size=97, padded_vocab=128, backend="reference", degree=2):
        super().__init__()
        self.backend, self.vocab, self.dk = backend, vocab_size, d_key
        self.embed = nn.Embedding(padded_vocab, d_model)
        self.blocks = nn.ModuleList(Block(kind, mlp, d_model, heads, d_key, d_value, d_mlp, degree)
                                    for _ in range(layers))
        self.norm = nn.RMSNorm(d_model)
        self.unembed = nn.Linear(d_model, padded_vocab, bias=False)
        self.powers = sorted({blk.row_power for blk in self.blocks})

    def make_ctx(self, doc):
        pos = doc_positions(doc)
        inv = 1.0 / (10000.0 ** (torch.arange(0, self.dk, 2, device=doc.device, dtype=torch.float32) / self.dk))
        ang = pos.float()[..., None] * inv
        rope_tab = (ang.cos()[:, None], ang.sin()[:, None])
        if self.backend == "reference":
            T = doc.shape[1]
            causal = torch.ones(T, T, dtype=torch.bool, device=doc.device).tril()
            vis = causal & (doc[:, :, None] == doc[:, None, :]) & (doc[:, :, None] >= 0) & (doc[:, None, :] >= 0)
            n = vis.sum(-1, keepdim=True).clamp(min=1).float()
            C = {p: (vis.float() * n.pow(-p))[:, None] for p in self.powers}
            return {"rope": rope_tab, "backend": "reference", "C": C}
        ctx = model_glue.fast_context(doc, pos, self.powers, self.backend)
        ctx["rope"] = rope_tab
        return ctx

    def forward(self, idx, doc, tgt):
        ctx = self.make_ctx(doc)
        x = self.embed(idx)
        for blk in self.blocks:
            x = blk(x, ctx)
        logits = self.unembed(self.norm(x))[..., :self.vocab]
        return logits, F.cross_entropy(logits.reshape(-1, self.vocab).float(), tgt.reshape(-1), ignore_index=-100)
