"""The decoder's attention core, written so that no batched product ever receives a
transposed right operand.

transformers' eager attention (the reference's choice, decoder.py:568-598) forms
``Q̃·K̃ᵀ`` with ``K̃ᵀ`` as a transposed view, and autograd's backward of every batched product
``A·B`` forms ``δC·Bᵀ`` with ``Bᵀ`` a transposed view. On this pool's MI355X boxes the platform
guidance is that bf16 batched products (``torch.bmm`` and what calls it) have faulted the GPU
when their right operand was a transposed view, so the bf16 prover cannot run them. This core
computes the same six products of the reference's inventory (``S``, ``O``, ``dA``, ``dV``,
``dQ``, ``dK``; reference decoder.py:416-471) with every right operand contiguous:

    forward:   S  = Q̃ · (K̃ᵀ)ᶜ          O  = A · Ṽ
    backward:  dA = δO · (Ṽᵀ)ᶜ         dV = Aᵀ · δO       (the pair of O's backward)
               dQ = δS · K̃             dK = δSᵀ · Q̃       (the pair of S's backward)

``(X)ᶜ`` is a contiguous copy. A left operand may be a transposed view (``Aᵀ``, ``δSᵀ``):
those share storage with ``O``'s and ``dQ``'s ``A``, which the verifier exploits. ``dK`` comes
out as the canonical ``[n, d_h]`` leaf directly (autograd's own form is ``Q̃ᵀ·δS``, its
transpose). Each backward issues its pair in the order shown, which the decoder's labeling
relies on; the two products of a pair share a tensor (``dA``'s ``A`` is ``dV``'s ``B``, and
``dQ``'s ``A`` is the storage of ``dK``'s ``A``).

The softmax, scaling, mask and the GQA head repetition are the eager attention's own
arithmetic (softmax in fp32, then the query's dtype), so the glue the verifier replays is the
same computation.
"""

from __future__ import annotations

import torch

__all__ = ["ATTENTION", "register", "attention_forward"]

ATTENTION = "pots_contiguous_bmm"


def _check_right(b: torch.Tensor) -> None:
    if not b.is_contiguous():
        raise RuntimeError("a batched product's right operand must be contiguous here")


class _Scores(torch.autograd.Function):
    """``S = Q̃·K̃ᵀ`` over stacked heads ``[BH, n, d_h]``."""

    @staticmethod
    def forward(ctx, q: torch.Tensor, k: torch.Tensor) -> torch.Tensor:
        kt = k.transpose(1, 2).contiguous()
        _check_right(kt)
        ctx.save_for_backward(q, k)
        return torch.bmm(q, kt)

    @staticmethod
    def backward(ctx, g: torch.Tensor):
        q, k = ctx.saved_tensors
        g = g.contiguous()
        _check_right(k)
        _check_right(q)
        dq = torch.bmm(g, k)                  # dQ = δS·K̃
        dk = torch.bmm(g.transpose(1, 2), q)  # dK = δSᵀ·Q̃
        return dq, dk


class _Mix(torch.autograd.Function):
    """``O = A·Ṽ`` over stacked heads (``A`` the attention probabilities ``[BH, n, n]``)."""

    @staticmethod
    def forward(ctx, p: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
        _check_right(v)
        ctx.save_for_backward(p, v)
        return torch.bmm(p, v)

    @staticmethod
    def backward(ctx, g: torch.Tensor):
        p, v = ctx.saved_tensors
        g = g.contiguous()
        vt = v.transpose(1, 2).contiguous()
        _check_right(vt)
        da = torch.bmm(g, vt)                 # dA = δO·Ṽᵀ
        dv = torch.bmm(p.transpose(1, 2), g)  # dV = Aᵀ·δO
        return da, dv


def _heads(x: torch.Tensor, rep: int) -> torch.Tensor:
    """``[B, H_kv, n, d]`` → ``[B·H_kv·rep, n, d]``, each KV head repeated ``rep`` times for its
    query heads (GQA), as one contiguous stack."""
    b, h, n, d = x.shape
    if rep > 1:
        x = x[:, :, None].expand(b, h, rep, n, d)
    return x.reshape(b * h * rep, n, d).contiguous()


def attention_forward(module: torch.nn.Module, query: torch.Tensor, key: torch.Tensor,
                      value: torch.Tensor, attention_mask: torch.Tensor | None,
                      scaling: float, dropout: float = 0.0, **kwargs):
    """transformers' attention-function signature: ``query [B, H, n, d_h]``, ``key`` and
    ``value [B, H_kv, n, d_h]``, an additive float mask ``[B, 1, n, n]`` or None; returns
    ``(output [B, n, H, d_h], probabilities [B, H, n, n])``."""
    if dropout:
        raise ValueError("attention dropout must be off: a step must be deterministic")
    b, h, n, d = query.shape
    rep = module.num_key_value_groups
    # The products' format: autocast's when it is on (RoPE leaves Q and K in fp32 there, and
    # eager attention's matmuls would cast them), else the query's.
    dev = query.device.type
    dt = torch.get_autocast_dtype(dev) if torch.is_autocast_enabled(dev) else query.dtype
    q = query.to(dt).reshape(b * h, n, d).contiguous()
    k = _heads(key.to(dt), rep)
    v = _heads(value.to(dt), rep)
    scores = _Scores.apply(q, k).view(b, h, n, n) * scaling
    if attention_mask is not None:
        scores = scores + attention_mask
    probs = torch.nn.functional.softmax(scores, dim=-1, dtype=torch.float32).to(dt)
    out = _Mix.apply(probs.reshape(b * h, n, n), v)
    return out.view(b, h, n, d).transpose(1, 2).contiguous(), probs


_REGISTERED = False


def register() -> str:
    """Register the core (and the eager causal mask it takes) with transformers under
    :data:`ATTENTION`; idempotent. Returns the implementation name for a model config."""
    global _REGISTERED
    if not _REGISTERED:
        from transformers import AttentionInterface
        from transformers.masking_utils import AttentionMaskInterface, eager_mask
        AttentionInterface.register(ATTENTION, attention_forward)
        AttentionMaskInterface.register(ATTENTION, eager_mask)
        _REGISTERED = True
    return ATTENTION
