"""The Llama/Qwen2 decoder's declared computation: leaf layout, product inventory, the
prover's labeling and the verifier's replay.

Reference: verification/computation/instances/decoder.py:154-160 (``matmul_count_decoder``),
:320-400 (weight names and shapes) and :416-471 (``_inventory``). The order of weights and
products, their shapes and their κ classes follow the reference exactly, since they fix which
leaf is which and what challenge width each product gets.

Per layer: the q/k/v projections (with biases for Qwen2), ``n_s·n_h`` members each of
``S = Q·Kᵀ`` and ``O = A·V``, then o/gate/up/down; the head ``Λ = X·W_outᵀ`` in ``B`` row
blocks; then backward, layers in reverse: input and weight gradients of down/gate/up/o, the
members' ``dA, dV`` and ``dQ, dK``, and the input and weight gradients of q/k/v.

The prover side (:meth:`DecoderComputation.build_model`, :meth:`~DecoderComputation.loss`,
:meth:`~DecoderComputation.label_with_operands`) runs transformers' Llama/Qwen2 causal LM over
fp32 master weights, under autocast to bf16 for a bf16 computation (reference
decoder.py:551-598), the output layer in ``B`` row blocks when ``head_blocks`` asks for them
(:meth:`~DecoderComputation.forward_backward`), with this build's attention core
(``instances/attention.py``: eager attention's arithmetic, every batched product's right
operand contiguous), and maps the captured records onto the slots above by operand identity.
:class:`DecoderReplay` rebuilds check 5's operands and check 6b's glue gradients from the
committed leaves (reference decoder.py:1142,1682-1751).
"""

from __future__ import annotations

from collections.abc import Sequence
from functools import cached_property
from typing import Any

import torch

from verification.computation.interface import (DeclaredComputation, LabelingError,
                                               ProductKind, ProductSpec, Replay, load_weights)
from verification.computation.substitution import (CallPlan, CommittedProducts, ReplayError,
                                                   plan_calls)

LINEARS = ("q", "k", "v", "o", "gate", "up", "down")
_LINEAR_PATH = {
    "q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj",
    "o": "self_attn.o_proj", "gate": "mlp.gate_proj", "up": "mlp.up_proj",
    "down": "mlp.down_proj",
}
_BIASED = ("q", "k", "v")
_E = "model.embed_tokens.weight"
_W_OUT = "lm_head.weight"
_GAMMA_FINAL = "model.norm.weight"


def matmul_count_decoder(L: int, n_s: int, n_h: int, blocks: int = 1) -> int:
    """Products per step, ``M = L(21 + 6·n_s·n_h) + 3B``."""
    return L * (21 + 6 * n_s * n_h) + 3 * blocks


class DecoderComputation(DeclaredComputation):
    """``C`` for a decoder of the given shape and batch ``n_s × n``."""

    def __init__(self, *, L: int, d: int, d_f: int, n_h: int, n_kv: int, n_v: int,
                 n_s: int, n: int, d_h: int | None = None, tied: bool = True,
                 qkv_bias: bool = False, compute_dtype: torch.dtype = torch.float32,
                 head_blocks: int = 1, eta: float = 1e-4) -> None:
        if n_h % n_kv:
            raise ValueError(f"n_h={n_h} is not a multiple of n_kv={n_kv}")
        if head_blocks < 1 or n_s % head_blocks:
            raise ValueError(f"head_blocks {head_blocks} must divide n_s {n_s}")
        self.L, self.d, self.d_f, self.n_h, self.n_kv, self.n_v = L, d, d_f, n_h, n_kv, n_v
        self.d_h = d_h or d // n_h
        self._n_s, self.n = n_s, n
        self.tied, self.qkv_bias = tied, qkv_bias
        self.compute_dtype = compute_dtype
        self.head_blocks = head_blocks
        if not (isinstance(eta, float) and 0.0 < eta < float("inf")):
            raise ValueError(f"eta must be a positive finite float, got {eta!r}")
        self._eta = eta
        self.validate()

    # ---- the layout ---------------------------------------------------------------------

    @property
    def n_s(self) -> int:
        return self._n_s

    @property
    def N(self) -> int:
        return self.n_s * self.n

    @property
    def eta(self) -> float:
        return self._eta

    @cached_property
    def linear_weights(self) -> dict[str, tuple[int, ...]]:
        """Each linear weight's weight-gradient products (reference decoder.py:522-528): one
        ``L{l}.G_{x}`` per layer weight, and the head's row blocks when the head is untied."""
        by_name = {spec.name: spec.m for spec in self.products}
        out = {self.w(l, x): (by_name[f"L{l}.G_{x}"],)
               for l in range(1, self.L + 1) for x in LINEARS}
        if not self.tied:
            out[_W_OUT] = tuple(by_name[self.head_name("G", b)]
                                for b in range(self.head_blocks))
        return out

    @property
    def weight_dtype(self) -> torch.dtype:
        return torch.float32

    @property
    def product_dtype(self) -> torch.dtype:
        return self.compute_dtype

    @property
    def operand_dtype(self) -> torch.dtype:
        return self.compute_dtype

    def w(self, l: int, x: str) -> str:
        return f"model.layers.{l - 1}.{_LINEAR_PATH[x]}.weight"

    def bias(self, l: int, x: str) -> str | None:
        if self.qkv_bias and x in _BIASED:
            return f"model.layers.{l - 1}.{_LINEAR_PATH[x]}.bias"
        return None

    def linear_shape(self, x: str) -> tuple[int, int]:
        """``(out, in)`` of ``W_x``."""
        q_out, kv_out = self.n_h * self.d_h, self.n_kv * self.d_h
        return {"q": (q_out, self.d), "k": (kv_out, self.d), "v": (kv_out, self.d),
                "o": (self.d, q_out), "gate": (self.d_f, self.d), "up": (self.d_f, self.d),
                "down": (self.d, self.d_f)}[x]

    @property
    def w_out(self) -> str:
        return _E if self.tied else _W_OUT

    @cached_property
    def weight_names(self) -> tuple[str, ...]:
        names = [_E]
        for l in range(1, self.L + 1):
            names.append(f"model.layers.{l - 1}.input_layernorm.weight")
            for x in ("q", "k", "v", "o"):
                names.append(self.w(l, x))
                b = self.bias(l, x)
                if b is not None:
                    names.append(b)
            names.append(f"model.layers.{l - 1}.post_attention_layernorm.weight")
            names += [self.w(l, x) for x in ("gate", "up", "down")]
        names.append(_GAMMA_FINAL)
        if not self.tied:
            names.append(_W_OUT)
        return tuple(names)

    @cached_property
    def weight_shapes(self) -> dict[str, tuple[int, ...]]:
        shapes: dict[str, tuple[int, ...]] = {_E: (self.n_v, self.d), _GAMMA_FINAL: (self.d,),
                                              _W_OUT: (self.n_v, self.d)}
        for l in range(1, self.L + 1):
            shapes[f"model.layers.{l - 1}.input_layernorm.weight"] = (self.d,)
            shapes[f"model.layers.{l - 1}.post_attention_layernorm.weight"] = (self.d,)
            for x in LINEARS:
                shapes[self.w(l, x)] = self.linear_shape(x)
                b = self.bias(l, x)
                if b is not None:
                    shapes[b] = self.linear_shape(x)[:1]
        return {name: shapes[name] for name in self.weight_names}

    # ---- the inventory --------------------------------------------------------------------

    def head_name(self, kind: str, b: int) -> str:
        base = {"Lambda": "Lambda", "dF": "dF", "G": "G_E_head" if self.tied else "G_head"}[kind]
        return base if self.head_blocks == 1 else f"{base}[{b}]"

    @cached_property
    def _inventory(self) -> tuple[tuple[ProductSpec, ...], tuple[str, ...]]:
        N, n, d_h, d, n_v = self.N, self.n, self.d_h, self.d, self.n_v
        fwd, ig, wg, og = (ProductKind.FORWARD, ProductKind.INPUT_GRAD, ProductKind.WEIGHT_GRAD,
                           ProductKind.OPERAND_GRAD)
        rows: list[tuple] = []
        members = [(s, h) for s in range(self.n_s) for h in range(self.n_h)]

        def linear(l: int, x: str, kind: ProductKind) -> None:
            o, i = self.linear_shape(x)
            a, b = {fwd: ((N, i), (i, o)), ig: ((N, o), (o, i)), wg: ((o, N), (N, i))}[kind]
            role = {fwd: "Y", ig: "dX", wg: "G"}[kind] + f"_{x}"
            rows.append((f"L{l}.{role}", kind, a, b, self.w(l, x), l, None, role))

        for l in range(1, self.L + 1):
            for x in ("q", "k", "v"):
                linear(l, x, fwd)
            for s, h in members:
                rows.append((f"L{l}.S[{s},{h}]", fwd, (n, d_h), (d_h, n), None, l, (s, h), "S"))
            for s, h in members:
                rows.append((f"L{l}.O[{s},{h}]", fwd, (n, n), (n, d_h), None, l, (s, h), "O"))
            for x in ("o", "gate", "up", "down"):
                linear(l, x, fwd)
        R, B = N // self.head_blocks, self.head_blocks
        g_head = "G_E_head" if self.tied else "G_head"
        for b in range(B):
            rows.append((self.head_name("Lambda", b), fwd, (R, d), (d, n_v), self.w_out, None,
                         None, "Lambda"))
        for b in range(B):
            rows.append((self.head_name("dF", b), ig, (R, n_v), (n_v, d), self.w_out, None, None,
                         "dF"))
            rows.append((self.head_name("G", b), wg, (n_v, R), (R, d), self.w_out, None, None,
                         g_head))
        for l in range(self.L, 0, -1):
            for x in ("down", "gate", "up", "o"):
                linear(l, x, ig)
                linear(l, x, wg)
            for s, h in members:
                rows.append((f"L{l}.dA[{s},{h}]", og, (n, d_h), (d_h, n), None, l, (s, h), "dA"))
                rows.append((f"L{l}.dV[{s},{h}]", og, (n, n), (n, d_h), None, l, (s, h), "dV"))
            for s, h in members:
                rows.append((f"L{l}.dQ[{s},{h}]", og, (n, n), (n, d_h), None, l, (s, h), "dQ"))
                rows.append((f"L{l}.dK[{s},{h}]", og, (n, n), (n, d_h), None, l, (s, h), "dK"))
            for x in ("q", "k", "v"):
                linear(l, x, ig)
                linear(l, x, wg)
        biases = {self.w(l, x): b for l in range(1, self.L + 1) for x in LINEARS
                  if (b := self.bias(l, x)) is not None}
        specs = tuple(ProductSpec(m, name, kind, a, b, weight=w, layer=l, member=mem,
                                  bias=biases.get(w) if kind is fwd else None)
                      for m, (name, kind, a, b, w, l, mem, _) in enumerate(rows, start=1))
        return specs, tuple(r[-1] for r in rows)

    @property
    def products(self) -> tuple[ProductSpec, ...]:
        return self._inventory[0]

    @cached_property
    def operand_twins(self) -> dict[int, int]:
        """``{m₂: m₁}`` for the products whose ``A`` is, in a training step, the transpose of
        an earlier product's ``A`` (the same tensor): ``dV`` reads ``O``'s attention
        probabilities, ``dK`` reads ``dQ``'s ``δS``, a linear's ``G`` reads its ``dX``'s output
        gradient, and the head's weight gradient reads ``dF``'s logits gradient. The verifier
        finds such pairs from the operands themselves; this map lets a synthetic transcript
        lay its operands out the same way."""
        by_name = {spec.name: spec.m for spec in self.products}
        out: dict[int, int] = {}
        members = [(s, h) for s in range(self.n_s) for h in range(self.n_h)]
        for l in range(1, self.L + 1):
            for s_, h in members:
                out[by_name[f"L{l}.dV[{s_},{h}]"]] = by_name[f"L{l}.O[{s_},{h}]"]
                out[by_name[f"L{l}.dK[{s_},{h}]"]] = by_name[f"L{l}.dQ[{s_},{h}]"]
            for x in LINEARS:
                out[by_name[f"L{l}.G_{x}"]] = by_name[f"L{l}.dX_{x}"]
        for b in range(self.head_blocks):
            out[by_name[self.head_name("G", b)]] = by_name[self.head_name("dF", b)]
        return out

    def product_class(self, spec: ProductSpec) -> str:
        return self._inventory[1][spec.m - 1]

    # ---- prover side ----------------------------------------------------------------------

    def build_model(self) -> torch.nn.Module:
        """transformers' causal LM of this shape (Qwen2 with q/k/v biases, else Llama), random
        init, in the weights' dtype (the fp32 masters the layout declares), in eval mode (no
        dropout), on the current default device. A bf16 computation runs it under autocast
        (:meth:`loss`), as the reference does (decoder.py:551-598).

        Attention runs through this build's own core (``instances/attention.py``) instead of
        transformers' eager function: the same products and glue, with no batched product
        ever given a transposed right operand."""
        from transformers import LlamaConfig, LlamaForCausalLM, Qwen2Config, Qwen2ForCausalLM

        from verification.computation.instances.attention import register
        cfg_cls, model_cls = (Qwen2Config, Qwen2ForCausalLM) if self.qkv_bias else \
            (LlamaConfig, LlamaForCausalLM)
        cfg = cfg_cls(vocab_size=self.n_v, hidden_size=self.d, intermediate_size=self.d_f,
                      num_hidden_layers=self.L, num_attention_heads=self.n_h,
                      num_key_value_heads=self.n_kv, head_dim=self.d_h,
                      max_position_embeddings=max(self.n, 16), tie_word_embeddings=self.tied)
        if not self.qkv_bias:
            cfg.attention_bias = False
            cfg.mlp_bias = False
        cfg._attn_implementation = register()
        cfg.attention_dropout = 0.0
        model = model_cls(cfg).to(self.weight_dtype).eval()
        active = [name for name, mod in model.named_modules()
                  if isinstance(mod, torch.nn.Dropout) and mod.p > 0]
        if active:
            raise ValueError(f"dropout is active in {active[:3]}: a step must be deterministic")
        return model

    def autocast(self, device: torch.device):
        """The compute format over the fp32 masters: autocast to it on ``device``'s type, or
        nothing when the two are the same (reference decoder.py:551-556)."""
        import contextlib
        if self.compute_dtype == self.weight_dtype:
            return contextlib.nullcontext()
        return torch.autocast(device.type, dtype=self.compute_dtype)

    def _autocast_off(self, device: torch.device):
        """Autocast switched off inside an autocast region (a head block's backward)."""
        import contextlib
        if self.compute_dtype == self.weight_dtype:
            return contextlib.nullcontext()
        return torch.autocast(device.type, enabled=False)

    @staticmethod
    def _batch(records, dev: torch.device) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        ids = torch.stack([r.ids for r in records]).to(device=dev, dtype=torch.long)
        targets = torch.stack([r.targets for r in records]).to(device=dev, dtype=torch.long)
        mask = torch.stack([r.mask for r in records]).to(device=dev, dtype=torch.float32)
        return ids, targets, mask

    def _block_loss(self, logits: torch.Tensor, targets: torch.Tensor, mask: torch.Tensor,
                    total: torch.Tensor) -> torch.Tensor:
        """The masked cross-entropy of some rows over the whole batch's mask count, in fp32:
        the shares of a partition of the batch sum to the loss (reference decoder.py:638-649)."""
        ce = torch.nn.functional.cross_entropy(logits.float().reshape(-1, self.n_v),
                                               targets.reshape(-1), reduction="none")
        return (ce * mask.reshape(-1)).sum() / total

    def loss(self, model: torch.nn.Module, records) -> torch.Tensor:
        """Mean cross-entropy of the targets over the masked tokens; the model runs in the
        compute format, the loss in fp32."""
        dev = next(model.parameters()).device
        ids, targets, mask = self._batch(records, dev)
        with self.autocast(dev):
            logits = model(input_ids=ids).logits
        return self._block_loss(logits, targets, mask, mask.sum())

    def forward_backward(self, model: torch.nn.Module, records, stage) -> torch.Tensor:
        """One training pass. With one head block, the loss over the whole batch and its
        backward. With ``B = head_blocks`` blocks (reference decoder.py:740-770): the features
        ``F`` (embedding through the final norm) once; then per block ``b`` (sequences
        ``b·n_s/B`` onwards), its rows of ``F`` copied off ``F``'s graph, ``Λ_b`` and the
        block's share of the loss, and right away that share's gradients: ``dF_b`` and the
        head weight's ``G_b`` (then the block's logits are dropped, so no ``N × n_v`` array
        is held); the head weight's gradient is the blocks' ``G_b`` widened to the weight
        dtype and added in block order, plus (tied) the embedding's own; ``F``'s backward
        takes the blocks' ``dF_b`` stacked. The head weight is cast to the compute format once
        for all blocks; the backward runs with autocast off."""
        if self.head_blocks == 1:
            return super().forward_backward(model, records, stage)
        dev = next(model.parameters()).device
        ids, targets, mask = self._batch(records, dev)
        total = mask.sum()
        head = model.get_output_embeddings()
        w = head.weight
        per = self.n_s // self.head_blocks
        loss: torch.Tensor | None = None
        g: torch.Tensor | None = None
        dfs: list[torch.Tensor] = []
        with self.autocast(dev):
            with stage("forward"):
                f = model.model(input_ids=ids).last_hidden_state
            for b in range(self.head_blocks):
                rows = slice(b * per, (b + 1) * per)
                with stage("forward"):
                    fb = f.detach()[rows].clone().requires_grad_()
                    part = self._block_loss(head(fb), targets[rows], mask[rows], total)
                with stage("backward"), self._autocast_off(dev):
                    df, gb = torch.autograd.grad(part, [fb, w])
                dfs.append(df)
                g = gb.to(self.weight_dtype) if g is None else g + gb.to(self.weight_dtype)
                part = part.detach()
                loss = part if loss is None else loss + part
                del fb, df, gb, part
            with stage("backward"), self._autocast_off(dev):
                f.backward(torch.cat(dfs))
            del f, dfs
        w.grad = g if w.grad is None else g + w.grad
        return loss

    def label(self, capture, model: torch.nn.Module) -> list[torch.Tensor]:
        return self.label_with_operands(capture, model)[0]

    # ---- verifier side --------------------------------------------------------------------

    def replay(self, leaves: Any) -> Replay:
        """Check 5's operands: the prover's captured ones when given (``use_operands``), else
        the replay of the committed leaves (:class:`DecoderReplay`)."""
        given = getattr(self, "_operands", None)
        return given if given is not None else DecoderReplay(self, leaves)

    def call_plan(self, model: torch.nn.Module, records: Sequence[Any]) -> CallPlan:
        """Which call of a training pass fills which slot; the same for every step of this
        computation, so it is planned once (``substitution.plan_calls``)."""
        plan = getattr(self, "_call_plan", None)
        if plan is None:
            plan = self._call_plan = plan_calls(self, model, records)
        return plan

    def label_with_operands(self, capture, model: torch.nn.Module,
                            call_slots: dict[int, list[tuple[int | None, str, bool]]] | None
                            = None
                            ) -> tuple[list[torch.Tensor], dict[int, tuple[torch.Tensor,
                                                                           torch.Tensor]]]:
        """``(P_1..P_M, {m: (A_m, B_m)})`` from the capture, mapped by operand identity
        (reference decoder.py:774-1100 maps the same slots from eager attention's forms).

        Linear products: a forward's ``B`` views its weight, or autocast's copy of it; an
        input gradient's ``B`` is that weight (or copy); a weight gradient's output is the
        weight's ``.grad``, or under autocast the product whose whole output ``.grad`` copies
        to fp32. The head's ``B`` is ``W_out``; the tied head's weight gradient is the product
        whose ``B`` is the head's input. Attention (the core in ``instances/attention.py``):
        the two batched products after layer ``ℓ``'s q/k/v are ``S`` then ``O``; in backward,
        ``dV`` reads ``O``'s ``A`` (transposed) and ``dA`` is the product whose ``A`` is
        ``dV``'s ``B`` (``δO``); ``dK`` reads ``S``'s ``A`` as its ``B`` and ``dQ`` is the other
        product over ``dK``'s ``A`` storage (``δS``).

        ``call_slots``, when given, receives for each labeled call (by capture index) the slots
        its output fills: ``(member index or None, slot name, transposed)``; this core fills
        no slot transposed.
        """
        if len(capture.glue_outer) > 1:
            raise LabelingError(f"{len(capture.glue_outer)} q=1 products; only the rotary "
                                f"table's is expected")
        if any(r.a is None for r in capture.records):
            raise LabelingError("the capture's operands were released before labeling")
        by_weight = {self.w(l, x): (l, x) for l in range(1, self.L + 1) for x in LINEARS}
        slots: dict[str, tuple[torch.Tensor, torch.Tensor, torch.Tensor]] = {}
        spec_by_name = {s.name: s for s in self.products}

        def fill(name, a, b, p, rec, member=None):
            if call_slots is not None:
                call_slots.setdefault(rec.index, []).append((member, name, False))
            if name in slots:
                raise LabelingError(f"slot {name} filled twice")
            spec = spec_by_name.get(name)
            if spec is None:
                raise LabelingError(f"no declared slot {name}")
            got = (tuple(a.shape), tuple(b.shape), tuple(p.shape))
            want = (spec.a_shape, spec.b_shape, spec.p_shape)
            if got != want:
                raise LabelingError(f"{name}: shapes {got} != declared {want}")
            slots[name] = (a, b, p)

        def members(role, l, rec):
            if rec.batch != self.n_s * self.n_h:
                raise LabelingError(f"L{l}.{role}: a batch of {rec.batch}, expected "
                                    f"{self.n_s * self.n_h}")
            for i, (a, b, p) in enumerate(rec.members()):
                s_, h = divmod(i, self.n_h)
                fill(f"L{l}.{role}[{s_},{h}]", a, b, p, rec, i)

        def weight_of(info) -> str | None:
            return info.param_name or info.param_copy

        def storage(t):
            return t.untyped_storage().data_ptr()

        fwd = [r for r in capture.records if r.phase == "forward"]
        bwd = [r for r in capture.records if r.phase == "backward"]
        s_rec: dict[int, Any] = {}
        o_rec: dict[int, Any] = {}
        head_in: dict[int, int] = {}  # storage of each head block's A -> its block
        layer = None
        seen = 0
        for rec in fwd:
            name = weight_of(rec.b_info)
            if rec.batch is not None:
                if layer is None:
                    raise LabelingError(f"batched record #{rec.index} before any layer")
                seen += 1
                if seen == 1:
                    s_rec[layer] = rec
                elif seen == 2:
                    o_rec[layer] = rec
                else:
                    raise LabelingError(f"layer {layer}: more than two forward batched products")
            elif name in by_weight:
                l, x = by_weight[name]
                if x == "q":
                    layer, seen = l, 0
                fill(f"L{l}.Y_{x}", rec.a, rec.b, rec.out, rec)
            elif name == self.w_out and rec.out.shape[-1] == self.n_v:
                b = len(head_in)
                if b >= self.head_blocks or storage(rec.a) in head_in:
                    raise LabelingError(f"head record #{rec.index}: more than "
                                        f"{self.head_blocks} head blocks, or one A twice")
                head_in[storage(rec.a)] = b
                fill(self.head_name("Lambda", b), rec.a, rec.b, rec.out, rec)
            else:
                raise LabelingError(f"forward record #{rec.index} matches no slot")
        for l in range(1, self.L + 1):
            if l not in s_rec or l not in o_rec:
                raise LabelingError(f"layer {l}: the attention products were not seen")
            members("S", l, s_rec[l])
            members("O", l, o_rec[l])

        # which weight's gradient each record's output became (its own storage, or the
        # fp32 copy autocast makes of it)
        grad_of: dict[int, str] = {}
        for pname, prm in model.named_parameters():
            if prm.grad is None:
                continue
            i = capture.output_copied_by(prm.grad)
            if i is None:
                i = capture.produced_by(prm.grad)
            if i is not None:
                grad_of[i] = pname
        o_a = {storage(o_rec[l].a): l for l in o_rec}
        s_a = {storage(s_rec[l].a): l for l in s_rec}
        pair_a: dict[int, tuple[str, int]] = {}  # storage of δO or δS -> (role, layer)
        deferred = []
        n_df = 0
        for rec in bwd:
            if rec.batch is not None:
                if storage(rec.a) in o_a:
                    l = o_a[storage(rec.a)]
                    members("dV", l, rec)
                    pair_a[storage(rec.b)] = ("dA", l)
                elif storage(rec.b) in s_a:
                    l = s_a[storage(rec.b)]
                    members("dK", l, rec)
                    pair_a[storage(rec.a)] = ("dQ", l)
                else:
                    deferred.append(rec)
                continue
            name = weight_of(rec.b_info)
            if name in by_weight:
                l, x = by_weight[name]
                fill(f"L{l}.dX_{x}", rec.a, rec.b, rec.out, rec)
            elif name == self.w_out:
                if n_df >= self.head_blocks:
                    raise LabelingError(f"backward record #{rec.index}: more than "
                                        f"{self.head_blocks} head input gradients")
                fill(self.head_name("dF", n_df), rec.a, rec.b, rec.out, rec)
                n_df += 1
            elif grad_of.get(rec.index) in by_weight:
                l, x = by_weight[grad_of[rec.index]]
                fill(f"L{l}.G_{x}", rec.a, rec.b, rec.out, rec)
            elif storage(rec.b) in head_in and tuple(rec.out.shape) == (self.n_v, self.d):
                fill(self.head_name("G", head_in[storage(rec.b)]), rec.a, rec.b, rec.out, rec)
            else:
                raise LabelingError(f"backward record #{rec.index} matches no slot")
        for rec in deferred:
            role = pair_a.get(storage(rec.a))
            if role is None:
                raise LabelingError(f"backward batched record #{rec.index} matches no slot")
            members(role[0], role[1], rec)
        missing = [s.name for s in self.products if s.name not in slots]
        if missing:
            raise LabelingError(f"{len(missing)} slots never filled, e.g. {missing[:3]}")
        products = [slots[s.name][2] for s in self.products]
        operands = {s.m: slots[s.name][:2] for s in self.products}
        return products, operands


class DecoderReplay(Replay):
    """The verifier's glue replay of one decoder step, from the committed leaves only
    (reference decoder.py:1142-1751, checks 3, 5 and 6b).

    The model is built at the computation's shape and loaded with the committed ``W_t``; one
    training pass on the committed batch runs with every checked product replaced by its
    committed leaf (``substitution.CommittedProducts``), so every operand a product receives
    (``X·`` after RMSNorm, ``Q̃, K̃`` after RoPE and ``repeat_kv``, the attention
    probabilities, ``δY`` through SiLU and softmax, …) is glue recomputed from committed
    values. The operands are kept as the ops received them and served in any order, each
    checked unchanged since; the backward leaves each glue weight's full gradient (the norms'
    γ, the biases and, tied, the embedding: its own backward plus the committed ``G_E_head``)
    for check 6b. A pass that departs from the plan is :class:`ReplayError`, a verifier bug;
    a leaf that fails to read raises its own error, which check 5 maps to a rejection.
    """

    def __init__(self, computation: DecoderComputation, leaves: Any,
                 device: torch.device | str | None = None) -> None:
        c = self.c = computation
        self.leaves = leaves
        if device is None:
            device = torch.device("cuda", torch.cuda.current_device()) \
                if torch.cuda.is_available() else "cpu"
        self.device = torch.device(device)
        records = [self._get(c.record_index(i)) for i in range(c.n_s)]
        with self.device:
            model = c.build_model()
        load_weights(c, model, {n: self._get(c.w_t_index(n)) for n in c.weight_names})
        plan = c.call_plan(model, records)
        index = {spec.name: c.product_index(spec.m) for spec in c.products}
        mode = CommittedProducts(plan, lambda slot: self._get(index[slot]))
        model.zero_grad(set_to_none=True)
        with torch.enable_grad(), mode:
            c.forward_backward(model, records, mode.phase)
        if mode.calls != plan.n_calls or len(mode.held) != c.M:
            raise ReplayError(f"the replay made {mode.calls} calls for {len(mode.held)} slots; "
                              f"the plan has {plan.n_calls} calls for {c.M}")
        self._held = mode.held
        self._batched = mode.batched
        self._glue = {}
        for name in c.glue_gradient_weights:
            g = model.get_parameter(name).grad
            if g is None:
                raise ReplayError(f"the replay's backward left no gradient for {name}")
            self._glue[name] = g.detach()

    def _get(self, index: int) -> Any:
        reader = getattr(self.leaves, "leaf", None)
        obj = reader(index) if reader is not None else self.leaves[index]
        return obj.to(self.device) if isinstance(obj, torch.Tensor) else obj

    def operands(self, m: int) -> tuple[torch.Tensor, torch.Tensor]:
        name = self.c.product(m).name
        a, b, va, vb = self._held[name]
        if a._version != va or b._version != vb:
            raise ReplayError(f"an operand of {name} changed after its product read it")
        return a, b

    def operand_group(self, ms: Sequence[int],
                      dtype: torch.dtype | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """The members of one batched product (every member of one attention call, in batch
        order) served as the call's whole operands, after one version check of each (reference
        decoder.py:1695-1751 serves the same group, copied); any other ``ms`` takes the
        default."""
        c = self.c
        names = tuple(c.product(m).name for m in ms)
        got = self._batched.get(names[0]) if names and dtype is None else None
        if got is None or got[0] != names:
            return super().operand_group(ms, dtype)
        _, a, b, va, vb, flipped = got
        if a._version != va or b._version != vb:
            raise ReplayError(f"an operand of {names[0]} changed after its product read it")
        return (b.transpose(1, 2), a.transpose(1, 2)) if flipped else (a, b)

    def glue_gradients(self) -> dict[str, torch.Tensor]:
        """Each glue weight's full gradient from the replay's backward."""
        return dict(self._glue)


# The configurations the benchmark and the tests use.
def smollm2_135m(n_s: int = 4, n: int = 256) -> DecoderComputation:
    return DecoderComputation(L=30, d=576, d_f=1536, n_h=9, n_kv=3, n_v=49152, n_s=n_s, n=n,
                              tied=True, qkv_bias=False, compute_dtype=torch.float32)


def qwen2_0_5b_shape(n_s: int = 8, n: int = 1024) -> DecoderComputation:
    return DecoderComputation(L=24, d=896, d_f=4864, n_h=14, n_kv=2, n_v=151936, n_s=n_s, n=n,
                              tied=True, qkv_bias=True, compute_dtype=torch.bfloat16)


def qwen2_1_5b_shape(n_s: int = 4, n: int = 2048) -> DecoderComputation:
    return DecoderComputation(L=28, d=1536, d_f=8960, n_h=12, n_kv=2, n_v=151936, n_s=n_s,
                              n=n, d_h=128, tied=True, qkv_bias=True,
                              compute_dtype=torch.bfloat16)
