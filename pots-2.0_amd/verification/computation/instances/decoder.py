"""The Llama/Qwen2 decoder's declared computation: leaf layout and product inventory only.

Reference: verification/computation/instances/decoder.py:154-160 (``matmul_count_decoder``),
:320-400 (weight names and shapes) and :416-471 (``_inventory``). The order of weights and
products, their shapes and their κ classes follow the reference exactly, since they fix which
leaf is which and what challenge width each product gets. The model itself (HF modules,
autocast, the replay that rebuilds operands) is outside this build.

Per layer: the q/k/v projections (with biases for Qwen2), ``n_s·n_h`` members each of
``S = Q·Kᵀ`` and ``O = A·V``, then o/gate/up/down; the head ``Λ = X·W_outᵀ`` in ``B`` row
blocks; then backward, layers in reverse: input and weight gradients of down/gate/up/o, the
members' ``dA, dV`` and ``dQ, dK``, and the input and weight gradients of q/k/v.
"""

from __future__ import annotations

from functools import cached_property

import torch

from verification.computation.interface import DeclaredComputation, ProductKind, ProductSpec

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

    def product_class(self, spec: ProductSpec) -> str:
        return self._inventory[1][spec.m - 1]


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
