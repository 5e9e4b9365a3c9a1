"""Constant-weight MoE layers whose decode and prefill outputs have a closed form.

Every expert matrix is a constant: q4nx with scale 0 and the constant as the group
minimum (``quant/q4nx.py:160-175``: a group whose maximum equals its bf16 floor gets
scale 0 and codes 0), so every output row of a projection is ``c * sum(x)``.  With

* hidden states on the bf16 grid in [1, 4) (so every fp32 sum over H of them is exact
  in any order: H * 4 < 2^13 on a 2^-7 grid),
* gate constants large enough that ``g >= 17`` (``sigmoid(g) == 1`` exactly in fp32, so
  SwiGLU is the exact product ``g * u``),
* a router whose rows are ``2^-11`` on the k chosen experts and 0 elsewhere (the chosen
  experts have equal positive logits, the others 0: the top-k set is fixed, and the
  renormalised weights are exactly 1/k for k a power of two),

every value of the layer is a short chain of exact fp32 operations and bf16 roundings
that this module evaluates with Python scalars and torch's bf16 conversion -- a
restatement from the reference's text (``host/raon.py:1288-1330`` for a token,
``host/backend.py:466-510`` for the ascending-id fp32 combine, ``:402-417`` for one
projection), independent of ``oracle.moe``'s array code.  All output rows of a layer
are equal, so the state of a whole stack is one scalar per layer plus the elementwise
residual add.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch


def bf16(v: float) -> float:
    """Round a float32 value to bf16 (RNE) with torch's conversion."""
    return float(torch.tensor(np.float32(v), dtype=torch.float32).to(torch.bfloat16).to(torch.float32))


def f32(v: float) -> float:
    return float(np.float32(v))


@dataclass
class ConstLayer:
    """One layer: the chosen routed experts and each expert's gate/up/down constants
    (index ``n_routed`` is the shared expert)."""

    hidden: int
    inter: int
    n_routed: int
    top_k: int
    chosen: list
    cg: list
    cu: list
    cd: list

    def router_f32(self) -> np.ndarray:
        w = np.zeros((self.n_routed, self.hidden), np.float32)
        w[self.chosen] = 2.0 ** -11
        return w

    def router_bf16(self) -> np.ndarray:
        return (self.router_f32().view(np.uint32) >> 16).astype(np.uint16)

    def gate_up_f32(self, e: int) -> np.ndarray:
        w = np.empty((2 * self.inter, self.hidden), np.float32)
        w[: self.inter] = self.cg[e]
        w[self.inter:] = self.cu[e]
        return w

    def down_f32(self, e: int, inter_pad: int) -> np.ndarray:
        d = np.zeros((self.hidden, inter_pad), np.float32)
        d[:, : self.inter] = self.cd[e]
        return d


def make_const_layer(hidden: int, inter: int, n_routed: int, top_k: int, seed: int) -> ConstLayer:
    """Seeded constants; ``top_k`` must be a power of two (renormalised weights 1/k exact)."""
    if top_k & (top_k - 1):
        raise ValueError("top_k must be a power of two for the exact 1/k weights")
    rng = np.random.default_rng(seed)
    chosen = sorted(int(e) for e in rng.choice(n_routed, top_k, replace=False))
    n = n_routed + 1
    # bf16-exact constants: a power of two times a 2- or 3-bit mantissa.
    a_g = -int(np.log2(hidden)) + 5          # g = c_g * S >= 32 for S >= hidden
    a_u = -int(np.round(np.log2(1.5 * hidden)))
    a_d = -8 - int(np.ceil(np.log2(inter * 70.0)))  # expert rows of ~2^-8: h grows slowly
    cg = [2.0 ** a_g * (4 + e % 4) / 4 for e in range(n)]
    cu = [2.0 ** a_u * (4 + (e // 4) % 4) / 4 for e in range(n)]
    cd = [2.0 ** a_d * (8 + e % 8) / 8 for e in range(n)]
    return ConstLayer(hidden, inter, n_routed, top_k, chosen, cg, cu, cd)


def expert_row(lay: ConstLayer, e: int, s: float) -> float:
    """Every output row of expert e for an input whose element sum is s (exact)."""
    g = bf16(f32(lay.cg[e] * s))
    u = bf16(f32(lay.cu[e] * s))
    if g < 17.0:
        raise AssertionError("closed form needs sigmoid(g) == 1 (g >= 17)")
    act = bf16(f32(g * u))                   # SwiGLU with sigmoid(g) == 1
    return bf16(f32(lay.inter * act * lay.cd[e]))  # exact: I equal products, one rounding


def layer_out(lay: ConstLayer, s: float) -> float:
    """``RTNE(f32(routed) + f32(shared))`` of host/raon.py:1316-1326, with routed the
    ascending-id fp32 sum of ``f32(row) * w`` (host/backend.py:488-510), w = 1/k."""
    w = f32(1.0 / lay.top_k)
    acc = 0.0
    for e in sorted(lay.chosen):
        acc = f32(acc + f32(expert_row(lay, e, s) * w))
    routed = bf16(acc)
    return bf16(f32(routed + expert_row(lay, lay.n_routed, s)))


def residual_stack(layers: list, x_f32: np.ndarray) -> np.ndarray:
    """``x <- RTNE(x + out(x))`` through every layer; x as float32 bf16 values."""
    h = np.asarray(x_f32, np.float32).copy()
    for lay in layers:
        s = float(np.sum(h.astype(np.float64)))
        if s <= 0 or np.any(h < 1.0) or np.any(h >= 4.0):
            raise AssertionError("closed form needs hidden values in [1, 4)")
        out = layer_out(lay, s)
        h = torch.from_numpy(h + np.float32(out)).to(torch.bfloat16).to(torch.float32).numpy()
    return h


def inputs(n: int, hidden: int, seed: int) -> np.ndarray:
    """bf16 bit patterns of values in [1, 2): exponent 0, random 7-bit mantissas."""
    rng = np.random.default_rng(seed)
    return (0x3F80 | rng.integers(0, 128, (n, hidden))).astype(np.uint16)
