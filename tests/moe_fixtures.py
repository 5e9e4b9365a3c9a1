"""Seeded synthetic MoE layers for the parity tests (BASELINE.json config shapes).

Weights are drawn N(0, std) in fp32, quantized and packed with the oracle's q4nx
codec into the reference's bundle geometry (kernels/moe/pack.py: experts back to
back, gate rows then up rows, down zero-padded to Ipad).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from oracle import moe as om
from oracle.bf16 import f32_to_bf16
from oracle.q4nx import pack_gemv, quantize


@dataclass
class SynthLayer:
    geom: object
    gate_up: bytes
    down: bytes
    router: np.ndarray  # uint16 [E, H]
    bias: np.ndarray | None
    score: str

    def bank(self) -> om.ExpertBank:
        g = self.geom
        return om.ExpertBank(self.gate_up, self.down, g.n_experts, g.hidden, g.inter, g.inter_pad, cache=g.n_experts)

    def router_spec(self) -> om.RouterSpec:
        return om.RouterSpec(self.router, self.geom.top_k, score=self.score, bias=self.bias)

    def oracle_layer(self) -> om.Layer:
        return om.Layer(self.bank(), self.router_spec(), self.geom.shared_id if self.geom.n_shared else None)


def make_layer(geom, seed: int, std: float = 0.02, score: str = "softmax", bias: np.ndarray | None = None) -> SynthLayer:
    rng = np.random.default_rng(seed)
    gu, dn = [], []
    for _ in range(geom.n_experts):
        w = rng.normal(0.0, std, (2 * geom.inter, geom.hidden)).astype(np.float32)
        gu.append(pack_gemv(*quantize(w)))
        d = np.zeros((geom.hidden, geom.inter_pad), np.float32)
        d[:, : geom.inter] = rng.normal(0.0, std, (geom.hidden, geom.inter))
        dn.append(pack_gemv(*quantize(d)))
    router = f32_to_bf16(rng.normal(0.0, 0.02, (geom.n_routed, geom.hidden)).astype(np.float32))
    return SynthLayer(geom, b"".join(gu), b"".join(dn), router, bias, score)


def random_tokens(n: int, hidden: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return f32_to_bf16(rng.standard_normal((n, hidden)).astype(np.float32))


def routing_margin(x_u16: np.ndarray, spec: om.RouterSpec) -> float:
    """Gap between the k-th and (k+1)-th selection scores of one token (tie check)."""
    _, _, logits = om.route_token(x_u16, spec)
    scores = om.router_scores(logits, spec.score)
    choice = scores if spec.bias is None else scores + spec.bias
    s = np.sort(choice)[::-1]
    return float(s[spec.top_k - 1] - s[spec.top_k]) if s.size > spec.top_k else np.inf


def compare_bf16(a_u16: np.ndarray, b_u16: np.ndarray) -> tuple[float, float, float]:
    """(max-abs, rel-L2, fraction of bit-identical elements) of two bf16 arrays."""
    from oracle.bf16 import bf16_to_f32

    a = bf16_to_f32(a_u16).astype(np.float64)
    b = bf16_to_f32(b_u16).astype(np.float64)
    d = a - b
    rel = float(np.linalg.norm(d) / max(np.linalg.norm(b), 1e-30))
    return float(np.abs(d).max()), rel, float(np.mean(a_u16 == b_u16))
