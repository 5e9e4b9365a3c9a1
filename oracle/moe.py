"""Reference CPU MoE path (oracle; test infrastructure only).

Restates the NumPy host path of raon-npu for one mixture-of-experts layer:

* ``linear``        -- ``host/backend.py:402-417`` (fp32 ``np.dot`` then RTNE to bf16)
* ``situ_glu``      -- ``host/backend.py:47-62``
* ``swiglu``        -- ``kernels/moe/reference.py:127-180`` (``gate_beta=None`` branch)
* ``route_token``   -- ``host/raon.py:1224-1247`` (sigmoid + selection bias, the
                       reference router) and the softmax router BASELINE.json's
                       configs name (same steps with softmax scores)
* ``moe_experts``   -- ``host/backend.py:466-510`` (ascending expert id, fp32 sum)
* ``moe_token``     -- ``host/raon.py:1288-1330`` (routed + shared, RTNE of the sum)
* ``moe_experts_grouped`` -- the contract of ``npu/backend.py:4845-4979``:
                       per token the ``moe_experts`` result, plus the shared
                       down rows from a precomputed ``shared_gu``
* ``prefill_layer`` -- ``host/raon.py:1565-1621`` (grouped branch)
* ``residual_stack`` -- BASELINE config 4's 48-layer decode (residual add between
                       layers; the reference model has no such stack -- this is the
                       benchmark's definition).

Expert weights come from q4nx ``pack_gemv`` bytes exactly as the reference's
``DWeights`` serves them (``npu/backend.py:1246-1273``): ``parse_gemv`` then
``dequantize_simple`` into fp32, gate rows then up rows in one ``[2I, H]``
matrix (``kernels/moe/pack.py:136-172``), down ``[H, Ipad]`` with the input
columns past ``I`` zero (``kernels/moe/pack.py:190-224``).

Pins (tests/test_oracle_moe.py):
* ``situ_glu``/``swiglu``: the known answers of ``bench/moe/test_moe_ref.py:408-437``
  (g=100,u=2 -> 200; g=0 -> 0) and closed-form values at other points.
* ``linear``: float64 matrix product within fp32 error bounds, and bit-for-bit
  against ``bf16(float32(x) @ W.T)`` computed by torch on CPU.
* ``route_token``: top-k equals ``torch.topk`` of the same scores (a library
  routine) whenever the k/k+1 margin is not a tie; weights sum to the scaling
  factor; softmax scores equal ``torch.softmax``.
* ``moe_experts``: the order-sensitivity regression of
  ``kernels/moe_grouped/test_planner.py:127-155`` (ascending id, not route order),
  invariance to permuting the (id, weight) pairs, the k=1/w=1 reduction to a
  plain expert chain, and the 10.5 known answer of
  ``bench/moe/test_moe_ref.py:430-437``.
* ``moe_experts_grouped``: equals the planner gather/scatter path
  (``oracle.planner``), restating ``kernels/moe_grouped/test_planner.py:67-105``.
* ``prefill_layer`` (tests/test_oracle_stack.py): byte-equal to ``moe_token`` per token,
  as the reference's grouped-prefill parity test requires of its grouped path
  (``host/test_prefill_grouped_parity.py:42-115``); equal to a closed form on
  constant-weight experts (every projection ``c * sum(x)``, every sum exact), batched
  and token-serial alike.
* ``residual_stack`` (BASELINE config 4's stack; the reference has no such stack):
  equal, bit for bit, to the same closed form evaluated with Python scalars and torch's
  bf16 rounding over several layers; all-zero experts return the input unchanged; and
  planted mistakes (one rounding around the residual add instead of two, no shared
  expert, gate and up swapped, the lowest-scoring experts selected) all fail that
  comparison.
"""

from __future__ import annotations

from collections import OrderedDict
from dataclasses import dataclass, field

import numpy as np

from .bf16 import bf16_to_f32, f32_to_bf16
from .q4nx import dequantize_simple, parse_gemv


def linear(w_f32: np.ndarray, x: np.ndarray) -> np.ndarray:
    """``y = x @ W.T``: bf16 (uint16) input -> bf16 output, fp32 input -> fp32 output."""
    is_f32 = x.dtype == np.float32
    xf = x if is_f32 else bf16_to_f32(x)
    y = np.dot(xf, w_f32.T)
    return y.astype(np.float32) if is_f32 else f32_to_bf16(y)


def situ_glu(gate, value, gate_beta: float = 4.0, value_beta: float = 25.0) -> np.ndarray:
    """SiTU-GLU in fp32: ``gb*tanh(g/gb)*sigmoid(g) * vb*tanh(v/vb)``."""
    g = bf16_to_f32(gate) if gate.dtype == np.uint16 else gate.astype(np.float32, copy=False)
    v = bf16_to_f32(value) if value.dtype == np.uint16 else value.astype(np.float32, copy=False)
    sig = 1.0 / (1.0 + np.exp(-g))
    return (gate_beta * np.tanh(g / gate_beta) * sig) * (value_beta * np.tanh(v / value_beta))


def swiglu(gate, up) -> np.ndarray:
    """SiLU-GLU in fp32: ``g*sigmoid(g) * u`` with the overflow-free sigmoid of
    ``kernels/moe/reference.py:160-170``."""
    g = bf16_to_f32(gate) if gate.dtype == np.uint16 else gate.astype(np.float32, copy=False)
    u = bf16_to_f32(up) if up.dtype == np.uint16 else up.astype(np.float32, copy=False)
    e = np.exp(-np.abs(g))
    sig = np.where(g >= 0, 1.0 / (1.0 + e), e / (1.0 + e)).astype(np.float32)
    return (g * sig) * u


def glu(gate, up, gate_beta, value_beta) -> np.ndarray:
    """Activation selector: SwiGLU when ``gate_beta is None`` (the ``gate_beta=None``
    convention of ``kernels/moe/reference.py:151-171``), SiTU-GLU otherwise."""
    if gate_beta is None:
        return swiglu(gate, up)
    return situ_glu(gate, up, gate_beta=gate_beta, value_beta=value_beta)


@dataclass
class RouterSpec:
    """Router of one MoE layer.

    ``score`` is ``"sigmoid"`` (the reference router, ``host/raon.py:1233-1234``) or
    ``"softmax"``.  ``bias`` is the selection-only
    ``e_score_correction_bias`` (``host/raon.py:1237``); ``renormalize`` and
    ``scaling`` follow ``host/raon.py:1242-1245``.
    """

    weight_bf16: np.ndarray  # uint16 [E, H]
    top_k: int
    score: str = "softmax"
    bias: np.ndarray | None = None  # float32 [E]
    renormalize: bool = True
    scaling: float = 1.0

    def weight_f32(self) -> np.ndarray:
        return bf16_to_f32(self.weight_bf16)


def router_scores(logits: np.ndarray, score: str) -> np.ndarray:
    if score == "sigmoid":
        return 1.0 / (1.0 + np.exp(-logits))
    if score == "softmax":
        z = np.exp(logits - np.max(logits))
        return z / np.sum(z)
    raise ValueError(f"unknown router score {score!r}")


def route_token(x_u16: np.ndarray, router: RouterSpec, w_f32: np.ndarray | None = None):
    """One token's ``(top ids int64 [k], weights f32 [k], logits f32 [E])``.

    ``host/raon.py:1224-1247``.  Ties in the selection score keep the lower expert
    id first (stable sort); the reference's default ``argsort`` leaves exact ties
    unspecified, so parity tests check the k/k+1 margin instead of relying on ties.
    """
    w = router.weight_f32() if w_f32 is None else w_f32
    logits = np.dot(bf16_to_f32(x_u16), w.T).astype(np.float32)
    scores = router_scores(logits, router.score).astype(np.float32)
    choice = scores if router.bias is None else scores + router.bias
    top = np.argsort(-choice, kind="stable")[: router.top_k]
    chosen = scores[top]
    if router.renormalize:
        chosen = chosen / (np.sum(chosen) + 1e-20)
    return top, (chosen * router.scaling).astype(np.float32), logits


class ExpertBank:
    """q4nx expert weights of one layer, served as fp32 the way ``DWeights`` does.

    ``gate_up`` holds ``E`` experts' ``pack_gemv`` bytes back to back, each a
    ``[2I, H]`` matrix (gate rows then up rows); ``down`` holds ``[H, Ipad]``
    matrices.  The shared expert, when present, is expert index ``E-1`` of both
    bundles (``kernels/moe/pack.py:40-44``: routed 0..127, shared 128).
    Dequantized experts are cached LRU (``npu/backend.py:940-1058``).
    """

    def __init__(self, gate_up: bytes, down: bytes, n_experts: int, hidden: int, inter: int,
                 inter_pad: int | None = None, cache: int = 32):
        self.gate_up = np.frombuffer(gate_up, dtype=np.uint8) if isinstance(gate_up, (bytes, bytearray)) else np.asarray(gate_up, np.uint8)
        self.down = np.frombuffer(down, dtype=np.uint8) if isinstance(down, (bytes, bytearray)) else np.asarray(down, np.uint8)
        self.n_experts = n_experts
        self.hidden = hidden
        self.inter = inter
        self.inter_pad = inter_pad if inter_pad is not None else -(-inter // 256) * 256
        self.gu_bytes = 2 * inter * hidden * 5 // 8
        self.dn_bytes = hidden * self.inter_pad * 5 // 8
        if self.gate_up.size != n_experts * self.gu_bytes or self.down.size != n_experts * self.dn_bytes:
            raise ValueError("bundle sizes do not match the expert geometry")
        self._cache: OrderedDict[int, tuple[np.ndarray, np.ndarray, np.ndarray]] = OrderedDict()
        self._cap = max(1, cache)

    def expert(self, e: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        """``(gate [I,H], up [I,H], down [H,I])`` fp32 for expert ``e``."""
        hit = self._cache.get(e)
        if hit is not None:
            self._cache.move_to_end(e)
            return hit
        gu = self.gate_up[e * self.gu_bytes : (e + 1) * self.gu_bytes]
        c, s, m = parse_gemv(gu, K=self.hidden, M=2 * self.inter)
        w = dequantize_simple(c, s, m)
        dn = self.down[e * self.dn_bytes : (e + 1) * self.dn_bytes]
        c2, s2, m2 = parse_gemv(dn, K=self.inter_pad, M=self.hidden)
        d = np.ascontiguousarray(dequantize_simple(c2, s2, m2)[:, : self.inter])
        out = (np.ascontiguousarray(w[: self.inter]), np.ascontiguousarray(w[self.inter :]), d)
        self._cache[e] = out
        while len(self._cache) > self._cap:
            self._cache.popitem(last=False)
        return out

    def down_proj(self, e: int) -> np.ndarray:
        """``[H, I]`` fp32 down projection of expert ``e``."""
        return self.expert(e)[2]


class DExpertBank:
    """Experts of one layer in the weights-d bundles, served as fp32 the way ``DWeights``
    does (``npu/backend.py:1246-1273``, ``:1228-1239``).

    ``moe_b1`` holds ``n_routed`` q4nx experts ``[2I, H]`` back to back; ``moe_b2`` holds
    ``n_routed + 1`` bfp16 experts ``[H, Ipad]`` whose last one is the shared expert's down
    projection (``npu/backend.py:624-700``); ``shared_gu`` is the shared expert's bfp16
    ``[2I, H]`` gate/up matrix (or None).  bfp16 weights decode as ``m * 2**(e - 133)``
    (``parse_bfp16_gemv``, quant/bfp16.py:412-440).  Duck-types ``ExpertBank`` for the
    functions below, the shared expert being expert ``n_routed``.
    """

    def __init__(self, moe_b1, moe_b2, n_routed: int, hidden: int, inter: int, shared_gu=None, cache: int = 32):
        from . import bfp16 as _b16

        self._b16 = _b16
        self.moe_b1 = np.frombuffer(moe_b1, np.uint8) if isinstance(moe_b1, (bytes, bytearray)) else np.asarray(moe_b1, np.uint8).reshape(-1)
        self.moe_b2 = np.frombuffer(moe_b2, np.uint8) if isinstance(moe_b2, (bytes, bytearray)) else np.asarray(moe_b2, np.uint8).reshape(-1)
        self.n_routed, self.hidden, self.inter = n_routed, hidden, inter
        self.inter_pad = -(-inter // 256) * 256
        self.gu_bytes = 2 * inter * hidden * 5 // 8
        self.dn_bytes = hidden * self.inter_pad * 9 // 8
        if self.moe_b1.size != n_routed * self.gu_bytes or self.moe_b2.size != (n_routed + 1) * self.dn_bytes:
            raise ValueError("bundle sizes do not match the weights-d expert geometry")
        self.shared_gu = None if shared_gu is None else _b16.parse_gemv(shared_gu, K=hidden, M=2 * inter)
        self._cache: OrderedDict[int, tuple[np.ndarray, np.ndarray, np.ndarray]] = OrderedDict()
        self._cap = max(1, cache)

    def down_proj(self, e: int) -> np.ndarray:
        """``[H, I]`` fp32 down projection of expert ``e`` (``n_routed`` = shared)."""
        dn = self.moe_b2[e * self.dn_bytes : (e + 1) * self.dn_bytes]
        return np.ascontiguousarray(self._b16.parse_gemv(dn, K=self.inter_pad, M=self.hidden)[:, : self.inter])

    def expert(self, e: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        hit = self._cache.get(e)
        if hit is not None:
            self._cache.move_to_end(e)
            return hit
        if e == self.n_routed:
            if self.shared_gu is None:
                raise ValueError("the shared expert's gate/up (shared_gu) was not given")
            w = self.shared_gu
        else:
            gu = self.moe_b1[e * self.gu_bytes : (e + 1) * self.gu_bytes]
            w = dequantize_simple(*parse_gemv(gu, K=self.hidden, M=2 * self.inter))
        out = (np.ascontiguousarray(w[: self.inter]), np.ascontiguousarray(w[self.inter :]), self.down_proj(e))
        self._cache[e] = out
        while len(self._cache) > self._cap:
            self._cache.popitem(last=False)
        return out


def expert_chain(bank: ExpertBank, e: int, x_u16: np.ndarray, gate_beta, value_beta) -> np.ndarray:
    """gate, up, activation -> RTNE, down for one expert: bf16 ``[H]`` out."""
    g, u, d = bank.expert(e)
    act = f32_to_bf16(glu(linear(g, x_u16), linear(u, x_u16), gate_beta, value_beta))
    return linear(d, act)


def combine_routed(rows: dict, top_ids, top_weights) -> np.ndarray:
    """``RTNE(sum in ascending expert id of f32(row_e) * w_e)`` (``host/backend.py:488-510``).

    ``rows`` maps expert id -> bf16 output row.  Each step is a float32 multiply
    then a float32 add (two roundings), exactly as the reference's ``+=``.
    """
    acc = None
    for e, wt in sorted(((int(e), float(w)) for e, w in zip(top_ids, top_weights)), key=lambda t: t[0]):
        term = bf16_to_f32(rows[e]) * wt
        acc = np.zeros_like(term) + term if acc is None else acc + term
    return f32_to_bf16(acc)


def moe_experts(bank: ExpertBank, x_u16, top_ids, top_weights, gate_beta=4.0, value_beta=25.0) -> np.ndarray:
    """Weighted routed sum for one token (``host/backend.py:466-510``).

    Experts are visited in ascending id regardless of route order; the sum is fp32
    and rounded to bf16 once at the end.
    """
    rows = {int(e): expert_chain(bank, int(e), x_u16, gate_beta, value_beta) for e in top_ids}
    return combine_routed(rows, top_ids, top_weights)


def shared_expert(bank: ExpertBank, shared_id: int, x_u16, gate_beta, value_beta) -> np.ndarray:
    """Shared expert output (``host/raon.py:1314-1324``)."""
    return expert_chain(bank, shared_id, x_u16, gate_beta, value_beta)


def shared_gate_up(bank: ExpertBank, shared_id: int, x_u16) -> np.ndarray:
    """``[2I]`` bf16 shared gate+up rows (``linear_batch`` of ``host/raon.py:1572-1577``)."""
    g, u, _ = bank.expert(shared_id)
    return np.concatenate([linear(g, x_u16), linear(u, x_u16)], axis=-1)


def moe_token(bank: ExpertBank, router: RouterSpec, x_u16, gate_beta=4.0, value_beta=25.0,
              shared_id: int | None = None, router_w_f32=None):
    """Router + routed experts + shared expert for one token (``host/raon.py:1288-1330``).

    Returns ``(out bf16 [H], top, weights, logits)``.
    """
    top, wts, logits = route_token(x_u16, router, router_w_f32)
    routed = moe_experts(bank, x_u16, top, wts, gate_beta, value_beta)
    if shared_id is None:
        return routed, top, wts, logits
    sh = shared_expert(bank, shared_id, x_u16, gate_beta, value_beta)
    return f32_to_bf16(bf16_to_f32(routed) + bf16_to_f32(sh)), top, wts, logits


def moe_experts_grouped(bank: ExpertBank, x_u16, top_ids, top_weights, shared_gu, shared_id: int,
                        gate_beta=4.0, value_beta=25.0):
    """``(routed [T,H], shared_down [T,H])`` of the grouped prefill contract, token by token.

    ``npu/backend.py:4845-4979``: routed rows equal ``moe_experts`` per token; the
    shared down rows are ``down(RTNE(act(shared_gu)))`` of the shared expert.
    """
    inter = bank.inter
    d = bank.down_proj(shared_id)
    routed = np.stack([moe_experts(bank, x_u16[t], top_ids[t], top_weights[t], gate_beta, value_beta)
                       for t in range(x_u16.shape[0])])
    act = f32_to_bf16(glu(shared_gu[:, :inter], shared_gu[:, inter:], gate_beta, value_beta))
    shared_down = np.stack([linear(d, act[t]) for t in range(x_u16.shape[0])])
    return routed, shared_down


def moe_experts_grouped_batched(bank: ExpertBank, x_u16, top_ids, top_weights, shared_gu, shared_id: int,
                                gate_beta=4.0, value_beta=25.0):
    """Same contract as ``moe_experts_grouped``, with one fp32 matrix product per expert.

    The per-expert products use BLAS GEMM instead of per-token GEMV, so single
    outputs may differ from the token-serial form by fp32 summation order (and so
    by one bf16 ulp after rounding); the combine order is unchanged.  Used to keep
    the oracle fast at BASELINE config 3/5 sizes.
    """
    t_count, k = top_ids.shape
    inter = bank.inter
    xf = bf16_to_f32(x_u16)
    down_rows = np.zeros((t_count, k, x_u16.shape[1]), dtype=np.uint16)
    for e in np.unique(top_ids):
        tok, rte = np.nonzero(top_ids == e)
        g, u, d = bank.expert(int(e))
        xe = xf[tok]
        act = f32_to_bf16(glu(f32_to_bf16(xe @ g.T), f32_to_bf16(xe @ u.T), gate_beta, value_beta))
        down_rows[tok, rte] = f32_to_bf16(bf16_to_f32(act) @ d.T)
    routed = np.empty_like(x_u16)
    for t in range(t_count):
        acc = np.zeros(x_u16.shape[1], dtype=np.float32)
        for r in np.argsort(top_ids[t], kind="stable"):
            acc += bf16_to_f32(down_rows[t, r]) * float(top_weights[t, r])
        routed[t] = f32_to_bf16(acc)
    d = bank.down_proj(shared_id)
    act = f32_to_bf16(glu(shared_gu[:, :inter], shared_gu[:, inter:], gate_beta, value_beta))
    shared_down = f32_to_bf16(bf16_to_f32(act) @ d.T)
    return routed, shared_down


def prefill_layer(bank: ExpertBank, router: RouterSpec, x_u16, shared_id: int, gate_beta=4.0, value_beta=25.0,
                  batched: bool = False):
    """Grouped-branch MoE prefill of ``T`` tokens (``host/raon.py:1565-1602``).

    Returns ``(out [T,H], top [T,k], weights [T,k])``.
    """
    wf = router.weight_f32()
    routes = [route_token(x_u16[t], router, wf) for t in range(x_u16.shape[0])]
    top = np.stack([r[0] for r in routes])
    wts = np.stack([r[1] for r in routes]).astype(np.float32)
    if batched:
        g, u, _ = bank.expert(shared_id)
        xf = bf16_to_f32(x_u16)
        sgu = np.concatenate([f32_to_bf16(xf @ g.T), f32_to_bf16(xf @ u.T)], axis=1)
        routed, sdown = moe_experts_grouped_batched(bank, x_u16, top, wts, sgu, shared_id, gate_beta, value_beta)
    else:
        sgu = np.stack([shared_gate_up(bank, shared_id, x_u16[t]) for t in range(x_u16.shape[0])])
        routed, sdown = moe_experts_grouped(bank, x_u16, top, wts, sgu, shared_id, gate_beta, value_beta)
    return f32_to_bf16(bf16_to_f32(routed) + bf16_to_f32(sdown)), top, wts


@dataclass
class Layer:
    """One MoE layer for the oracle: expert bank + router + shared expert id."""

    bank: ExpertBank
    router: RouterSpec
    shared_id: int | None
    _router_f32: np.ndarray | None = field(default=None, repr=False)

    def router_f32(self) -> np.ndarray:
        if self._router_f32 is None:
            self._router_f32 = self.router.weight_f32()
        return self._router_f32


def residual_stack(layers: list[Layer], x_u16, gate_beta=None, value_beta=None):
    """``x <- RTNE(f32(x) + f32(moe_token(x)))`` through every layer."""
    h = np.asarray(x_u16, dtype=np.uint16)
    for lyr in layers:
        out, *_ = moe_token(lyr.bank, lyr.router, h, gate_beta, value_beta, lyr.shared_id, lyr.router_f32())
        h = f32_to_bf16(bf16_to_f32(h) + bf16_to_f32(out))
    return h
