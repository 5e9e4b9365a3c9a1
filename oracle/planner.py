"""Grouped-MoE dispatch planner (oracle; test infrastructure only).

Restates ``kernels/moe_grouped/planner.py:18-322`` with the slot geometry of
``kernels/moe_grouped/layout.py:22-23`` (8 slots per call, at most 8 rows per job).

The dispatch permutation the GPU must reproduce bit-exactly is the flattened job
order of ``build_plan``: assignments ``(token, route)`` grouped by expert in
ascending id, and inside one expert in row-major ``(token, route)`` order
(``planner.py:89-96``).  ``dispatch_order`` returns that order directly.

Pins (tests/test_oracle_planner.py): the job-split and rows known answers of
``kernels/moe_grouped/test_planner.py:15-52``, the gather/scatter == token-serial
MoE equality of ``:67-105``, the job-order regression of ``:127-155``, and
``dispatch_order`` == a ``numpy.lexsort`` by (expert, token, route).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .bf16 import bf16_to_f32, f32_to_bf16
from .moe import glu

SLOTS = 8
TMAX = 8


@dataclass(frozen=True)
class Assignment:
    token: int
    route: int
    expert: int


@dataclass(frozen=True)
class Job:
    expert: int
    assignments: tuple
    shared: bool = False

    def __post_init__(self):
        if not 1 <= len(self.assignments) <= TMAX:
            raise ValueError(f"job must contain 1..{TMAX} assignments")
        if any(a.expert != self.expert for a in self.assignments):
            raise ValueError("all job assignments must use the job expert")


@dataclass(frozen=True)
class Call:
    jobs: tuple
    expert_slots: tuple

    def __post_init__(self):
        if len(self.jobs) != SLOTS or len(self.expert_slots) != SLOTS:
            raise ValueError(f"a call requires exactly {SLOTS} slots")

    @property
    def rows(self) -> tuple:
        return tuple(0 if j is None else len(j.assignments) for j in self.jobs)


@dataclass(frozen=True)
class Plan:
    token_count: int
    route_count: int
    jobs: tuple
    calls: tuple
    include_shared: bool

    @property
    def useful_rows(self) -> int:
        return sum(len(j.assignments) for j in self.jobs)


def _validate_ids(top_ids, n_routed: int) -> np.ndarray:
    ids = np.asarray(top_ids)
    if ids.ndim != 2 or ids.shape[0] < 1 or ids.shape[1] < 1:
        raise ValueError("top_ids must have shape [tokens, routes]")
    if not np.issubdtype(ids.dtype, np.integer):
        raise TypeError("top_ids must be an integer array")
    if np.any(ids < 0) or np.any(ids >= n_routed):
        raise ValueError(f"routed expert IDs must be in 0..{n_routed - 1}")
    s = np.sort(ids, axis=1)
    if np.any(s[:, 1:] == s[:, :-1]):
        raise ValueError("each token must route to distinct experts")
    return ids


def build_plan(top_ids, *, include_shared: bool = False, n_routed: int = 128) -> Plan:
    """Ascending-expert jobs of at most 8 rows, packed 8 per call (``planner.py:76-108``).

    The shared expert (id ``n_routed``) gets one row per token after all routed
    jobs when ``include_shared``; an under-full last call repeats its first
    expert in the empty slots.
    """
    ids = _validate_ids(top_ids, n_routed)
    per_expert: dict[int, list[Assignment]] = {}
    for t in range(ids.shape[0]):
        for r in range(ids.shape[1]):
            e = int(ids[t, r])
            per_expert.setdefault(e, []).append(Assignment(t, r, e))
    jobs: list[Job] = []
    for e in sorted(per_expert):
        rows = per_expert[e]
        jobs += [Job(e, tuple(rows[i : i + TMAX])) for i in range(0, len(rows), TMAX)]
    if include_shared:
        sh = [Assignment(t, -1, n_routed) for t in range(ids.shape[0])]
        jobs += [Job(n_routed, tuple(sh[i : i + TMAX]), shared=True) for i in range(0, len(sh), TMAX)]
    calls = []
    for i in range(0, len(jobs), SLOTS):
        part = jobs[i : i + SLOTS]
        slots = tuple(part) + (None,) * (SLOTS - len(part))
        calls.append(Call(slots, tuple(j.expert if j is not None else part[0].expert for j in slots)))
    return Plan(ids.shape[0], ids.shape[1], tuple(jobs), tuple(calls), include_shared)


def dispatch_order(top_ids, n_routed: int = 128):
    """Flat dispatch permutation of ``build_plan`` (routed jobs only).

    Returns ``(order int32 [T*k], offsets int32 [E+1])``: ``order[p]`` is the
    assignment index ``token*k + route`` at expert-sorted position ``p``;
    expert ``e`` owns positions ``offsets[e]:offsets[e+1]``.
    """
    ids = _validate_ids(top_ids, n_routed)
    plan = build_plan(ids, n_routed=n_routed)
    k = ids.shape[1]
    order = np.array([a.token * k + a.route for j in plan.jobs for a in j.assignments], dtype=np.int32)
    counts = np.bincount(ids.reshape(-1), minlength=n_routed)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    return order, offsets


def gather_inputs(plan: Plan, routed, shared=None) -> list[np.ndarray]:
    """Zero-padded ``[8, 8, K]`` call tensors (``planner.py:130-162``)."""
    r = np.asarray(routed, dtype=np.uint16)
    if r.ndim not in (2, 3) or r.shape[0] != plan.token_count:
        raise ValueError("routed inputs must be [T,K] or [T,R,K]")
    s = None if shared is None else np.asarray(shared, dtype=np.uint16)
    if plan.include_shared and (s is None or s.shape[0] != plan.token_count):
        raise ValueError("shared inputs [T,K] are required by this plan")
    out = []
    for call in plan.calls:
        x = np.zeros((SLOTS, TMAX, r.shape[-1]), dtype=np.uint16)
        for slot, job in enumerate(call.jobs):
            if job is None:
                continue
            for row, a in enumerate(job.assignments):
                if job.shared:
                    x[slot, row] = s[a.token]
                elif r.ndim == 2:
                    x[slot, row] = r[a.token]
                else:
                    x[slot, row] = r[a.token, a.route]
        out.append(x)
    return out


def scatter_b1(plan: Plan, outputs) -> np.ndarray:
    """Per-call outputs -> ``[T, R, M]`` rows (``planner.py:242-258``)."""
    arrays = list(outputs)
    if len(arrays) != len(plan.calls):
        raise ValueError("one output tensor is required per call")
    m = np.asarray(arrays[0]).shape[-1]
    res = np.zeros((plan.token_count, plan.route_count, m), dtype=np.uint16)
    for call, out in zip(plan.calls, arrays):
        for slot, job in enumerate(call.jobs):
            if job is None or job.shared:
                continue
            for row, a in enumerate(job.assignments):
                res[a.token, a.route] = out[slot, row]
    return res


def make_b2_inputs(gate_up, shared_gate_up, inter: int, gate_beta=4.0, value_beta=25.0):
    """Activation -> RTNE of routed ``[T,R,2I]`` and shared ``[T,2I]`` rows (``planner.py:261-283``)."""
    gu = np.asarray(gate_up, dtype=np.uint16)
    sh = np.asarray(shared_gate_up, dtype=np.uint16)
    routed = f32_to_bf16(glu(gu[..., :inter], gu[..., inter:], gate_beta, value_beta))
    shared = f32_to_bf16(glu(sh[..., :inter], sh[..., inter:], gate_beta, value_beta))
    return routed, shared


def scatter_b2(plan: Plan, outputs, top_ids, top_weights):
    """Per-token fp32 sum in ascending expert id, RTNE; plus shared rows (``planner.py:286-322``)."""
    arrays = list(outputs)
    ids = np.asarray(top_ids)
    w = np.asarray(top_weights, dtype=np.float32)
    if ids.shape != (plan.token_count, plan.route_count) or w.shape != ids.shape:
        raise ValueError("top_ids/top_weights must match the plan")
    m = np.asarray(arrays[0]).shape[-1]
    rows: dict[tuple[int, int], np.ndarray] = {}
    shared = np.zeros((plan.token_count, m), dtype=np.uint16)
    for call, out in zip(plan.calls, arrays):
        for slot, job in enumerate(call.jobs):
            if job is None:
                continue
            for row, a in enumerate(job.assignments):
                if job.shared:
                    shared[a.token] = out[slot, row]
                else:
                    rows[(a.token, a.route)] = np.array(out[slot, row])
    final = np.zeros((plan.token_count, m), dtype=np.uint16)
    for t in range(plan.token_count):
        acc = np.zeros(m, dtype=np.float32)
        for r in sorted(range(plan.route_count), key=lambda q: int(ids[t, q])):
            acc += bf16_to_f32(rows[(t, r)]) * float(w[t, r])
        final[t] = f32_to_bf16(acc)
    return final, shared
