"""Pins of oracle.planner: the reference planner's known answers (kernels/moe_grouped/test_planner.py)."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import planner as op


@pytest.mark.parametrize("tokens,expected_jobs", [(1, 1), (8, 1), (9, 2), (17, 3)])
def test_job_splits(tokens, expected_jobs):
    ids = np.full((tokens, 1), 7, dtype=np.int64)
    plan = op.build_plan(ids)
    assert len(plan.jobs) == expected_jobs
    assert [len(j.assignments) for j in plan.jobs] == [min(8, tokens - s) for s in range(0, tokens, 8)]
    assert all(c.expert_slots[-1] == 7 for c in plan.calls)
    x = np.arange(tokens * 5, dtype=np.uint16).reshape(tokens, 5)
    calls = op.gather_inputs(plan, x)
    outs = [c[..., :3].copy() for c in calls]
    np.testing.assert_array_equal(op.scatter_b1(plan, outs)[:, 0], x[:, :3])


def test_call_rows_property():
    ids = np.array([[0, 1]] * 5 + [[0, 2]] * 6, dtype=np.int64)
    plan = op.build_plan(ids, include_shared=True)
    assert plan.calls[0].rows == (8, 3, 5, 6, 8, 3, 0, 0)
    assert sum(plan.calls[0].rows) == plan.useful_rows == ids.size + ids.shape[0]


def test_validation():
    with pytest.raises(ValueError, match="distinct"):
        op.build_plan(np.array([[3, 3]]))
    with pytest.raises(ValueError, match="0..127"):
        op.build_plan(np.array([[128]]))
    with pytest.raises(TypeError):
        op.build_plan(np.array([[1.0]]))


def test_dispatch_order_is_stable_expert_sort():
    rng = np.random.default_rng(5)
    T, k, E = 300, 8, 64
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)])
    order, offsets = op.dispatch_order(ids, n_routed=E)
    flat = ids.reshape(-1)
    ref = np.lexsort((np.arange(flat.size), flat))  # by expert, then flat index (= token, route)
    np.testing.assert_array_equal(order, ref)
    np.testing.assert_array_equal(offsets[1:] - offsets[:-1], np.bincount(flat, minlength=E))
    assert offsets[0] == 0 and offsets[-1] == flat.size
