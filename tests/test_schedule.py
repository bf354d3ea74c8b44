"""The partial kernel's token-balanced schedule, checked on the CPU through
``l20_pd_plan_runs`` (the same RunCursor code the kernel runs).

Properties: every (sequence, split) item is covered by exactly one run; a run
stays inside one sequence and spans at most 1024 tokens; every walk ends; the
token work of the workgroups is balanced to within one run of the mean.
"""

import numpy as np
import pytest

import l20_pd_cabi as cabi

BIG = 1 << 30


def n_splits(length, split):
    return max(1, -(-length // split)) if length > 0 else 1


def check_plan(lens, split, grid, l_cap=BIG):
    lens = [int(v) for v in lens]
    runs = cabi.plan_runs(lens, split, l_cap, grid)
    seen = {}
    max_items = max(1, 1024 // split)
    for w, b, s0, s1 in runs:
        assert 0 <= w < grid and 0 <= b < len(lens)
        clamped = max(0, min(lens[b], l_cap))
        assert 0 <= s0 <= s1 < n_splits(clamped, split)
        assert s1 - s0 + 1 <= max_items
        for s in range(s0, s1 + 1):
            assert (b, s) not in seen, f"item {(b, s)} covered twice"
            seen[(b, s)] = w
    expected = {(b, s) for b, L in enumerate(lens) for s in range(n_splits(max(0, min(L, l_cap)), split))}
    assert set(seen) == expected
    return runs


@pytest.mark.parametrize("lens,split,grid", [
    ([129], 64, 3),            # one sequence starting at token 0 (the last share is unbounded)
    ([129], 64, 256),
    ([2304], 128, 5),
    ([0, 0, 5], 64, 4),        # empty sequences
    ([0], 64, 1),
    ([0, 0, 0], 64, 8),
    ([1, 15, 16, 17, 500], 96, 7),
    ([131072, 131072], 1024, 512),
    ([4096] * 64, 512, 1024),
])
def test_plan_covers_every_item_once(lens, split, grid):
    check_plan(lens, split, grid)


def test_plan_random_cases_terminate_and_cover():
    rng = np.random.default_rng(3)
    for _ in range(300):
        batch = int(rng.integers(1, 40))
        lens = rng.integers(0, 3000, batch)
        lens[rng.random(batch) < 0.15] = 0
        split = int(rng.choice([64, 80, 128, 256, 512, 1024]))
        grid = int(rng.integers(1, 600))
        check_plan(lens, split, grid, l_cap=int(rng.choice([BIG, 2048, 100])))


def test_plan_balances_lognormal_batch():
    rng = np.random.default_rng(37)
    lens = np.clip(np.round(np.exp(np.log(1024) + rng.standard_normal(128))), 16, 8192).astype(int)
    split, grid = 128, 512
    runs = check_plan(lens, split, grid)
    work = np.zeros(grid)
    for w, b, s0, s1 in runs:
        work[w] += min((s1 + 1) * split, lens[b]) - s0 * split
    mean = lens.sum() / grid
    assert work.max() <= mean + split
    assert abs(work.sum() - lens.sum()) == 0
