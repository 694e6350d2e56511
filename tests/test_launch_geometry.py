"""The forward's launch geometry (``engine.geometry``), on the CPU: every plan is one the
kernel accepts (groups of whole XCDs, ranges covering the network, at most 8 items per
thread, the accumulator within LDS), and the group count follows the batch."""

import pytest

from wiretorch_amd import engine

N_CU, MAX_LDS = 256, 160 * 1024


def _check(B, N, K, plan):
    groups, R, range_n = plan
    tpg = -(-B // groups)
    assert 1 <= groups <= min(B, 64)
    assert groups * R <= max(N_CU, groups)
    assert range_n % 32 == 0 and R * range_n >= N and (R - 1) * range_n < N
    assert tpg * range_n <= 8 * engine.BLOCK
    assert max(K, 1) * tpg * range_n * 8 <= MAX_LDS - 54 * 1024
    if groups > engine.XCDS:
        # workgroup i is in group i % groups and on XCD i % 8: one XCD per group
        assert groups % engine.XCDS == 0
        for g in range(groups):
            assert len({(g + groups * r) % engine.XCDS for r in range(R)}) == 1


@pytest.mark.parametrize("B,N,K", [(1, 1000, 3), (8, 140_000, 3), (12, 10_000, 3),
                                   (32, 10_000, 3), (64, 10_000, 3), (9, 80_000, 3),
                                   (17, 20_000, 6), (100, 2_000, 4), (5, 50_000, 8)])
def test_plans_are_valid(B, N, K):
    _check(B, N, K, engine.geometry(B, N, K, N_CU, MAX_LDS))


def test_one_trial_per_group_where_the_batch_allows():
    assert engine.geometry(32, 10_000, 3, N_CU, MAX_LDS) == (32, 8, 1280)  # configuration 1
    assert engine.geometry(64, 10_000, 3, N_CU, MAX_LDS)[0] == 64  # configuration 3
    assert engine.geometry(8, 140_000, 3, N_CU, MAX_LDS)[0] == 8  # configuration 2
    assert engine.geometry(12, 10_000, 3, N_CU, MAX_LDS)[0] == 8  # whole XCDs past 8


def test_large_network_takes_fewer_groups():
    # 8 groups of 9 trials give one group 2 trials over its 32 workgroups: 2 x 2528
    # items each, whose accumulator is past the LDS budget; 4 groups of up to 3 trials
    # over 63 workgroups (3 x 1280 items each) fit
    assert engine.geometry(9, 80_000, 3, N_CU, MAX_LDS) == (4, 63, 1280)
    with pytest.raises(ValueError):  # B x N / 256 items per workgroup: past any grouping
        engine.geometry(64, 140_000, 3, N_CU, MAX_LDS)


def test_group_limit(monkeypatch):
    monkeypatch.setattr(engine, "MAX_GROUPS", 8)
    assert engine.geometry(32, 10_000, 3, N_CU, MAX_LDS) == (8, 32, 320)
    with pytest.raises(ValueError):
        engine.geometry(64, 10_000_000, 3, N_CU, MAX_LDS)
