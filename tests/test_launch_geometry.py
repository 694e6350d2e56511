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


# ---------------------------------------------------------------------------------
# Per-range parameter rows (engine._range_types): more distinct rows than one LDS table
# holds, as long as each target range holds at most MAX_TYPES of them.
# ---------------------------------------------------------------------------------


@pytest.mark.parametrize("N,block,range_n", [(5000, 10, 1024), (4321, 7, 640), (3000, 3, 768)])
def test_range_rows_cover_every_neuron(N, block, range_n):
    """Rows in contiguous blocks of neurons (shuffled row ids): each neuron finds its own
    row through its range's list, the lists ascend, and none exceeds MAX_TYPES."""
    import torch

    n_rows = -(-N // block)
    ids = torch.randperm(n_rows, generator=torch.Generator().manual_seed(N))
    type_of = ids[torch.arange(N) // block].to(torch.int32)
    local, range_rows, most = engine._range_types(type_of, n_rows, range_n)
    assert n_rows > engine.MAX_TYPES and range_rows is not None
    assert range_rows.shape == (-(-N // range_n), engine.MAX_TYPES)
    assert 1 <= most <= engine.MAX_TYPES
    rng = torch.arange(N) // range_n
    assert torch.equal(range_rows[rng, local.long()], type_of)
    assert bool((local >= 0).all()) and bool((local < most).all())
    for r in range(range_rows.shape[0]):
        n_r = int(torch.unique(type_of[rng == r]).numel())
        assert bool((range_rows[r, 1:n_r] > range_rows[r, : n_r - 1]).all())


def test_few_rows_keep_the_global_table():
    import torch

    type_of = torch.randint(0, 200, (3000,), dtype=torch.int32)
    local, range_rows, most = engine._range_types(type_of, 200, 512)
    assert range_rows is None and most == 200 and local is type_of


def test_interleaved_rows_are_refused():
    """Distinct rows spread over a range beyond MAX_TYPES: refused, with the reason."""
    import torch

    type_of = (torch.arange(4000) % 1000).to(torch.int32)
    with pytest.raises(NotImplementedError, match="distinct per-neuron parameter rows"):
        engine._range_types(type_of, 1000, 1024)
