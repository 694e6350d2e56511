"""``wt_events_count`` / ``wt_events_fill`` (the per-source event lists of the weight
gradients) against the torch formulation they replace — nonzero, sort by (source, row),
bincount — on ragged sizes (rows not a multiple of the 256-row chunk, one column, no
events, every entry an event) and signed values: identical indptr, rows and values."""

import pytest
import torch

from wiretorch_amd import engine

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _torch_events(flat):
    BT, n = flat.shape
    bt, j = torch.nonzero(flat, as_tuple=True)
    order = torch.argsort(j * BT + bt)
    j, bt = j[order], bt[order]
    indptr = torch.zeros(n + 1, dtype=torch.int64, device=flat.device)
    indptr[1:] = torch.cumsum(torch.bincount(j, minlength=n), 0)
    return indptr, bt, flat[bt, j]


@pytest.mark.parametrize("BT,n,density", [
    (1, 1, 1.0), (255, 7, 0.3), (256, 300, 0.01), (257, 300, 0.0), (1000, 1, 0.5),
    (70_000, 37, 0.02), (3_000, 10_000, 0.002), (513, 64, 1.0),
])
def test_events_match_torch(BT, n, density):
    g = torch.Generator(device=DEV).manual_seed(BT * 131 + n)
    vals = torch.randn((BT, n), device=DEV, generator=g)
    keep = torch.rand((BT, n), device=DEV, generator=g) < density
    flat = torch.where(keep, vals, torch.zeros_like(vals))
    want = _torch_events(flat)
    got = engine._events(flat.reshape(1, BT, n), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for w, h, name in zip(want, got, ("indptr", "bt", "value")):
        assert torch.equal(w.cpu(), h.cpu()), name


def test_events_of_no_source():
    got = engine._events(torch.zeros((2, 3, 0), device=DEV),
                         torch.cuda.current_stream().cuda_stream)
    assert got[0].tolist() == [0] and got[1].numel() == 0 and got[2].numel() == 0
