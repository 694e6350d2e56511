"""``wt_events_count`` / ``wt_events_fill`` (the per-source event lists of the weight
gradients) against the torch formulation they replace — nonzero, sort by (source, row),
bincount — on ragged sizes (rows not a multiple of the 256-row chunk, one column, no
events, every entry an event) and signed values: identical indptr, rows (int32) and
values; without values (spikes) the same indptr and rows and no value list."""

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
    stream = torch.cuda.current_stream().cuda_stream
    got = engine._events(flat.reshape(1, BT, n), stream)
    torch.cuda.synchronize()
    assert got[1].dtype == torch.int32
    for w, h, name in zip(want, got, ("indptr", "bt", "value")):
        assert torch.equal(w.cpu(), h.cpu().to(w.dtype)), name
    indptr, bt, value = engine._events((flat != 0).float().reshape(1, BT, n), stream,
                                       values=False)
    assert value is None
    assert torch.equal(indptr.cpu(), want[0].cpu())
    assert torch.equal(bt.cpu().long(), want[1].cpu())


def test_events_of_no_source():
    got = engine._events(torch.zeros((2, 3, 0), device=DEV),
                         torch.cuda.current_stream().cuda_stream)
    assert got[0].tolist() == [0] and got[1].numel() == 0 and got[2].numel() == 0


@pytest.mark.parametrize("spikes", [True, False], ids=["spikes", "values"])
def test_weight_gradients_by_source_and_by_target(spikes):
    """The two event-driven weight gradients (``wt_weight_gradient``: one thread per
    synapse; ``wt_weight_gradient_by_target``: by (pathway, target) row) through the C-ABI
    on the same events, against the dense float64 product activity^T dL/da at the
    synapses: two pathways over 200 sources, a source in no pathway, 3 trials x 50
    steps; spike activity without an event value list, signed values with one."""
    import ctypes

    from wiretorch_amd import _lib

    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    g = torch.Generator(device=DEV).manual_seed(11 + spikes)
    n_src, N, B, T = 200, 300, 3, 50
    W = torch.randn((n_src, N), device=DEV, generator=g)
    W = torch.where(torch.rand((n_src, N), device=DEV, generator=g) < 0.05, W,
                    torch.zeros_like(W))
    rows = [torch.arange(0, 120, device=DEV), torch.arange(120, 199, device=DEV)]
    side = engine._from_pathways([(r, W[r]) for r in rows], n_src, N, DEV)
    act = (torch.rand((B, T, n_src), device=DEV, generator=g) < 0.1).float()
    if not spikes:
        act = act * torch.randn((B, T, n_src), device=DEV, generator=g)
    grad_A = torch.randn((2, B, T, N), device=DEV, generator=g)
    indptr, bt, value = engine._events(act, stream, values=not spikes)
    c = side.conn
    edge_src = side.edge_src(stream)
    by_source = torch.full((c.n_edges,), float("nan"), device=DEV)
    abi = side.abi(1, N, stream)
    _lib.check(lib.wt_weight_gradient(ctypes.byref(abi), edge_src.data_ptr(), c.n_edges,
                                      indptr.data_ptr(), bt.data_ptr(), _lib.ptr(value),
                                      grad_A.data_ptr(), B, T, N, 0, by_source.data_ptr(),
                                      stream), "wt_weight_gradient")
    in_indptr, in_edge = side.by_target(N, 2, stream)
    scratch = torch.empty((2 * N, B * T), device=DEV)
    by_target = torch.full((c.n_edges,), float("nan"), device=DEV)
    _lib.check(lib.wt_weight_gradient_by_target(
        edge_src.data_ptr(), c.n_edges, in_indptr.data_ptr(), in_edge.data_ptr(), 2, N,
        indptr.data_ptr(), bt.data_ptr(), _lib.ptr(value), grad_A.data_ptr(), B * T,
        scratch.data_ptr(), by_target.data_ptr(), stream), "wt_weight_gradient_by_target")
    torch.cuda.synchronize()
    # the dense product at the synapses, float64
    want = torch.zeros(c.n_edges, dtype=torch.float64, device=DEV)
    tgt = c.targets.long()
    for k, r in enumerate(rows):
        dense = act[:, :, r].double().reshape(B * T, -1).T @ grad_A[k].double().reshape(B * T, N)
        full = torch.zeros((n_src, N), dtype=torch.float64, device=DEV)
        full[r] = dense
        on = c.pathway[edge_src] == k
        want[on] = full[edge_src[on], tgt[on]]
    off = c.pathway[edge_src] < 0
    assert bool(off.any()) or int((c.pathway < 0).sum()) == 1
    want[off] = 0.0
    scale = float(want.abs().max())
    on = ~off
    for got in (by_source, by_target):
        assert not bool(torch.isnan(got[on]).any())
        assert float((got[on].double() - want[on]).abs().max()) <= 1e-5 * scale
    assert bool((by_source[off] == 0).all())
