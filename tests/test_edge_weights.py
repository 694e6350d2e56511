"""Learnt recurrent weights formed synapse by synapse (``network._edge_connectome``), on
the CPU: the compressed form the HIP engine is given for a side whose blocks are learnt
full-rank projections holds the same synapses, weights and parameter gradients, bit for
bit, as the dense rows the reference assembles (``network.py:731-764``)."""

import torch

import scenarios as sc


def _learnt(seed=sc.SEED):
    built = sc.recurrent(sc.BATCH_SIZE, seed, learnt_weights=True)
    model = built.model
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for p in model.parameters():
            p.add_(0.05 * torch.randn(p.shape, generator=g))
    side = next(i for i, s in enumerate(model._sides) if s.recurrent)
    pathways = [p for p in model.pathways if p.side == side]
    return model, side, pathways


def test_synapses_and_weights_equal_the_dense_rows():
    model, side, pathways = _learnt()
    conn = model._edge_connectome(side)
    assert conn.n_pathways == len(pathways) == 2 and conn.n_edges > 0
    for k, pathway in enumerate(pathways):
        rows, W = conn.dense_rows(k)
        assert torch.equal(rows, getattr(model, f"_rows_{pathway.index}"))
        assert torch.equal(W, model._assemble(pathway).detach())
    # CSR by source, targets ascending within a source
    starts = torch.zeros(conn.n_edges, dtype=torch.bool)
    starts[conn.indptr[:-1][conn.indptr[:-1] < conn.n_edges]] = True
    steps = conn.targets[1:].long() - conn.targets[:-1].long()
    assert bool(((steps > 0) | starts[1:]).all())


def test_parameter_gradients_equal_the_dense_path():
    """A loss linear in the synapses' weights: the log-weights' gradients through the
    synapse-by-synapse form equal those through the dense rows and their gather."""
    model, side, pathways = _learnt()
    conn = model._edge_connectome(side)
    g = torch.Generator().manual_seed(5)
    coef = torch.randn(conn.n_edges, generator=g)
    model.zero_grad()
    (conn.weights * coef).sum().backward()
    sparse = {n: p.grad.clone() for n, p in model.named_parameters() if p.grad is not None}
    model.zero_grad()
    e_src = torch.repeat_interleave(torch.arange(conn.n_sources), conn.out_degree())
    total = 0.0
    for k, pathway in enumerate(pathways):
        W = model._assemble(pathway)
        rows, _ = conn.dense_rows(k)
        pick = conn.pathway[e_src] == k
        local = torch.searchsorted(rows, e_src[pick])  # the synapse's row within W
        total = total + (W[local, conn.targets[pick].long()] * coef[pick]).sum()
    total.backward()
    dense = {n: p.grad.clone() for n, p in model.named_parameters() if p.grad is not None}
    assert sparse.keys() == dense.keys() and sparse
    for name in sparse:
        assert torch.equal(sparse[name], dense[name]), name


def test_kernels_are_never_given_weights_off_the_side_device():
    """A compressed side refuses, before any launch, weights the kernels could not read:
    on another device than its structure, or not float32 (``engine._Side.abi``)."""
    import numpy as np
    import pytest

    from wiretorch_amd import connectome, engine

    conn = connectome.from_edges(4, 5, np.array([0, 0, 2]), np.array([1, 3, 4]),
                                 np.array([0.5, 1.0, 2.0]), np.array([0, -1, 0, -1]), 1)
    side = engine._Side(conn, conn.pathway.to(torch.int32))
    with pytest.raises(ValueError, match="float32 on the side's device"):
        side.abi(1, 32, 0, conn.weights.double())
    with pytest.raises(ValueError, match="float32 on the side's device"):
        side.abi(1, 32, 0, conn.weights.to("meta"))
