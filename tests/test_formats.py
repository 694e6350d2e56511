"""On-disk connectome formats (CPU): a compressed connectome and a whole-side
``SparseProjection`` written to ``.npz`` and read back are the same arrays, drive the
oracle to the same raster, and malformed archives are refused; the network's state
round-trips through ``get_checkpoint_state`` / ``load_checkpoint_state``."""

import numpy as np
import pytest
import torch

import oracle.dynamics as oracle_engine
import scenarios as sc
from wiretorch_amd import connectome, synthetic
from wiretorch_amd.projections import SparseProjection


def _small_fly(**kw):
    return synthetic.fly_scale_network(N=800, n_types=30, mean_degree=40, k_max=200, B=2,
                                       T=60, **kw)


def test_connectome_round_trip(tmp_path):
    wl = synthetic.fly_scale(N=800, n_types=30, mean_degree=40, k_max=200, B=2, T=60)
    conn = wl.drive.sparse_recurrent
    path = connectome.save(conn, tmp_path / "rec")
    back = connectome.load(path)
    assert (back.n_sources, back.n_targets, back.n_pathways) == (conn.n_sources, conn.n_targets,
                                                                conn.n_pathways)
    for name in ("indptr", "targets", "weights", "pathway"):
        a, b = getattr(conn, name), getattr(back, name)
        assert a.dtype == b.dtype and torch.equal(a, b), name


def test_connectome_structure_is_checked(tmp_path):
    conn = connectome.from_edges(4, 5, [0, 0, 2], [1, 3, 4], [1.0, 2.0, 3.0], [0, 0, 0, -1], 1)
    good = connectome.save(conn, tmp_path / "c.npz")
    connectome.load(good)
    with np.load(good) as f:
        arrays = dict(f)
    arrays["targets"] = np.array([3, 1, 4], dtype=np.int32)  # descending within source 0
    np.savez(tmp_path / "bad.npz", **arrays)
    with pytest.raises(ValueError, match="ascending"):
        connectome.load(tmp_path / "bad.npz")
    arrays["targets"] = np.array([1, 3, 5], dtype=np.int32)  # out of range
    np.savez(tmp_path / "bad.npz", **arrays)
    with pytest.raises(ValueError, match="range"):
        connectome.load(tmp_path / "bad.npz")


@pytest.mark.parametrize("learn_sf", [False, True])
def test_sparse_projection_round_trip_drives_the_same_network(tmp_path, learn_sf):
    wl = _small_fly(learn_sf=learn_sf)
    model = wl.model
    proj = model.rec_projections
    path = proj.save(tmp_path / "rec")
    back = SparseProjection.load(path, learn_sf=learn_sf)
    for name in ("indptr", "targets", "counts", "pair"):
        assert torch.equal(getattr(proj, name), getattr(back, name)), name
    assert torch.equal(proj.factors().detach(), back.factors().detach())
    assert torch.equal(proj().detach(), back().detach())
    x = torch.from_numpy(wl.x).float()
    sc.use_engine(model, oracle_engine)
    with torch.no_grad():
        model.reset_state()
        want = model(x)
        model.rec_projections = back
        model.reset_state()
        got = model(x)
    assert want.sum() > 0 and torch.equal(got, want)


def test_checkpoint_state_round_trip():
    wl = _small_fly()
    model = wl.model
    sc.use_engine(model, oracle_engine)
    x = torch.from_numpy(wl.x).float()
    with torch.no_grad():
        model.reset_state()
        model(x[:, :30])
        state = model.get_checkpoint_state()
        want = model(x[:, 30:])
        model.load_checkpoint_state(state)
        got = model(x[:, 30:])
    assert set(state) == {"v", "g", "refractory"}
    assert torch.equal(got, want)
