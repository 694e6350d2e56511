"""Connectivity blocks, one per (source cell type, target cell type).

A ``Projection`` produces its ``(n_source, n_target)`` weight block on demand. The
caching mode tells the network what may be computed once:

* ``"fixed"`` (``FrozenProjection``): weights fixed at construction;
* ``"scaling_factors"`` (``ScalingFactorProjection``): a fixed connectome times one
  learnt factor, which the network applies to the synaptic kernel;
* ``"weights"`` (``FullRankProjection``, ``LowRankProjection``, ``SignedProjection``):
  weights assembled from parameters on every call.

Follows ``src/wiretorch/network_simulators/projections.py:34-216`` (the same four
classes, parameterisations and caching modes) and ``:340-392``
(``make_frozen_projections``).
"""

from __future__ import annotations

import numpy as np
import torch
from torch import nn

PairKey = tuple[str, str]


def _float32(values) -> torch.Tensor:
    if isinstance(values, np.ndarray):
        return torch.from_numpy(values).float()
    return values.float()


class Projection(nn.Module):
    """One (source type, target type) block; subclasses define ``forward``."""

    def __init__(self, n_source: int, n_target: int):
        super().__init__()
        self.n_source = int(n_source)
        self.n_target = int(n_target)

    @property
    def caching_mode(self) -> str:
        raise NotImplementedError

    def forward(self) -> torch.Tensor:  # type: ignore[override]
        raise NotImplementedError

    def kernel_factor(self):
        """A factor the network applies to the synaptic kernel (None: none)."""
        return None


class FrozenProjection(Projection):
    """Constant weights (a buffer)."""

    def __init__(self, weights):
        w = _float32(weights)
        if w.ndim != 2:
            raise ValueError(f"weights must be 2D, got shape {tuple(w.shape)}")
        super().__init__(*w.shape)
        self.register_buffer("_weights", w)

    @property
    def caching_mode(self) -> str:
        return "fixed"

    def forward(self) -> torch.Tensor:
        return self._weights


class ScalingFactorProjection(Projection):
    """A fixed connectome and one learnt scaling factor, ``exp(log_sf)``."""

    def __init__(self, connectome, init_sf: float = 1.0):
        c = _float32(connectome)
        if c.ndim != 2:
            raise ValueError(f"connectome must be 2D, got shape {tuple(c.shape)}")
        super().__init__(*c.shape)
        self.register_buffer("connectome", c)
        self.log_sf = nn.Parameter(
            torch.tensor(float(np.log(init_sf + 1e-8)), dtype=torch.float32)
        )

    @property
    def caching_mode(self) -> str:
        return "scaling_factors"

    def forward(self) -> torch.Tensor:
        return torch.exp(self.log_sf) * self.connectome

    def kernel_factor(self) -> torch.Tensor:
        return torch.exp(self.log_sf)


class FullRankProjection(Projection):
    """Learnt per-connection log-weights: ``exp(log_weights) * mask``."""

    def __init__(self, init_weights, mask=None):
        w = _float32(init_weights)
        if w.ndim != 2:
            raise ValueError(f"init_weights must be 2D, got shape {tuple(w.shape)}")
        super().__init__(*w.shape)
        self.log_weights = nn.Parameter(torch.log(w + 1e-8))
        m = torch.ones_like(w) if mask is None else _float32(mask)
        if m.shape != w.shape:
            raise ValueError(f"mask shape {tuple(m.shape)} != {tuple(w.shape)}")
        self.register_buffer("mask", m)

    @property
    def caching_mode(self) -> str:
        return "weights"

    def forward(self) -> torch.Tensor:
        return torch.exp(self.log_weights) * self.mask


class LowRankProjection(Projection):
    """Low-rank log-weights: ``exp(U @ V) * mask``."""

    def __init__(self, n_source, n_target, rank, U_init=None, V_init=None, mask=None):
        super().__init__(n_source, n_target)
        if rank <= 0:
            raise ValueError(f"rank must be positive, got {rank}")
        spread = 1.0 / np.sqrt(rank)
        U = torch.randn(n_source, rank) * spread if U_init is None else _float32(U_init)
        V = torch.randn(rank, n_target) * spread if V_init is None else _float32(V_init)
        if tuple(U.shape) != (n_source, rank) or tuple(V.shape) != (rank, n_target):
            raise ValueError("U_init / V_init have the wrong shape")
        self.U = nn.Parameter(U)
        self.V = nn.Parameter(V)
        m = torch.ones(n_source, n_target) if mask is None else _float32(mask)
        if tuple(m.shape) != (n_source, n_target):
            raise ValueError(f"mask shape {tuple(m.shape)} != ({n_source}, {n_target})")
        self.register_buffer("mask", m)

    @property
    def caching_mode(self) -> str:
        return "weights"

    def forward(self) -> torch.Tensor:
        return torch.exp(self.U @ self.V) * self.mask


class SignedProjection(Projection):
    """Learnt per-connection weights of either sign: ``weights * mask``.

    The reference's projections are all non-negative (log-parameterised,
    ``projections.py:121-216``) and take the sign from the synapse type; a rate network
    with a dense signed matrix (a random ``N(0, g^2/N)`` recurrent matrix and its Gaussian
    input weights) learns the weights themselves. ``mask`` (default: every connection)
    fixes which entries exist."""

    def __init__(self, init_weights, mask=None):
        w = _float32(init_weights)
        if w.ndim != 2:
            raise ValueError(f"init_weights must be 2D, got shape {tuple(w.shape)}")
        super().__init__(*w.shape)
        self.weights = nn.Parameter(w.clone())
        if mask is not None:
            m = _float32(mask)
            if m.shape != w.shape:
                raise ValueError(f"mask shape {tuple(m.shape)} != {tuple(w.shape)}")
            self.register_buffer("mask", m)
        else:
            self.mask = None

    @property
    def caching_mode(self) -> str:
        return "weights"

    def forward(self) -> torch.Tensor:
        return self.weights if self.mask is None else self.weights * self.mask


def _members(types: np.ndarray, names: list[str]) -> dict[str, np.ndarray]:
    return {name: np.flatnonzero(types == i) for i, name in enumerate(names)}


def make_frozen_projections(
    rec_weights,
    ff_weights,
    cell_type_indices,
    ff_cell_type_indices,
    cell_type_names,
    ff_cell_type_names,
    scaling_factors_rec=None,
    scaling_factors_ff=None,
):
    """``FrozenProjection`` blocks of a recurrent and a feedforward matrix, every
    (source type, target type) pair, optionally scaled per pair."""
    targets = _members(np.asarray(cell_type_indices), cell_type_names)
    ff_sources = _members(np.asarray(ff_cell_type_indices), ff_cell_type_names)

    def blocks(weights, sources, source_names, factors):
        out = {}
        for a, src in enumerate(source_names):
            for b, tgt in enumerate(cell_type_names):
                block = weights[np.ix_(sources[src], targets[tgt])].astype(np.float32)
                if factors is not None:
                    block = block * float(factors[a, b])
                out[(src, tgt)] = FrozenProjection(block)
        return out

    return (
        blocks(rec_weights, targets, cell_type_names, scaling_factors_rec),
        blocks(ff_weights, ff_sources, ff_cell_type_names, scaling_factors_ff),
    )


def projection_mask(projection: Projection) -> np.ndarray:
    """Where a projection has connections (at construction), as a bool array."""
    for name in ("connectome", "mask", "_weights"):
        tensor = getattr(projection, name, None)
        if isinstance(tensor, torch.Tensor):
            return tensor.detach().cpu().numpy() != 0
    if isinstance(projection, SignedProjection):
        return np.ones((projection.n_source, projection.n_target), dtype=bool)
    raise TypeError(f"unknown Projection subclass {type(projection).__name__}")
