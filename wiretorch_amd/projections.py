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

from pathlib import Path

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

    def edge_mask(self) -> torch.Tensor | None:
        """The entries the block can hold (nonzero), if ``edge_values`` forms entries one
        at a time; None if the block is only formed whole."""
        return None

    def edge_values(self, flat: torch.Tensor) -> torch.Tensor:
        """The block's entries at row-major positions ``flat``, formed for those entries
        only: equal, entry for entry, to ``self()`` there (and differentiable alike)."""
        raise NotImplementedError


class FrozenProjection(Projection):
    """Constant weights (a buffer)."""

    def __init__(self, weights):
        w = _float32(weights)
        if w.ndim != 2:
            raise ValueError(f"weights of shape {tuple(w.shape)}: a (source, target) matrix expected")
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
            raise ValueError(f"connectome of shape {tuple(c.shape)}: a (source, target) matrix expected")
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
            raise ValueError(f"initial weights of shape {tuple(w.shape)}: a (source, target) matrix expected")
        super().__init__(*w.shape)
        self.log_weights = nn.Parameter(torch.log(w + 1e-8))
        m = torch.ones_like(w) if mask is None else _float32(mask)
        if m.shape != w.shape:
            raise ValueError(f"mask {tuple(m.shape)} and weights {tuple(w.shape)} differ in shape")
        self.register_buffer("mask", m)

    @property
    def caching_mode(self) -> str:
        return "weights"

    def forward(self) -> torch.Tensor:
        return torch.exp(self.log_weights) * self.mask

    def edge_mask(self) -> torch.Tensor:
        return self.mask

    def edge_values(self, flat: torch.Tensor) -> torch.Tensor:
        # (index_select: ``flat`` holds distinct positions, and the gradient is then
        # scattered without sorting them)
        return (torch.exp(self.log_weights.reshape(-1).index_select(0, flat))
                * self.mask.reshape(-1).index_select(0, flat))


class LowRankProjection(Projection):
    """Low-rank log-weights: ``exp(U @ V) * mask``."""

    def __init__(self, n_source, n_target, rank, U_init=None, V_init=None, mask=None):
        super().__init__(n_source, n_target)
        if rank <= 0:
            raise ValueError(f"rank {rank} is not a positive number")
        spread = 1.0 / np.sqrt(rank)
        U = torch.randn(n_source, rank) * spread if U_init is None else _float32(U_init)
        V = torch.randn(rank, n_target) * spread if V_init is None else _float32(V_init)
        if tuple(U.shape) != (n_source, rank) or tuple(V.shape) != (rank, n_target):
            raise ValueError("U_init / V_init have the wrong shape")
        self.U = nn.Parameter(U)
        self.V = nn.Parameter(V)
        m = torch.ones(n_source, n_target) if mask is None else _float32(mask)
        if tuple(m.shape) != (n_source, n_target):
            raise ValueError(f"mask {tuple(m.shape)} is not ({n_source}, {n_target})")
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
            raise ValueError(f"initial weights of shape {tuple(w.shape)}: a (source, target) matrix expected")
        super().__init__(*w.shape)
        self.weights = nn.Parameter(w.clone())
        if mask is not None:
            m = _float32(mask)
            if m.shape != w.shape:
                raise ValueError(f"mask {tuple(m.shape)} and weights {tuple(w.shape)} differ in shape")
            self.register_buffer("mask", m)
        else:
            self.mask = None

    @property
    def caching_mode(self) -> str:
        return "weights"

    def forward(self) -> torch.Tensor:
        return self.weights if self.mask is None else self.weights * self.mask

    def edge_mask(self) -> torch.Tensor | None:
        return self.mask

    def edge_values(self, flat: torch.Tensor) -> torch.Tensor:
        return (self.weights.reshape(-1).index_select(0, flat)
                * self.mask.reshape(-1).index_select(0, flat))


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


# ====================================================================
# A whole side in compressed form (connectomes too large for dense blocks)
# ====================================================================


#: Format tag of the ``.npz`` archives ``SparseProjection.save`` writes.
SPARSE_FORMAT = "wiretorch_amd.sparse_projection/1"


class SparseProjection(nn.Module):
    """Every synapse of one input side, compressed by source, with one scaling factor per
    (source cell type, target cell type) pair.

    The reference describes a side as one dense ``(n_source, n_target)`` block per type
    pair, each a ``ScalingFactorProjection`` (``projections.py:100-131``: weights
    ``exp(log_sf) * connectome``, the factor applied to the synapse kernel). At fly scale
    (140k neurons, 8000 cell types, ~50M synapses) neither the blocks (one module per
    pair, dense rows of 140k) nor the network's dense masks can exist. This holds the same
    information by synapse:

    * ``indptr`` ``(n_source + 1,)`` int64, ``targets`` ``(E,)`` int32 ascending per
      source, ``counts`` ``(E,)`` float32 — the connectome (synapse counts);
    * ``pair`` ``(E,)`` int64 — each synapse's (source type, target type) pair,
      ``source_type * n_target_types + target_type``;
    * the factors ``(n_source_types, n_target_types)``: the parameter ``log_sf`` when
      learnt, else the buffer ``sf``.

    ``forward()`` gives each synapse's weight ``count * sf[pair]`` (float32), the factor
    folded into the weights rather than the kernel: the activation it feeds is the same
    sum. Duplicate (source, target) entries in the input are summed.
    """

    caching_mode = "sparse"

    def __init__(self, n_source: int, n_target: int, source, target, counts, source_types,
                 target_types, sf=1.0, learn_sf: bool = False, n_source_types=None,
                 n_target_types=None):
        super().__init__()
        as_long = lambda a: torch.as_tensor(np.asarray(a) if not torch.is_tensor(a) else a).long()  # noqa: E731
        src, tgt = as_long(source), as_long(target)
        c = torch.as_tensor(counts if torch.is_tensor(counts) else np.asarray(counts)).float()
        device = src.device
        src_types, tgt_types = as_long(source_types).to(device), as_long(target_types).to(device)
        self.n_source, self.n_target = int(n_source), int(n_target)
        if src_types.numel() != self.n_source or tgt_types.numel() != self.n_target:
            raise ValueError("source_types / target_types must give one type per neuron")
        if src.numel() and (int(src.min()) < 0 or int(src.max()) >= self.n_source
                            or int(tgt.min()) < 0 or int(tgt.max()) >= self.n_target):
            raise ValueError("synapse endpoints out of range")
        n_st = int(n_source_types if n_source_types is not None else int(src_types.max()) + 1)
        n_tt = int(n_target_types if n_target_types is not None else int(tgt_types.max()) + 1)
        key = src * self.n_target + tgt
        key, order = torch.sort(key)
        c = c.to(device)[order]
        uniq, inverse = torch.unique_consecutive(key, return_inverse=True)
        if uniq.numel() != key.numel():  # repeated pairs: their counts summed (in float64)
            merged = torch.zeros(uniq.numel(), dtype=torch.float64, device=device)
            merged.index_add_(0, inverse, c.double())
            c = merged.float()
        s_u, t_u = uniq // self.n_target, uniq % self.n_target
        indptr = torch.zeros(self.n_source + 1, dtype=torch.int64, device=device)
        indptr[1:] = torch.cumsum(torch.bincount(s_u, minlength=self.n_source), 0)
        self.register_buffer("indptr", indptr)
        self.register_buffer("targets", t_u.to(torch.int32).contiguous())
        self.register_buffer("counts", c.contiguous())
        self.register_buffer("pair", (src_types[s_u] * n_tt + tgt_types[t_u]).contiguous())
        self.n_source_types, self.n_target_types = n_st, n_tt
        table = torch.as_tensor(sf if torch.is_tensor(sf) else np.asarray(sf, dtype=np.float32))
        table = table.float().to(device).expand(n_st, n_tt).contiguous()
        if learn_sf:
            if not bool((table > 0).all()):
                raise ValueError("learnt scaling factors must start positive")
            # log(sf + 1e-8) in float64, rounded once: ScalingFactorProjection's start
            self.log_sf = nn.Parameter(torch.log(table.double() + 1e-8).float())
        else:
            self.register_buffer("sf", table)
        self._memo = None

    @property
    def n_edges(self) -> int:
        return int(self.targets.numel())

    def factors(self) -> torch.Tensor:
        """``(n_source_types, n_target_types)`` scaling factors."""
        return torch.exp(self.log_sf) if hasattr(self, "log_sf") else self.sf

    def forward(self) -> torch.Tensor:  # type: ignore[override]
        """``(E,)`` float32 synapse weights, ``count * sf[pair]``. Without autograd
        (fixed factors, or under ``no_grad``) the result is reused while the factors and
        counts are unchanged."""
        table = self.log_sf if hasattr(self, "log_sf") else self.sf
        tracking = torch.is_grad_enabled() and table.requires_grad
        key = (table.data_ptr(), table._version, self.counts.data_ptr(), self.counts._version,
               self.pair.data_ptr())
        if not tracking and self._memo is not None and self._memo[0] == key:
            return self._memo[1]
        w = self.counts * self.factors().reshape(-1)[self.pair]
        if not tracking:
            self._memo = (key, w.detach())
        return w

    def _apply(self, fn, recurse=True):
        self._memo = None  # device or dtype moves invalidate the reused weights
        return super()._apply(fn, recurse)

    def save(self, path):
        """Write the connectome and the current factors to ``path`` (``.npz``, plain
        arrays): ``SparseProjection.load`` rebuilds the projection without re-sorting."""
        path = Path(path)
        np.savez(
            path, format=np.array(SPARSE_FORMAT), n_source=np.int64(self.n_source),
            n_target=np.int64(self.n_target), n_source_types=np.int64(self.n_source_types),
            n_target_types=np.int64(self.n_target_types),
            indptr=self.indptr.cpu().numpy(), targets=self.targets.cpu().numpy(),
            counts=self.counts.cpu().numpy(), pair=self.pair.cpu().numpy(),
            sf=self.factors().detach().cpu().numpy(),
            **({"log_sf": self.log_sf.detach().cpu().numpy()} if hasattr(self, "log_sf") else {}),
        )  # fmt: skip
        return path if path.suffix == ".npz" else path.with_name(path.name + ".npz")

    @classmethod
    def load(cls, path, learn_sf: bool = False, device="cpu") -> "SparseProjection":
        """A projection written by ``save`` (its factors learnt from there if ``learn_sf``)."""
        from wiretorch_amd.connectome import check_structure

        with np.load(Path(path), allow_pickle=False) as f:
            if str(f["format"]) != SPARSE_FORMAT:
                raise ValueError(f"{path}: not a {SPARSE_FORMAT} archive")
            arrays = {k: f[k] for k in ("indptr", "targets", "counts", "pair", "sf")}
            log_sf = f["log_sf"] if "log_sf" in f.files else None
            sizes = {k: int(f[k]) for k in ("n_source", "n_target", "n_source_types",
                                             "n_target_types")}
        n_src, n_tgt = sizes["n_source"], sizes["n_target"]
        check_structure(n_src, n_tgt, arrays["indptr"], arrays["targets"], arrays["counts"],
                        np.zeros(n_src, dtype=np.int64), 1)
        n_pairs = sizes["n_source_types"] * sizes["n_target_types"]
        if arrays["sf"].shape != (sizes["n_source_types"], sizes["n_target_types"]) or (
                arrays["pair"].size and (arrays["pair"].min() < 0 or arrays["pair"].max() >= n_pairs)):
            raise ValueError(f"{path}: scaling factors or pair indices do not match")
        self = cls.__new__(cls)
        nn.Module.__init__(self)
        self.n_source, self.n_target = n_src, n_tgt
        self.n_source_types, self.n_target_types = sizes["n_source_types"], sizes["n_target_types"]
        for name in ("indptr", "targets", "counts", "pair"):
            self.register_buffer(name, torch.from_numpy(arrays[name]).to(device))
        table = torch.from_numpy(arrays["sf"]).float().to(device)
        if learn_sf and log_sf is not None:  # the learnt logarithms themselves
            self.log_sf = nn.Parameter(torch.from_numpy(log_sf).float().to(device))
        elif learn_sf:
            self.log_sf = nn.Parameter(torch.log(table.double() + 1e-8).float())
        else:
            self.register_buffer("sf", table)
        self._memo = None
        return self

    def dense(self) -> torch.Tensor:
        """``(n_source, n_target)`` weights, for small networks (tests, inspection)."""
        if self.n_source * self.n_target > 1 << 28:
            raise ValueError("too large for a dense matrix")
        W = torch.zeros((self.n_source, self.n_target), device=self.counts.device)
        src = torch.repeat_interleave(torch.arange(self.n_source, device=self.counts.device),
                                      self.indptr[1:] - self.indptr[:-1])
        W[src, self.targets.long()] = self.forward()
        return W
