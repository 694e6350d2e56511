"""Compressed connectomes: the sparse form of a ``Drive``'s pathways.

The reference stores each pathway as dense ``(n_rows, N)`` weight rows
(``network_simulators/network.py:106-157``), which cannot hold a fly-scale connectome
(140k² floats). A ``Connectome`` holds the same information by source:

* ``indptr`` ``(n_sources + 1,)`` int64 and ``targets`` ``(E,)`` int32, ``weights``
  ``(E,)`` float32: source ``j``'s synapses are ``indptr[j]:indptr[j + 1]``, targets
  ascending;
* ``pathway`` ``(n_sources,)`` int64: the pathway each source feeds (-1: none). For a
  network built from projections this is the source's cell type pathway; for a fly-scale
  connectome with per-type-pair scaling factors folded into ``weights`` it is the
  receptor kind (excitatory / inhibitory).

``a_k[b, n] = sum over sources j of pathway k of x[b, j] * W[j, n]`` is the activation
both forms define.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch


@dataclass
class Connectome:
    n_sources: int
    n_targets: int
    indptr: torch.Tensor
    targets: torch.Tensor
    weights: torch.Tensor
    pathway: torch.Tensor
    n_pathways: int

    @property
    def n_edges(self) -> int:
        return int(self.targets.numel())

    @property
    def device(self) -> torch.device:
        return self.targets.device

    def to(self, device) -> "Connectome":
        return Connectome(
            self.n_sources, self.n_targets, self.indptr.to(device),
            self.targets.to(device), self.weights.to(device),
            self.pathway.to(device), self.n_pathways,
        )  # fmt: skip

    def out_degree(self) -> torch.Tensor:
        return self.indptr[1:] - self.indptr[:-1]

    def dense_rows(self, k: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Pathway ``k`` as the reference's ``(rows, W)``: for tests on small networks."""
        rows = torch.nonzero(self.pathway == k).flatten()
        W = torch.zeros((rows.numel(), self.n_targets), dtype=torch.float32,
                        device=self.device)
        for i, j in enumerate(rows.tolist()):
            a, b = int(self.indptr[j]), int(self.indptr[j + 1])
            W[i, self.targets[a:b].long()] = self.weights[a:b]
        return rows, W


def from_pathways(pathways: list[tuple[torch.Tensor, torch.Tensor]], n_sources: int,
                  n_targets: int) -> Connectome:
    """The compressed form of dense pathways ``[(rows, W (n_rows, N))]``; source rows of
    different pathways must be disjoint. Zero weights are dropped."""
    device = pathways[0][1].device if pathways else torch.device("cpu")
    pathway = torch.full((n_sources,), -1, dtype=torch.int64, device=device)
    per_source_W = torch.zeros((n_sources, n_targets), dtype=torch.float32, device=device)
    for k, (rows, W) in enumerate(pathways):
        rows = rows.to(device).long()
        if bool((pathway[rows] >= 0).any()):
            raise ValueError("pathways share source rows; the compressed form needs them disjoint")
        pathway[rows] = k
        per_source_W[rows] = W.detach().float()
    return from_dense(per_source_W, pathway, len(pathways))


def from_dense(W: torch.Tensor, pathway: torch.Tensor, n_pathways: int) -> Connectome:
    """Compress ``(n_sources, N)`` weights (zeros dropped), sources tagged by pathway."""
    W = W.detach().float()
    nz = W != 0
    counts = nz.sum(dim=1)
    indptr = torch.zeros(W.shape[0] + 1, dtype=torch.int64, device=W.device)
    indptr[1:] = torch.cumsum(counts, dim=0)
    src, tgt = torch.nonzero(nz, as_tuple=True)  # row-major: targets ascending per row
    return Connectome(
        int(W.shape[0]), int(W.shape[1]), indptr, tgt.to(torch.int32).contiguous(),
        W[src, tgt].contiguous(), pathway.to(W.device).long().contiguous(), int(n_pathways),
    )  # fmt: skip


def from_edges(n_sources: int, n_targets: int, src: np.ndarray, tgt: np.ndarray,
               weights: np.ndarray, pathway: np.ndarray, n_pathways: int,
               device="cpu") -> Connectome:
    """From an edge list (duplicates of one (source, target) pair are summed)."""
    src = np.asarray(src, dtype=np.int64)
    tgt = np.asarray(tgt, dtype=np.int64)
    w = np.asarray(weights, dtype=np.float32)
    key = src * n_targets + tgt
    order = np.argsort(key, kind="stable")
    key, w = key[order], w[order]
    uniq, first = np.unique(key, return_index=True)
    if uniq.size != key.size:  # sum duplicates in float64, then round once
        w = np.add.reduceat(w.astype(np.float64), first).astype(np.float32)
    s = uniq // n_targets
    t = uniq % n_targets
    counts = np.bincount(s, minlength=n_sources)
    indptr = np.zeros(n_sources + 1, dtype=np.int64)
    np.cumsum(counts, out=indptr[1:])
    return Connectome(
        int(n_sources), int(n_targets), torch.from_numpy(indptr).to(device),
        torch.from_numpy(t.astype(np.int32)).to(device), torch.from_numpy(w).to(device),
        torch.from_numpy(np.asarray(pathway, dtype=np.int64)).to(device), int(n_pathways),
    )  # fmt: skip
