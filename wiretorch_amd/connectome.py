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

On disk (``save`` / ``load``) a connectome is one ``.npz`` archive of plain arrays —
``indptr``, ``targets``, ``weights``, ``pathway`` and the sizes — written and read with
numpy (no pickled objects), so a fly-scale graph (50M synapses: ~0.6 GB) is built once and
reloaded in seconds. The reference keeps connectivity only as dense per-type-pair arrays
(``projections.py:290-495``).
"""

from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

#: Format tag of the ``.npz`` archives ``save`` writes.
FORMAT = "wiretorch_amd.connectome/csr-by-source/1"


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


def save(conn: Connectome, path) -> Path:
    """Write ``conn`` to ``path`` (``.npz``): CSR by source, targets ascending per source."""
    path = Path(path)
    np.savez(
        path, format=np.array(FORMAT), n_sources=np.int64(conn.n_sources),
        n_targets=np.int64(conn.n_targets), n_pathways=np.int64(conn.n_pathways),
        indptr=conn.indptr.detach().cpu().numpy().astype(np.int64),
        targets=conn.targets.detach().cpu().numpy().astype(np.int32),
        weights=conn.weights.detach().cpu().numpy().astype(np.float32),
        pathway=conn.pathway.detach().cpu().numpy().astype(np.int64),
    )  # fmt: skip
    return path if path.suffix == ".npz" else path.with_name(path.name + ".npz")


def load(path, device="cpu") -> Connectome:
    """A connectome written by ``save``; its structure is checked (sizes, ranges, targets
    strictly ascending within each source)."""
    with np.load(Path(path), allow_pickle=False) as f:
        if str(f["format"]) != FORMAT:
            raise ValueError(f"{path}: not a {FORMAT} archive")
        n_src, n_tgt = int(f["n_sources"]), int(f["n_targets"])
        indptr, targets = f["indptr"], f["targets"]
        weights, pathway = f["weights"], f["pathway"]
        n_path = int(f["n_pathways"])
    check_structure(n_src, n_tgt, indptr, targets, weights, pathway, n_path)
    return Connectome(
        n_src, n_tgt, torch.from_numpy(indptr).to(device), torch.from_numpy(targets).to(device),
        torch.from_numpy(weights).to(device), torch.from_numpy(pathway).to(device), n_path,
    )  # fmt: skip


def check_structure(n_src, n_tgt, indptr, targets, weights, pathway, n_path) -> None:
    """Raise ``ValueError`` unless the arrays form a valid CSR-by-source connectome."""
    E = targets.shape[0]
    if indptr.shape != (n_src + 1,) or indptr[0] != 0 or indptr[-1] != E:
        raise ValueError("indptr must have n_sources + 1 entries from 0 to the edge count")
    if np.any(np.diff(indptr) < 0):
        raise ValueError("indptr must be non-decreasing")
    if weights.shape != (E,) or pathway.shape != (n_src,):
        raise ValueError("weights must have one entry per edge, pathway one per source")
    if E and (targets.min() < 0 or targets.max() >= n_tgt):
        raise ValueError("targets out of range")
    if n_src and (pathway.max() >= n_path or pathway.min() < -1):
        raise ValueError("pathway ids must be -1 or below n_pathways")
    if E > 1:
        starts = np.zeros(E, dtype=bool)
        starts[indptr[:-1][indptr[:-1] < E]] = True
        if np.any((np.diff(targets.astype(np.int64)) <= 0) & ~starts[1:]):
            raise ValueError("targets must be strictly ascending within each source")
