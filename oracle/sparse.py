"""Propagation through a compressed connectome on the CPU — TEST INFRASTRUCTURE ONLY
(see ``oracle/__init__.py``).

``activations(conn, s)`` gives ``a_k[r, n] = sum over sources j of pathway k of
s[r, j] * W[j, n]`` — the quantity the reference computes as ``s[:, rows] @ W`` per
pathway (``network_simulators/network.py:260-271``, ``:142-157``) — event by event:
only sources with ``s != 0`` are visited. Products are rounded to float32 (as the
reference's float32 product does) and summed in float64, then rounded to float32 once:
for spike inputs this is the exactly rounded sum, i.e. the reference's value up to the
order-dependent rounding of its float32 accumulation.
"""

from __future__ import annotations

import torch


def expand(indptr: torch.Tensor, sources: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Edge indices of ``sources`` back to back, and each edge's position in ``sources``."""
    starts = indptr[sources]
    counts = indptr[sources + 1] - starts
    owner = torch.repeat_interleave(torch.arange(sources.numel()), counts)
    first = torch.cumsum(counts, 0) - counts
    edge = torch.arange(int(counts.sum())) - first[owner] + starts[owner]
    return edge, owner


def activations(conn, s: torch.Tensor) -> torch.Tensor:
    """``(n_pathways, R, n_targets)`` float32 from ``s`` ``(R, n_sources)``."""
    s = s.detach().cpu().float()
    indptr = conn.indptr.cpu()
    targets = conn.targets.cpu().long()
    weights = conn.weights.cpu()
    pathway = conn.pathway.cpu()
    R = s.shape[0]
    out = torch.zeros((conn.n_pathways, R, conn.n_targets), dtype=torch.float64)
    for r in range(R):
        src = torch.nonzero(s[r] * (pathway >= 0)).flatten()
        if src.numel() == 0:
            continue
        edge, owner = expand(indptr, src)
        values = (weights[edge] * s[r, src][owner]).double()  # float32 product, then widen
        out[:, r].index_put_((pathway[src][owner], targets[edge]), values, accumulate=True)
    return out.float()
