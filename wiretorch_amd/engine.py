"""The HIP engine: ``simulate`` and its autograd function, over ``libwiretorch_amd.so``.

``simulate(v, g, x, drive, p, *, refractory, ..., probabilities, track, track_batch_idx,
retain) -> Run`` keeps the reference's contract (``conductance/engine.py:71-89``): the
inputs are never modified (state is copied before the kernels update it in place), the
returned ``Run`` holds spikes ``(B, T, N)``, the final ``v``, ``g`` as a ``(B, N, 2, S)``
view, the refractory counters, probabilities and the tracked variables.

What differs from the reference is underneath:

* one persistent launch (``wt_cond_run``) runs all T steps of a chunk, recurrent or
  feedforward — the feedforward drive is propagated from the input's nonzero entries
  per step instead of being materialised as ``(K_ff, B, T, N)`` by matmuls
  (``network_simulators/engine.py:123-145``);
* connectivity is compressed by source (``connectome.Connectome``); dense pathways are
  converted once (cached while their tensors are unchanged);
* gradients (``_Run``, the counterpart of ``_FeedforwardScan`` / ``_RecurrentRun``,
  ``conductance/engine.py:444-544``) come from ``wt_cond_scan_backward`` — or, when the
  drive asks for gradients through the recurrent spikes (``recurrent_gradients``),
  ``wt_cond_recurrent_backward`` — and the event-driven ``wt_weight_gradient``.

The engine runs only on a GPU with the library built; it raises otherwise. Not
supported (raising ``NotImplementedError``): per-step gradient retention
(``retain``), float16 storage, sampled spikes, presynaptic dynamics. The NMDA Mg block
(``Physiology.mg_c`` / ``mg_a``) and spike-frequency adaptation (``Physiology.adapt`` /
``adapt_decay`` / ``E_adapt``, its conductances entering as ``adaptation`` and leaving as
``Run.adaptation``) are evaluated in the forward and both backward passes.
"""

from __future__ import annotations

import math
from collections import OrderedDict
from dataclasses import dataclass, field, replace

import torch

from wiretorch_amd import _lib
from wiretorch_amd.connectome import Connectome, from_dense
from wiretorch_amd.inputs import PoissonInput
from wiretorch_amd.network import Drive, Physiology, Run

#: Physiology the backward pass can differentiate, in ``Physiology`` names.
PHYSIOLOGY = ("theta", "U_reset", "E_L", "C_m", "beta", "E_syn", "decay", "jump", "adapt",
              "adapt_decay", "E_adapt")
BLOCK = 1024
#: Upper limit on trial groups (the kernel takes up to 64); ``geometry`` picks the count.
MAX_GROUPS = 64
XCDS = 8
MAX_TYPES = 256
#: When a list, every ``wt_cond_run`` launch appends a pair of events recorded on its
#: stream just before and after it (``bench.py`` times the kernel with them).
LAUNCH_EVENTS: list | None = None
#: When a dict, each part of a call appends a pair of events recorded on its stream just
#: before and after it, under its name: ``"forward"`` (``wt_cond_run``), ``"backward"``
#: (``wt_cond_scan_backward`` / ``wt_cond_recurrent_backward``) and
#: ``"weight_gradient"`` (the events listing and ``wt_weight_gradient``).
PART_EVENTS: dict | None = None


class _timed:
    """Records a pair of events around a block into ``PART_EVENTS[name]``."""

    def __init__(self, name):
        self.name = name

    def __enter__(self):
        if PART_EVENTS is not None:
            self.start = torch.cuda.Event(enable_timing=True)
            self.start.record()

    def __exit__(self, *exc):
        if PART_EVENTS is not None and exc[0] is None:
            stop = torch.cuda.Event(enable_timing=True)
            stop.record()
            PART_EVENTS.setdefault(self.name, []).append((self.start, stop))
#: When a list, launches run ``wt_cond_run_timed`` and append the per-workgroup phase
#: ticks ``(groups * R, 8)`` (profiling only, forwards without saved tensors,
#: probabilities or tracking; the phases are listed with the entry point).
PHASE_TIMING: list | None = None
#: Phase slots per workgroup that ``wt_cond_run_timed`` writes.
PHASES = 8
#: The forward's per-workgroup event list (entries: 1024, or 2048 where the accumulator
#: leaves room); 0 = chosen per call (``_list_size``). Results do not depend on it; tests
#: set it to exercise both kernels and the rounds.
MAX_LIST = 0
#: Nominal firing rate (Hz) for the list size: the 2048-entry list is taken where a
#: workgroup's trials could list more than 512 fired sources per step at this rate.
_LIST_RATE_HZ = 50.0


def _list_size(B: int, N: int, groups: int, dt_ms: float) -> int:
    """1024 or 2048: the larger list costs registers, so it is taken only where dense
    firing would overflow the smaller one (every workgroup lists the fired sources of
    all its group's trials)."""
    if MAX_LIST:
        return MAX_LIST
    tpg = -(-B // groups)
    expected = tpg * N * _LIST_RATE_HZ * dt_ms / 1000.0
    return 2048 if expected > 512 else 1024


# =====================================================================
# Connectivity as the kernels take it
# =====================================================================


@dataclass
class _Side:
    """A compressed input side on the device, with what the launches derive from it."""

    conn: Connectome
    pathway32: torch.Tensor
    #: For a side built from dense pathways: each source's row within its pathway.
    row_local: torch.Tensor | None = None
    dense_shapes: tuple = ()
    #: the largest per-target sum of |weight| (0-d float64 on the device; 0 when empty)
    max_in_sum: object = 0.0
    #: For a side built from dense pathways: per pathway, its edges (positions in edge
    #: order, a slice where they are consecutive) and their flat indices into the
    #: pathway's (rows, N) weight matrix.
    dense_edges: tuple = ()
    #: the version of ``conn.weights`` the side was built with
    weights_version: int = -1
    _split: dict = field(default_factory=dict)
    _edge_src: torch.Tensor | None = None
    _by_target: dict = field(default_factory=dict)

    def with_weights(self, weights: torch.Tensor) -> "_Side":
        """The same structure with other edge weights; what is derived from the
        structure alone (range splits, edge sources, the by-target order) is shared."""
        c = self.conn
        conn = Connectome(c.n_sources, c.n_targets, c.indptr, c.targets, weights, c.pathway,
                          c.n_pathways)
        side = _Side(conn, self.pathway32, row_local=self.row_local,
                     dense_shapes=self.dense_shapes,
                     dense_edges=self.dense_edges, _split=self._split,
                     _by_target=self._by_target)
        side._edge_src = self.edge_src(torch.cuda.current_stream(c.device).cuda_stream)
        side.max_in_sum = _max_in_sum(conn, self.target_order())
        return side

    @property
    def n_src(self) -> int:
        return self.conn.n_sources

    def split(self, R: int, range_n: int, stream) -> torch.Tensor:
        key = (R, range_n)
        if key not in self._split:
            c = self.conn
            split = torch.zeros((max(c.n_sources, 1), R + 1), dtype=torch.int64, device=c.device)
            if c.n_edges == 0:  # every range of every source is empty: the zeros stand
                self._split[key] = split
                return split
            _lib.check(
                _lib.load().wt_split_ranges(c.indptr.data_ptr(), c.targets.data_ptr(),
                                            c.n_sources, R, range_n, split.data_ptr(), stream),
                "wt_split_ranges",
            )  # fmt: skip
            self._split[key] = split
        return self._split[key]

    def edge_src(self, stream) -> torch.Tensor:
        if self._edge_src is None:
            c = self.conn
            out = torch.empty(c.n_edges, dtype=torch.int64, device=c.device)
            if c.n_edges == 0:
                self._edge_src = out
                return out
            _lib.check(
                _lib.load().wt_edge_sources(c.indptr.data_ptr(), c.n_sources, out.data_ptr(), stream),
                "wt_edge_sources",
            )
            self._edge_src = out
        return self._edge_src

    def by_target(self, N: int, n_pathways: int, stream):
        """``(in_indptr, in_edge)``: the edges grouped by (pathway, target) row
        ``k * N + n``, in source order within a row (edges of no pathway left out)."""
        key = (N, n_pathways)
        if key not in self._by_target:
            c = self.conn
            edge_src = self.edge_src(stream)
            k = c.pathway[edge_src]
            row = torch.where(k >= 0, k * N + c.targets.long(), n_pathways * N)
            in_edge = torch.argsort(row, stable=True)
            counts = torch.bincount(row, minlength=n_pathways * N + 1)[: n_pathways * N]
            in_indptr = torch.zeros(n_pathways * N + 1, dtype=torch.int64, device=c.device)
            in_indptr[1:] = torch.cumsum(counts, 0)
            self._by_target[key] = (in_indptr, in_edge)
        return self._by_target[key]

    def target_order(self):
        """``(indptr, edge)``: every edge grouped by target (for per-target sums)."""
        if "targets" not in self._by_target:
            c = self.conn
            edge = torch.argsort(c.targets, stable=True)
            indptr = torch.zeros(c.n_targets + 1, dtype=torch.int64, device=c.device)
            indptr[1:] = torch.cumsum(torch.bincount(c.targets.long(), minlength=c.n_targets), 0)
            self._by_target["targets"] = (indptr, edge)
        return self._by_target["targets"]

    def abi(self, R: int, range_n: int, stream, weights: torch.Tensor | None = None) -> _lib.Side:
        c = self.conn
        w = c.weights if weights is None else weights
        if w.device != c.indptr.device or w.dtype != torch.float32 or not w.is_contiguous():
            raise ValueError(f"connectome weights on {w.device} ({w.dtype}) for a side on "
                             f"{c.indptr.device}: the kernels take float32 on the side's device")
        return _lib.Side(
            c.indptr.data_ptr(), self.split(R, range_n, stream).data_ptr(),
            c.targets.data_ptr(), w.data_ptr(), self.pathway32.data_ptr(), c.n_sources,
        )  # fmt: skip


def _empty_side(device) -> _Side:
    z = torch.zeros(1, dtype=torch.int64, device=device)
    conn = Connectome(0, 0, z, torch.zeros(1, dtype=torch.int32, device=device),
                      torch.zeros(1, device=device), z, 0)
    return _Side(conn, torch.zeros(1, dtype=torch.int32, device=device))


def _max_in_sum(conn: Connectome, order=None) -> torch.Tensor:
    """The largest per-target sum of |weight|, a 0-d float64 tensor on the connectome's
    device (never read back by the host): by atomic adds, or, given the edges in target
    order (``_Side.target_order``), as differences of a running sum at the targets'
    boundaries (no atomics: a few hundred edges share each target)."""
    if conn.n_edges == 0:
        return torch.zeros((), dtype=torch.float64, device=conn.device)
    w = conn.weights.detach()
    if order is None:
        per_target = torch.zeros(conn.n_targets, dtype=torch.float64, device=conn.device)
        per_target.index_add_(0, conn.targets.long(), w.abs().double())
    else:
        indptr, edge = order
        running = torch.zeros(conn.n_edges + 1, dtype=torch.float64, device=conn.device)
        torch.cumsum(w[edge].abs().double(), 0, out=running[1:])
        per_target = running[indptr[1:]] - running[indptr[:-1]]
    return per_target.max()


def _from_connectome(conn: Connectome, device) -> _Side:
    conn = conn.to(device)
    t = conn.targets
    if conn.n_edges:
        ascending = bool(((t[1:] > t[:-1]) | _row_starts(conn)[1:]).all())
        if not ascending or bool((t < 0).any()) or bool((t >= conn.n_targets).any()):
            raise ValueError("Connectome targets must be in range and strictly ascending per source")
    if conn.n_sources and (int(conn.pathway.max()) >= conn.n_pathways
                           or conn.pathway.numel() != conn.n_sources):
        raise ValueError("Connectome pathway ids must be < n_pathways (or -1)")
    if int(conn.indptr[-1]) != conn.n_edges or conn.indptr.numel() != conn.n_sources + 1:
        raise ValueError("Connectome indptr does not match its edges")
    side = _Side(conn, conn.pathway.to(torch.int32).contiguous())
    side.max_in_sum = _max_in_sum(conn, side.target_order())
    side.weights_version = conn.weights._version
    return side


def _row_starts(conn: Connectome) -> torch.Tensor:
    starts = torch.zeros(conn.n_edges, dtype=torch.bool, device=conn.device)
    first = conn.indptr[:-1][conn.indptr[:-1] < conn.n_edges]
    starts[first] = True
    return starts


def _from_pathways(pathways, n_src: int, N: int, device) -> _Side:
    W_all = torch.zeros((n_src, N), dtype=torch.float32, device=device)
    pathway = torch.full((n_src,), -1, dtype=torch.int64, device=device)
    row_local = torch.full((n_src,), -1, dtype=torch.int64, device=device)
    shapes = []
    for k, (rows, W) in enumerate(pathways):
        rows = rows.to(device).long()
        if bool((pathway[rows] >= 0).any()):
            raise NotImplementedError("pathways sharing source rows (presynaptic dynamics)")
        pathway[rows] = k
        row_local[rows] = torch.arange(rows.numel(), device=device)
        W_all[rows] = W.detach().to(device, torch.float32)
        shapes.append(tuple(W.shape))
    conn = from_dense(W_all, pathway, len(pathways))
    side = _Side(conn, pathway.to(torch.int32), row_local=row_local,
                 dense_shapes=tuple(shapes))
    side.max_in_sum = _max_in_sum(conn, side.target_order())
    none = torch.zeros(0, dtype=torch.int64, device=device)
    edges = [(none, none)] * len(pathways)
    if conn.n_edges:
        edge_src = side.edge_src(torch.cuda.current_stream(device).cuda_stream)
        k_of_edge = conn.pathway[edge_src]
        for k in range(len(pathways)):
            e = torch.nonzero(k_of_edge == k).flatten()
            flat = row_local[edge_src[e]] * N + conn.targets[e].long()
            if e.numel() and int(e[-1]) - int(e[0]) + 1 == e.numel():
                e = slice(int(e[0]), int(e[-1]) + 1)  # a pathway of consecutive sources
            edges[k] = (e, flat)
    side.dense_edges = tuple(edges)
    return side


_CACHE: OrderedDict = OrderedDict()
_CACHE_SIZE = 32
#: Sides of dense pathways by structure (source rows and shapes): a side whose weights
#: changed but whose nonzero pattern did not (learnt weights) takes the new values
#: without being compressed again.
_LAYOUTS: OrderedDict = OrderedDict()
_LAYOUTS_SIZE = 4


def _side_of(pathways, sparse, n_src: int, N: int, device) -> _Side:
    """The compressed side of a drive, cached while its tensors are unchanged. A
    compressed connectome's structure (indptr, targets, pathways) is validated and cached
    once; new edge weights on the same structure (learnt or folded each call) are taken
    without either (``_Side.with_weights``)."""
    if sparse is not None:
        c = sparse
        key = ("sparse",) + _key(c.indptr, c.targets, c.pathway) + (c.n_pathways,)
        hit = _CACHE.get(key)
        if hit is None:
            base = _from_connectome(sparse, device)
            _CACHE[key] = (base, (c.indptr, c.targets, c.pathway))
            while len(_CACHE) > _CACHE_SIZE:
                _CACHE.popitem(last=False)
        else:
            _CACHE.move_to_end(key)
            base = hit[0]
        w = c.weights.to(device)
        if base.conn.weights is w or (base.conn.weights.data_ptr() == w.data_ptr()
                                      and base.weights_version == w._version):
            return base
        side = base.with_weights(w)
        return side
    elif pathways:
        key = ("dense", n_src, N) + tuple(
            (rows.data_ptr(), W.data_ptr(), W._version, tuple(W.shape)) for rows, W in pathways
        )
        keep = tuple(t for pair in pathways for t in pair)
    else:
        return _empty_side(device)
    hit = _CACHE.get(key)
    if hit is not None:
        _CACHE.move_to_end(key)
        return hit[0]
    if sparse is not None:
        side = _from_connectome(sparse, device)
    else:
        side, derived = _dense_side(pathways, n_src, N, device)
        if derived:
            # weights recomputed each call (learnt projections) never come again: caching
            # them by value would only hold their dense matrices
            return side
    _CACHE[key] = (side, keep)  # holding the tensors keeps their addresses unique
    while len(_CACHE) > _CACHE_SIZE:
        _CACHE.popitem(last=False)
    return side


def _dense_side(pathways, n_src: int, N: int, device) -> tuple[_Side, bool]:
    """The side of dense pathways: from the layout of the same structure and nonzero
    pattern if one is cached (the edge weights gathered from the matrices; second item
    True), else compressed anew."""
    key = ("layout", n_src, N) + tuple(
        (rows.data_ptr(), rows._version, tuple(rows.shape), tuple(W.shape))
        for rows, W in pathways)
    hit = _LAYOUTS.get(key)
    if hit is not None:
        base, _keep = hit
        weights = torch.empty_like(base.conn.weights)
        off = []
        for (_, W), (e, flat) in zip(pathways, base.dense_edges):
            W = W.detach().to(device, torch.float32).reshape(-1)
            values = W[flat]
            weights[e] = values
            # the pattern is the layout's when W has as many nonzeros as the layout has
            # edges and is nonzero at each of them (one read of W, no stored mask)
            off.append(torch.count_nonzero(W) - flat.numel())
            off.append(torch.count_nonzero(values == 0))
        if not off or not bool(torch.stack(off).any()):
            _LAYOUTS.move_to_end(key)
            return base.with_weights(weights), True
    side = _from_pathways(pathways, n_src, N, device)
    _LAYOUTS[key] = (side, tuple(rows for rows, _ in pathways))
    while len(_LAYOUTS) > _LAYOUTS_SIZE:
        _LAYOUTS.popitem(last=False)
    return side, False


# =====================================================================
# Many pathways: one per receptor kind
# =====================================================================

#: Pathways the kernels accumulate separately (``WT_MAX_K``); a drive with more is folded.
MAX_PATHWAYS = 8
_GROUP_ROWS: OrderedDict = OrderedDict()


def _group_order(made: torch.Tensor, ks: range) -> list[list[int]]:
    """Pathways ``ks`` grouped by their row of ``made`` (first appearance first); cached
    per ``made`` tensor (reading it back is a host synchronisation)."""

    def make():
        groups: dict[bytes, list[int]] = {}
        rows = made.detach().to("cpu", torch.bool).numpy()
        for k in ks:
            groups.setdefault(rows[k].tobytes(), []).append(k)
        return list(groups.values())

    return _cached(("groups", ks.start, ks.stop) + _key(made), (made,), make)


def fold_pathways(drive: Drive) -> Drive:
    """The drive with its pathways folded into one per (side, synapse types made).

    Pathway ``k`` adds ``a_k ⊗ (jump · scale_k · made_k)`` (``conductance/dynamics.py:
    95-100,206-208``), ``a_k[n] = Σ_j s_j W_k[j, n]``. Pathways that make the same synapse
    types share ``made``, so their sum is ``(Σ_k Σ_j s_j · W_k[j, n] scale_k[n]) ⊗ (jump ·
    made)``: one pathway per group whose weights are ``W_k[j, n] · scale_k[n]`` (a float32
    product) and whose scale is 1. The sum is the same; its rounding is not the
    reference's sequence of per-pathway additions (each group's is exactly rounded, as
    every activation here). Recurrent groups come first, in order of first appearance.
    Differentiable: the folded weights are torch expressions of ``W_k`` and ``scale``."""
    K_rec, K = drive.K_rec, drive.K_rec + drive.K_ff
    sides = (
        (_group_order(drive.made, range(K_rec)), drive.recurrent, drive.sparse_recurrent, 0),
        (_group_order(drive.made, range(K_rec, K)), drive.feedforward, drive.sparse_feedforward,
         K_rec),
    )
    made, out = [], []
    for groups, dense, sparse, k0 in sides:
        made += [drive.made[g[0]] for g in groups]
        if sparse is not None:
            out.append(_fold_sparse(sparse, drive.scale[k0:k0 + sparse.n_pathways], groups, k0))
        else:
            out.append(_fold_dense(dense, drive.scale, groups, k0))
    N = drive.scale.shape[1]
    G = len(made)
    rec, ff = out
    return Drive(
        made=torch.stack(made) if made else drive.made[:0],
        scale=drive.scale.new_ones((G, N)).detach(),
        recurrent=rec if isinstance(rec, list) else [],
        feedforward=ff if isinstance(ff, list) else [],
        differentiable_inputs=drive.differentiable_inputs,
        recurrent_gradients=drive.recurrent_gradients,
        gates=drive.gates,
        sparse_recurrent=None if isinstance(rec, list) else rec,
        sparse_feedforward=None if isinstance(ff, list) else ff,
    )


def _fold_dense(pathways, scale, groups, k0):
    """One dense pathway per group: its members' rows back to back, each row's weights
    times its pathway's scale. The concatenated row indices are cached by the members'
    (so the engine's layout cache sees the same rows tensor each call)."""
    out = []
    for g in groups:
        members = [pathways[k - k0] for k in g]
        key = tuple((rows.data_ptr(), rows._version, rows.numel()) for rows, _ in members)
        rows_g = _GROUP_ROWS.get(key)
        if rows_g is None:
            rows_g = _GROUP_ROWS[key] = (torch.cat([rows.long() for rows, _ in members]),
                                         tuple(rows for rows, _ in members))
            while len(_GROUP_ROWS) > _CACHE_SIZE:
                _GROUP_ROWS.popitem(last=False)
        W_g = torch.cat([W * scale[k][None, :].to(W.dtype) for k, (_, W) in zip(g, members)])
        out.append((rows_g[0], W_g))
    return out


def _fold_sparse(conn: Connectome, scale, groups, k0):
    """The compressed side with each edge's weight times its pathway's scale at its
    target, sources tagged by group."""
    group_of = torch.full((max(conn.n_pathways, 1),), -1, dtype=torch.int64)
    for gi, g in enumerate(groups):
        group_of[[k - k0 for k in g]] = gi
    group_of = group_of.to(conn.device)
    pathway = torch.where(conn.pathway >= 0, group_of[conn.pathway.clamp(min=0)], -1)
    if conn.n_edges:
        counts = conn.indptr[1:] - conn.indptr[:-1]
        src = torch.repeat_interleave(torch.arange(conn.n_sources, device=conn.device), counts)
        k = conn.pathway[src].clamp(min=0)
        weights = conn.weights * scale[k, conn.targets.long()].to(conn.weights.dtype)
    else:
        weights = conn.weights
    return Connectome(conn.n_sources, conn.n_targets, conn.indptr, conn.targets, weights,
                      pathway, len(groups))


# =====================================================================
# One call
# =====================================================================


_DEVICE_INFO: dict = {}


def _device_info(device) -> tuple[int, int]:
    index = device.index if device.index is not None else torch.cuda.current_device()
    if index not in _DEVICE_INFO:
        n_cu, lds = _lib.I64(), _lib.I64()
        with torch.cuda.device(index):
            _lib.check(_lib.load().wt_device_info(n_cu, lds), "wt_device_info")
        _DEVICE_INFO[index] = (int(n_cu.value), int(lds.value))
    return _DEVICE_INFO[index]


def geometry(B: int, N: int, K: int, n_cu: int, max_lds: int) -> tuple[int, int, int]:
    """``(groups, R, range_n)``: trials round-robin over groups, each group's targets
    split over R workgroups (range_n a multiple of 32), about one (trial, neuron) item per
    thread and at most 8 per thread (they live in registers), within the LDS budget of
    the int64 accumulator ``K * trials * range_n`` and the fired bitmap.

    As many groups as fit, one trial each where the batch allows: every workgroup lists
    and looks up the fired sources of all its group's trials, and waits for its group's
    R arrivals each step, so fewer trials per group mean less of both for the same
    targets. Past 8, groups come in multiples of 8: workgroup i is in group i % groups
    and on XCD i % 8, so a group's workgroups share one XCD (and its L2)."""
    budget = max_lds - 54 * 1024  # static: event lists, type tables, own bits

    def plan(groups):
        tpg = -(-B // groups)
        limit = max(1, n_cu // groups)

        def fits(R):
            range_n = -(-(-(-N // R)) // 32) * 32
            lds = max(K, 1) * tpg * range_n * 8
            return lds <= budget and tpg * range_n <= 8 * BLOCK, range_n

        R = max(1, min(limit, -(-N * tpg // BLOCK)))
        ok, range_n = fits(R)
        while not ok and R < limit:
            R += 1
            ok, range_n = fits(R)
        return (groups, -(-N // range_n), range_n) if ok else None

    groups = max(1, min(MAX_GROUPS, B))
    while True:
        if groups > XCDS:
            groups -= groups % XCDS
        found = plan(groups)
        if found is not None:
            return found
        if groups == 1:
            raise ValueError(f"network too large for one launch (N {N}, batch {B}, {K} pathways)")
        groups = groups // 2  # more workgroups per group for a larger network


def _device_scalar(value, device) -> torch.Tensor:
    """A 0-d float64 tensor on ``device`` (a bound computed there, or a host zero)."""
    if isinstance(value, torch.Tensor):
        return value
    return _cached(("zero", str(device)), (), lambda: torch.zeros((), dtype=torch.float64,
                                                                   device=device))


def _classes(type_of: torch.Tensor):
    """Each neuron's class numbered from 0 in order of value, and each class's first
    neuron (computed once per class tensor)."""
    _, inv = torch.unique(type_of, return_inverse=True)
    n = int(inv.max()) + 1 if inv.numel() else 0
    first = torch.full((n,), inv.numel(), dtype=torch.int64, device=inv.device)
    first.scatter_reduce_(0, inv, torch.arange(inv.numel(), device=inv.device), "amin")
    return inv, first


def _type_table(tables: dict, scale: torch.Tensor, device, type_of=None):
    """The per-neuron values the forward reads — theta, U_reset, E_L, C_m, beta, n_ref
    and each pathway's kernel scale — as rows of distinct values and each neuron's row:
    networks built from cell types have few, which the kernel keeps in LDS. With
    ``type_of`` (classes within which the rows are equal: ``Physiology.type_of``) of at
    most ``MAX_TYPES`` classes, one row per class, taken from its first neuron; every
    neuron's row is compared with its class's on the device and a difference reported as
    a launch error. (More classes than one table holds are searched for their distinct
    rows as without ``type_of``: classes often share a row.)"""
    N = tables["theta"].shape[0]
    n_ref = (tables["n_ref"].float() if tables["n_ref"] is not None
             else torch.zeros(N, device=device))
    cols = [tables[n] for n in ("theta", "U_reset", "E_L", "C_m", "beta")] + [n_ref]
    rows = torch.cat([torch.stack(cols, dim=1), _f32(scale, device).T], dim=1)
    if type_of is not None:
        cls = type_of.detach().to(device)
        inv, first = _cached(("classes",) + _key(cls), (cls,), lambda: _classes(cls))
        if first.numel() > MAX_TYPES:  # more classes than one table: search (fewer rows)
            type_of = None
    if type_of is None:
        types, type_of = torch.unique(rows, dim=0, return_inverse=True)
        return types.contiguous(), type_of.to(torch.int32).contiguous()
    types = rows[first].contiguous()
    differs = (rows != types[inv]).any().to(torch.int32) * TABLE_MISMATCH
    _watch(differs.reshape(1))
    return types, inv.to(torch.int32).contiguous()


def _range_types(type_of: torch.Tensor, n_rows: int, range_n: int):
    """The rows each workgroup stages in LDS. With at most ``MAX_TYPES`` distinct rows,
    all of them: ``(type_of, None, n_rows)``. Otherwise per target range of ``range_n``
    neurons its own rows (at most ``MAX_TYPES``: networks whose neurons are grouped by
    cell type meet this with thousands of types): ``(local, range_rows, n_local)``, where
    ``range_rows[r, j]`` is the j-th row of range r (rows ascending, the rest padded with
    row 0), ``local[n]`` the index of neuron n's row there and ``n_local`` the largest
    count."""
    if n_rows <= MAX_TYPES:
        return type_of, None, n_rows
    N = type_of.numel()
    n_ranges = -(-N // range_n)
    rng = torch.arange(N, device=type_of.device) // range_n
    keys, inv = torch.unique(rng * n_rows + type_of.long(), return_inverse=True)
    key_range = keys // n_rows
    counts = torch.bincount(key_range, minlength=n_ranges)
    most = int(counts.max())
    if most > MAX_TYPES:
        raise NotImplementedError(
            f"a range of {range_n} neurons holds {most} distinct per-neuron parameter rows "
            f"(at most {MAX_TYPES}: physiology and kernel scales are expected to follow cell "
            "types, with the neurons of a type next to each other)")
    first = torch.cumsum(counts, 0) - counts  # each range's first key
    local = (inv - first[rng]).to(torch.int32).contiguous()
    range_rows = torch.zeros((n_ranges, MAX_TYPES), dtype=torch.int32, device=type_of.device)
    j = torch.arange(keys.numel(), device=type_of.device) - first[key_range]
    range_rows[key_range, j] = (keys % n_rows).to(torch.int32)
    return local, range_rows, most


def _key(*tensors) -> tuple:
    """Identity of tensors' current contents: address, version and shape."""
    return tuple((t.data_ptr(), t._version, tuple(t.shape), t.dtype) if t is not None else None
                 for t in tensors)


def _cached(key: tuple, keep: tuple, make):
    """``make()``, cached under ``key`` while the tensors in ``keep`` are unchanged
    (holding them keeps their addresses from being reused)."""
    hit = _CACHE.get(key)
    if hit is not None:
        _CACHE.move_to_end(key)
        return hit[0]
    value = make()
    _CACHE[key] = (value, keep)
    while len(_CACHE) > _CACHE_SIZE:
        _CACHE.popitem(last=False)
    return value


def _f32(t: torch.Tensor, device) -> torch.Tensor:
    return t.detach().to(device=device, dtype=torch.float32).contiguous()


@dataclass
class _Plan:
    """Shapes, tables and connectivity shared by the forward and backward launches."""

    B: int
    T: int
    N: int
    S: int
    K_rec: int
    K_ff: int
    n_in: int
    tables: dict
    rec: _Side
    ff: _Side
    geo: tuple
    #: (type_of, range_rows or None, n_types) of ``_range_types`` for this geometry
    range_types: tuple
    #: 0-d float64 device tensor: the largest |activation| (the kernel's fixed point)
    bound: torch.Tensor
    max_list: int
    refractory: bool
    #: spike-frequency adaptation (the physiology's adapt is set)
    adapting: bool
    probabilities: bool
    track: bool
    track_b: int
    stream: int
    device: torch.device
    #: gradients flow back through the recurrent spikes (set by ``simulate``)
    recurrent_gradients: bool = False
    #: on-device Poisson input in place of the input tensor (set by ``simulate``)
    poisson: PoissonInput | None = None

    @property
    def K(self) -> int:
        return self.K_rec + self.K_ff

    def abi_geometry(self) -> _lib.Geometry:
        groups, R, range_n = self.geo
        return _lib.Geometry(groups, R, range_n, -1, self.max_list, self.bound.data_ptr())

    def abi_tables(self, scale: torch.Tensor) -> _lib.Tables:
        if scale.device != self.device or scale.dtype != torch.float32 or not scale.is_contiguous():
            raise ValueError(f"kernel scales on {scale.device} ({scale.dtype}): the kernels take "
                             f"float32 on {self.device}")
        t = self.tables
        type_of, range_rows, n_types = self.range_types
        return _lib.Tables(
            t["theta"].data_ptr(), t["U_reset"].data_ptr(), t["E_L"].data_ptr(),
            t["C_m"].data_ptr(), t["beta"].data_ptr(),
            t["n_ref"].data_ptr() if t["n_ref"] is not None else None,
            t["E_syn"].data_ptr(), t["g_clip"].data_ptr(), t["decay"].data_ptr(),
            t["jump"].data_ptr(), t["made"].data_ptr(), scale.data_ptr(),
            t["dt"].data_ptr(), t["surr"].data_ptr(), t["types"].data_ptr(),
            type_of.data_ptr(), n_types, _lib.ptr(range_rows), _lib.ptr(t["mg_a"]),
            _lib.ptr(t["mg_lc"]), _lib.ptr(t["adapt"]), _lib.ptr(t["adapt_decay"]),
            _lib.ptr(t["E_adapt"]), self.N, self.S, self.K, self.K_rec,
        )  # fmt: skip


def _plan(v, x, drive: Drive, p: Physiology, probabilities, track, track_batch_idx) -> _Plan:
    device = x.device
    B, T, n_in = x.shape
    N = v.shape[1]
    S = p.E_syn.shape[0]
    if S > 8:
        raise NotImplementedError(f"at most 8 synapse types, got {S}")
    K_rec, K_ff = drive.K_rec, drive.K_ff
    if K_rec + K_ff > MAX_PATHWAYS:
        raise NotImplementedError(
            f"{K_rec + K_ff} pathways make more than {MAX_PATHWAYS} distinct (side, synapse "
            "types) combinations")
    if drive.made.shape != (K_rec + K_ff, S) or drive.scale.shape != (K_rec + K_ff, N):
        raise ValueError("drive.made / drive.scale do not match the pathways")
    rec = _side_of(drive.recurrent, drive.sparse_recurrent, N, N, device)
    ff = _side_of(drive.feedforward, drive.sparse_feedforward, n_in, N, device)
    if rec.n_src and rec.conn.n_targets != N:
        raise ValueError("recurrent connectome does not match the network size")
    if ff.n_src and (ff.n_src != n_in or ff.conn.n_targets != N):
        raise ValueError("feedforward connectome does not match the input and network")
    n_cu, max_lds = _device_info(device)
    groups, R, range_n = geometry(B, N, K_rec + K_ff, n_cu, max_lds)
    dt_ms = _cached(("dt",) + _key(p.dt), (p.dt,), lambda: float(p.dt))
    max_list = _list_size(B, N, groups, dt_ms)
    # the accumulators' bound stays on the device: the kernel derives its fractional bits
    bound = _device_scalar(rec.max_in_sum, device)
    if ff.n_src and ff.conn.n_edges:
        if isinstance(x, PoissonInput):  # spikes: at most 1
            x_max = _cached(("one", str(device)), (),
                            lambda: torch.ones((), dtype=torch.float64, device=device))
        else:
            xd = x.detach()
            x_max = _cached(("x_max",) + _key(xd), (xd,), lambda: xd.abs().max().double())
        ff_max = _device_scalar(ff.max_in_sum, device)
        bound = _cached(("bound",) + _key(bound, ff_max, x_max), (bound, ff_max, x_max),
                        lambda: bound + ff_max * x_max)
    names = ("theta", "U_reset", "E_L", "C_m", "beta", "E_syn", "g_clip", "decay", "jump")
    sources = tuple(getattr(p, name) for name in names) + (
        drive.made, drive.scale, p.dt, p.surr_scale, p.n_ref, p.mg_c, p.mg_a, p.adapt,
        p.adapt_decay, p.E_adapt, p.type_of)

    def make_tables():
        tables = {name: _f32(getattr(p, name), device) for name in names}
        tables["made"] = drive.made.to(device=device, dtype=torch.float32).contiguous()
        tables["dt"] = _f32(p.dt, device)
        tables["surr"] = _f32(p.surr_scale, device)
        tables["n_ref"] = (None if p.n_ref is None
                           else p.n_ref.to(device=device, dtype=torch.int32).contiguous())
        tables["types"], tables["type_of"] = _type_table(tables, drive.scale, device,
                                                         p.type_of)
        if p.mg_c is not None:  # the Mg block: log(mg_c) taken by torch on the CPU, as
            # the reference's CPU path takes it (-inf for a type without a block)
            tables["mg_a"] = _f32(p.mg_a, device)
            tables["mg_lc"] = torch.log(p.mg_c.detach().cpu().float()).to(device)
        else:
            tables["mg_a"] = tables["mg_lc"] = None
        for name in ("adapt", "adapt_decay", "E_adapt"):  # per neuron, when adapting
            tables[name] = _f32(getattr(p, name), device) if p.adapt is not None else None
        return tables

    # the tables (and the distinct-row search) are rebuilt only when a source changes
    tables = _cached(("tables", str(device)) + _key(*sources), sources, make_tables)
    types, type_of = tables["types"], tables["type_of"]
    range_types = _cached(("range_types", range_n) + _key(types, type_of), (types, type_of),
                          lambda: _range_types(type_of, int(types.shape[0]), range_n))
    return _Plan(
        B=B, T=T, N=N, S=S, K_rec=K_rec, K_ff=K_ff, n_in=n_in, tables=tables, rec=rec,
        ff=ff, geo=(groups, R, range_n), range_types=range_types, bound=bound,
        max_list=max_list,
        refractory=p.n_ref is not None, adapting=p.adapt is not None,
        probabilities=probabilities, track=track,
        track_b=(-1 if track_batch_idx is None else int(track_batch_idx)) if track else 0,
        stream=torch.cuda.current_stream(device).cuda_stream, device=device,
    )  # fmt: skip


def _launch(L: _Plan, x, scale, v, g, counter, spikes, prob, saved, tracked,
            rec_weights=None, ff_weights=None, adaptation=None, a_saved=None) -> None:
    groups, R, range_n = L.geo
    geo = L.abi_geometry()
    lib = _lib.load()
    scratch = torch.empty(int(lib.wt_cond_run_scratch_bytes(geo, L.B, L.T)),
                          dtype=torch.uint8, device=L.device)
    scratch[: int(lib.wt_cond_run_scratch_zeroed(geo))].zero_()
    v_saved, G_saved, held, A_saved = saved if saved is not None else (None,) * 4
    tv, tI, tg = ((tracked["v"], tracked["I"], tracked["g"]) if tracked is not None
                  else (None, None, None))
    ta = tracked.get("a") if tracked is not None else None
    if L.adapting and (adaptation is None or adaptation.shape != (L.B, L.N)
                       or adaptation.dtype != torch.float32 or not adaptation.is_contiguous()
                       or adaptation.device != L.device):
        raise ValueError(f"an adapting network needs its (B, N) float32 adaptation state on "
                         f"{L.device}")
    pin = L.poisson
    io = _lib.RunIO(
        None if pin is not None else x.data_ptr(), L.B, L.T, L.n_in, v.data_ptr(),
        g.data_ptr(), _lib.ptr(counter) if L.refractory else None, spikes.data_ptr(),
        _lib.ptr(prob), _lib.ptr(v_saved), _lib.ptr(G_saved), _lib.ptr(held),
        _lib.ptr(A_saved), _lib.ptr(tv), _lib.ptr(tI), _lib.ptr(tg), L.track_b,
        pin.prob.data_ptr() if pin is not None else None, pin.seed if pin is not None else 0,
        pin.t0 if pin is not None else 0,
        _lib.ptr(adaptation) if L.adapting else None, _lib.ptr(a_saved) if L.adapting else None,
        _lib.ptr(ta) if L.adapting else None,
    )  # fmt: skip
    rec = L.rec.abi(R, range_n, L.stream, rec_weights)
    ff = L.ff.abi(R, range_n, L.stream, ff_weights)
    tab = L.abi_tables(scale)
    if LAUNCH_EVENTS is not None:
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
    if PHASE_TIMING is not None:
        if prob is not None or saved is not None or tracked is not None:
            raise NotImplementedError("phase timing times forwards without saved tensors, "
                                      "probabilities or tracking")
        ticks = torch.zeros((groups * R, PHASES), dtype=torch.int64, device=L.device)
        _lib.check(lib.wt_cond_run_timed(tab, rec, ff, geo, io, scratch.data_ptr(),
                                         ticks.data_ptr(), L.stream), "wt_cond_run_timed")
        PHASE_TIMING.append(ticks)
    else:
        with _timed("forward"):
            _lib.check(lib.wt_cond_run(tab, rec, ff, geo, io, scratch.data_ptr(), L.stream),
                       "wt_cond_run")
    if LAUNCH_EVENTS is not None:
        stop.record()
        LAUNCH_EVENTS.append((start, stop))
    _watch(scratch[:4].view(torch.int32))


#: Error words of launches not yet checked: (event after the copy, pinned host word).
_PENDING: list = []
#: The error bit of a type table whose rows differ within a class (the kernels' error
#: words use the low bits).
TABLE_MISMATCH = 1 << 30


def _watch(word: torch.Tensor) -> None:
    """Copy a launch's error word to pinned host memory without waiting for it; it is
    checked once the copy has landed (``check_errors``, run at the start of every call
    and of every backward), so the host never stalls on the GPU here."""
    host = torch.empty(1, dtype=torch.int32, pin_memory=True)
    host.copy_(word, non_blocking=True)
    done = torch.cuda.Event()
    done.record()
    _PENDING.append((done, host))


def check_errors(wait: bool = False) -> None:
    """Raise if an earlier launch reported an error (a group barrier that timed out, or
    per-neuron tables that differ within a class of ``Physiology.type_of``): checks every
    launch whose error word has reached the host (with ``wait``, waits for all of
    them)."""
    still = []
    failed = 0
    for done, host in _PENDING:
        if wait:
            done.synchronize()
        elif not done.query():
            still.append((done, host))
            continue
        failed |= int(host[0])
    _PENDING[:] = still
    if failed & TABLE_MISMATCH:
        raise RuntimeError("Physiology.type_of: per-neuron tables or kernel scales differ "
                           "within a class; that call's results used each class's first "
                           "neuron's values")
    if failed:
        raise RuntimeError(f"wt_cond_run: a workgroup barrier timed out (flags {failed:#x})")


# =====================================================================
# Autograd
# =====================================================================


class _Run(torch.autograd.Function):
    """Spikes (and probabilities) of a chunk, differentiable in the kernel ``scale``,
    the input ``x``, the pathway weights and the physiology (``PHYSIOLOGY``)."""

    @staticmethod
    def forward(ctx, L: _Plan, n_rec_w: int, scale, x, v, g, counter, adaptation, *rest):
        weights, physiology = rest[: len(rest) - len(PHYSIOLOGY)], rest[-len(PHYSIOLOGY):]
        dev = L.device
        spikes = torch.empty((L.B, L.T, L.N), device=dev)
        prob = torch.empty_like(spikes) if L.probabilities else None
        v_saved = torch.empty_like(spikes)
        G_saved = torch.empty((L.B, L.T, L.N, L.S), device=dev)
        held = torch.empty((L.B, L.T, L.N), dtype=torch.int8, device=dev) if L.refractory else None
        A_saved = torch.empty((max(L.K, 1), L.B, L.T, L.N), device=dev)
        a_saved = torch.empty_like(spikes) if L.adapting else spikes.new_empty(0)
        want_decay = physiology[PHYSIOLOGY.index("decay")].requires_grad
        g_init = g.clone() if want_decay else None
        tracked = _tracked_buffers(L)
        _launch(L, x.detach().float().contiguous(), scale.detach().float().contiguous(), v, g,
                counter, spikes, prob, (v_saved, G_saved, held, A_saved), tracked,
                *_sparse_weights(L, weights, n_rec_w), adaptation=adaptation, a_saved=a_saved)
        ctx.L, ctx.n_rec_w, ctx.tracked = L, n_rec_w, tracked
        ctx.save_for_backward(scale, x, spikes, v_saved, G_saved,
                              held if held is not None else spikes.new_empty(0),
                              A_saved, g_init if g_init is not None else spikes.new_empty(0),
                              a_saved, *weights)
        ctx.mark_non_differentiable(v, g, counter, adaptation)
        return spikes, prob, v, g, counter, adaptation

    @staticmethod
    def backward(ctx, grad_spikes, grad_prob, _v, _g, _c, _a):
        check_errors(wait=True)  # the forward this backward differentiates is complete
        L, n_rec_w = ctx.L, ctx.n_rec_w
        (scale, x, spikes, v_saved, G_saved, held, A_saved, g_init, a_saved,
         *weights) = ctx.saved_tensors
        needs = ctx.needs_input_grad
        want_scale, want_x = needs[2], needs[3]
        w_needs = needs[8: 8 + len(weights)]
        p_needs = needs[8 + len(weights):]
        if grad_spikes is None:
            grad_spikes = torch.zeros_like(spikes)
        want_A = want_x or any(w_needs)
        dev = L.device
        B, T, N, S, K = L.B, L.T, L.N, L.S, L.K
        # Only the weight gradients want dL/da: the scan backward writes it directly as
        # the (pathway, target) rows they read, each trial's steps padded to 16
        T_pad = -(-T // 16) * 16
        as_rows = want_A and not want_x and not L.recurrent_gradients and K >= 1
        grad_A = (torch.empty((max(K, 1), B, T, N), device=dev) if want_A and not as_rows
                  else None)
        rows = (torch.empty((K * N, B * T_pad), device=dev), T_pad) if as_rows else None
        partial = torch.empty((max(K, 1), B, N), device=dev) if want_scale else None
        shapes = [(B, N)] * 5 + [(B, S, N), (B, 2, S, N), (B, 2, S, N)] + [(B, N)] * 3
        phys = [torch.empty(sh, device=dev) if want else None for sh, want in zip(shapes, p_needs)]
        io = _lib.BackwardIO(
            grad_spikes.contiguous().data_ptr(),
            _lib.ptr(grad_prob.contiguous()) if grad_prob is not None else None,
            spikes.data_ptr(), v_saved.data_ptr(), G_saved.data_ptr(),
            held.data_ptr() if L.refractory else None, A_saved.data_ptr(),
            g_init.data_ptr() if g_init.numel() else None, B, T,
            _lib.ptr(grad_A), _lib.ptr(partial), *[_lib.ptr(t) for t in phys[:8]],
            a_saved.data_ptr() if L.adapting else None, *[_lib.ptr(t) for t in phys[8:]],
            rows[0].data_ptr() if rows else None, T_pad if rows else 0,
        )  # fmt: skip
        tab = L.abi_tables(scale.detach().float().contiguous())
        lib = _lib.load()
        # the weight gradients' event lists are counted first: the host waits for their
        # totals while the backward kernel runs
        rec_counted = ff_counted = activity = None
        if any(w_needs[:n_rec_w]):
            rec_counted = _count_events(spikes, L.stream)
        if any(w_needs[n_rec_w:]):
            activity = (L.poisson.materialize(L.stream) if L.poisson is not None
                        else x.detach().float())
            ff_counted = _count_events(activity, L.stream)
        if L.recurrent_gradients:  # through the recurrent spikes: per-step coupling
            groups, R, range_n = L.geo
            rec_w = _sparse_weights(L, weights, n_rec_w)[0]
            rec = L.rec.abi(R, range_n, L.stream, rec_w)
            scratch = torch.empty(int(lib.wt_cond_recurrent_backward_scratch_bytes(S, L.K_rec, B, N)),
                                  dtype=torch.uint8, device=dev)
            with _timed("backward"):
                _lib.check(lib.wt_cond_recurrent_backward(tab, rec, io, scratch.data_ptr(),
                                                          L.stream), "wt_cond_recurrent_backward")
        else:
            with _timed("backward"):
                _lib.check(lib.wt_cond_scan_backward(tab, io, L.stream), "wt_cond_scan_backward")
        grad_scale = partial.sum(dim=1) if want_scale else None
        dims = [0] * 5 + [(0, 2), (0, 3), (0, 3)] + [0] * 3
        grad_phys = [t.sum(d) if t is not None else None for t, d in zip(phys, dims)]
        grad_w = [None] * len(weights)
        with _timed("weight_gradient"):
            if rec_counted is not None:
                grad_w[:n_rec_w] = _weight_grads(L, L.rec, spikes, grad_A, 0,
                                                 weights[:n_rec_w], w_needs[:n_rec_w],
                                                 rec_counted, spikes=True, rows=rows)
            if ff_counted is not None:
                grad_w[n_rec_w:] = _weight_grads(L, L.ff, activity, grad_A, L.K_rec,
                                                 weights[n_rec_w:], w_needs[n_rec_w:],
                                                 ff_counted, spikes=L.poisson is not None,
                                                 rows=rows)
        grad_x = _input_grad(L, x, grad_A, weights[n_rec_w:]) if want_x else None
        return (None, None, grad_scale, grad_x, None, None, None, None, *grad_w, *grad_phys)


def _tracked_buffers(L: _Plan):
    if not L.track:
        return None
    Bt = L.B if L.track_b < 0 else 1
    dev = L.device
    tracked = {
        "v": torch.empty((Bt, L.T, L.N), device=dev),
        "I": torch.empty((Bt, L.T, L.N, L.S + 1), device=dev),
        "g": torch.empty((Bt, L.T, L.N, 2, L.S), device=dev),
    }
    if L.adapting:
        tracked["a"] = torch.empty((Bt, L.T, L.N), device=dev)
    return tracked


def _sparse_weights(L: _Plan, weights, n_rec_w):
    """Weight tensors the kernels read directly (a compressed side's ``weights``)."""
    rec = ff = None
    if L.rec.row_local is None and n_rec_w == 1:
        rec = weights[0].detach().float().contiguous()
    if L.ff.row_local is None and len(weights) - n_rec_w == 1:
        ff = weights[n_rec_w].detach().float().contiguous()
    return rec, ff


def _count_events(activity: torch.Tensor, stream):
    """The first half of ``_events``: the per-source counts (``wt_events_count``) and
    their total, copied to pinned host memory behind an event — so that the host can
    queue more work (the backward kernel) before it waits for the total."""
    B, T, n = activity.shape
    BT = B * T
    flat = activity.reshape(BT, n).float().contiguous()
    dev = activity.device
    lib = _lib.load()
    scratch = torch.empty(max(int(lib.wt_events_scratch_bytes(BT, n)), 1), dtype=torch.uint8,
                          device=dev)
    indptr = torch.empty(n + 1, dtype=torch.int64, device=dev)
    _lib.check(lib.wt_events_count(flat.data_ptr(), BT, n, scratch.data_ptr(),
                                   indptr.data_ptr(), stream), "wt_events_count")
    total = torch.empty(1, dtype=torch.int64, pin_memory=True)
    total.copy_(indptr[n:], non_blocking=True)
    counted = torch.cuda.Event()
    counted.record(torch.cuda.current_stream(dev))
    return flat, scratch, indptr, total, counted


def _events(activity: torch.Tensor, stream, counted=None, values=True, T_pad=None):
    """Per source, its (trial*T_pad + step) events ascending (int32; ``T_pad`` = T unless
    given) and their values: ``(indptr, bt, value)`` from ``activity`` ``(B, T, n_src)``
    (``wt_events_count`` / ``wt_events_fill``; the host reads the number of events to size
    the lists). ``counted``: what ``_count_events`` returned for this activity, if it ran
    already; without ``values`` (an activity of spikes, 0 or 1) ``value`` is None."""
    T = activity.shape[1]
    flat, scratch, indptr, total, done = counted or _count_events(activity, stream)
    BT, n = flat.shape
    dev = activity.device
    lib = _lib.load()
    done.synchronize()
    total = int(total[0])
    bt = torch.empty(total, dtype=torch.int32, device=dev)
    value = torch.empty(total, dtype=torch.float32, device=dev) if values else None
    if total:
        _lib.check(lib.wt_events_fill(flat.data_ptr(), BT, n, scratch.data_ptr(),
                                      indptr.data_ptr(), bt.data_ptr(), _lib.ptr(value), T,
                                      T_pad or T, stream), "wt_events_fill")
    return indptr, bt, value


def _weight_grads(L: _Plan, side: _Side, activity, grad_A, k0, weights, needs, counted=None,
                  spikes=False, rows=None):
    """Gradients of a side's weight tensors from the event-driven support gradient:
    ``wt_weight_gradient_by_target`` over dL/da as (pathway, target) rows — ``rows``
    ``(all rows, T_pad)`` as the scan backward wrote them, else transposed from
    ``grad_A``. ``spikes``: the activity is 0 or 1 (its events carry no values)."""
    c = side.conn
    indptr, bt, value = _events(activity, L.stream, counted, values=not spikes,
                                T_pad=rows[1] if rows else None)
    grad_e = torch.zeros(c.n_edges, device=L.device)
    edge_src = side.edge_src(L.stream)
    n_path = int(c.n_pathways)
    if c.n_edges and n_path:
        in_indptr, in_edge = side.by_target(L.N, n_path, L.stream)
        if rows is not None:  # the rows of this side's pathways, as written
            BT = L.B * rows[1]
            side_rows, gA = rows[0][k0 * L.N: (k0 + n_path) * L.N], None
        else:
            BT = L.B * L.T
            side_rows = torch.empty((n_path * L.N, BT), device=L.device)
            gA = grad_A[k0: k0 + n_path]
        _lib.check(
            _lib.load().wt_weight_gradient_by_target(
                edge_src.data_ptr(), c.n_edges, in_indptr.data_ptr(), in_edge.data_ptr(),
                n_path, L.N, indptr.data_ptr(), bt.data_ptr(), _lib.ptr(value),
                _lib.ptr(gA), BT, side_rows.data_ptr(), grad_e.data_ptr(), L.stream),
            "wt_weight_gradient_by_target",
        )  # fmt: skip
    if side.row_local is None:  # compressed side: the gradient of its weights
        return [grad_e if needs[0] else None]
    out = []
    for k, (shape, need) in enumerate(zip(side.dense_shapes, needs)):
        if not need:
            out.append(None)
            continue
        G = torch.zeros(shape, device=L.device)
        if side.dense_edges:
            e, flat = side.dense_edges[k]
            G.view(-1)[flat] = grad_e[e]
        out.append(G)
    return out


def _input_grad(L: _Plan, x, grad_A, ff_weights):
    """dL/dx of the feedforward input: each pathway's dL/da carried back through W^T."""
    grad_x = torch.zeros_like(x, dtype=torch.float32)
    side = L.ff
    if side.row_local is None or not side.n_src:
        raise NotImplementedError("input gradients through a compressed feedforward side")
    pathway = side.conn.pathway
    for k, W in enumerate(ff_weights):
        rows = torch.nonzero(pathway == k).flatten()
        order = torch.argsort(side.row_local[rows])
        rows = rows[order]
        grad_x[:, :, rows] += grad_A[L.K_rec + k] @ W.detach().float().T
    return grad_x.to(x.dtype)


# =====================================================================
# Entry point
# =====================================================================


def simulate(
    v, g, x, drive: Drive, p: Physiology, *, refractory=None, gating=None,
    adaptation=None, probabilities=False, track=False, track_batch_idx=None, retain=None,
) -> Run:  # fmt: skip
    """Simulate ``x.shape[1]`` steps from ``(v, g)`` on the GPU; see the module docstring."""
    if not x.is_cuda:
        raise RuntimeError(f"the HIP engine runs on a GPU; the input is on {x.device}")
    check_errors()
    if retain is not None:
        raise NotImplementedError("per-step gradient retention (track_gradients)")
    gates = list(drive.gates or [])
    if any(gate is not None for gate in gates[: drive.K_rec]):
        raise NotImplementedError("presynaptic dynamics on recurrent pathways")
    if any(gate is not None for gate in gates):
        if gating is None:
            raise ValueError("a drive with presynaptic dynamics needs the gating state")
        x, drive, gating = _gate_inputs(drive, x, gating)
        run = simulate(v, g, x, drive, p, refractory=refractory, adaptation=adaptation,
                       probabilities=probabilities, track=track,
                       track_batch_idx=track_batch_idx)
        run.gating = gating
        return run
    if p.spike_mode != "deterministic":
        raise NotImplementedError("sampled spikes")
    if p.storage_dtype != torch.float32:
        raise NotImplementedError("float16 storage")
    device = x.device
    if drive.K_rec + drive.K_ff > MAX_PATHWAYS:
        drive = fold_pathways(drive)
    L = _plan(v, x, drive, p, probabilities, track, track_batch_idx)
    if isinstance(x, PoissonInput):  # drawn inside the forward; the tensor is a stand-in
        L.poisson = x
        x = torch.empty((0,), device=device)
    # The kernel updates the state in place: always work on copies, so the caller's
    # tensors keep their values (a permuted view may already be contiguous storage).
    v = v.detach().to(device=device, dtype=torch.float32).clone(
        memory_format=torch.contiguous_format)
    g_state = g.detach().to(device=device, dtype=torch.float32).permute(0, 2, 3, 1).clone(
        memory_format=torch.contiguous_format)
    if refractory is None:
        refractory = torch.zeros(v.shape, dtype=torch.int32, device=device)
    counter = refractory.to(device=device, dtype=torch.int32).clone(
        memory_format=torch.contiguous_format)
    # the adaptation conductances (updated in place, like the state); none without it
    if not L.adapting:
        adaptation = torch.empty((0,), device=device)
    elif adaptation is None:
        adaptation = torch.zeros(v.shape, device=device)
    else:
        adaptation = adaptation.detach().to(device=device, dtype=torch.float32).clone(
            memory_format=torch.contiguous_format)

    # a compressed side's weights are read by the kernels themselves: on the launch device
    # (a differentiable copy where they were built elsewhere)
    rec_w = ([drive.sparse_recurrent.weights.to(device)] if drive.sparse_recurrent is not None
             else [W for _, W in drive.recurrent])
    ff_w = ([drive.sparse_feedforward.weights.to(device)]
            if drive.sparse_feedforward is not None else [W for _, W in drive.feedforward])
    physiology = [getattr(p, name) for name in PHYSIOLOGY]
    scale = drive.scale.to(device)  # the kernels read it: on the launch device
    grad = torch.is_grad_enabled() and (
        scale.requires_grad or x.requires_grad
        or any(W.requires_grad for W in rec_w + ff_w)
        or any(t is not None and t.requires_grad for t in physiology)
    )  # fmt: skip
    L.recurrent_gradients = bool(drive.recurrent_gradients and L.K_rec and L.rec.n_src)
    if grad:
        spikes, prob, v, g_state, counter, adaptation = _Run.apply(
            L, len(rec_w), scale, x, v, g_state, counter, adaptation, *rec_w, *ff_w,
            *physiology
        )
        tracked = None
        if track:  # the buffers live on the autograd context; rebuild from the last run
            tracked = _last_tracked(spikes)
    else:
        spikes = torch.empty((L.B, L.T, L.N), device=device)
        prob = torch.empty_like(spikes) if probabilities else None
        tracked = _tracked_buffers(L)
        with torch.no_grad():
            rw, fw = _sparse_weights(L, rec_w + ff_w, len(rec_w))
            _launch(L, x.detach().float().contiguous(),
                    scale.detach().float().contiguous(), v, g_state, counter, spikes,
                    prob, None, tracked, rw, fw, adaptation=adaptation)
    return Run(
        output=spikes,
        v=v,
        syn=g_state.permute(0, 3, 1, 2),
        probabilities=prob,
        tracked=tracked,
        refractory=counter,
        gating=gating,
        adaptation=adaptation if L.adapting else None,
    )


def _gated_rows(rows_list, n_in: int, device):
    """Each feedforward pathway's rows as a block of input columns of its own (pathway k:
    columns off_k .. off_k + n_k - 1), after checking the rows against the input width
    once per rows tensor (a host read)."""
    out, off = [], 0
    for rows in rows_list:
        rows = rows.to(device).long()
        if rows.numel() and (int(rows.min()) < 0 or int(rows.max()) >= n_in):
            raise ValueError(f"feedforward rows outside the {n_in} input columns")
        out.append((rows.contiguous(), torch.arange(off, off + rows.numel(), device=device)))
        off += rows.numel()
    return out


def _gate_inputs(drive: Drive, x, gating):
    """Feedforward pathways with presynaptic dynamics (``network.py:226-250``): their
    factors stepped through the chunk on the device (``wt_gate_scan``), and every
    feedforward pathway's rows' input — times its factors where it has them — as a block
    of input columns of its own (pathways sharing source rows then take their own
    factors). Returns that input, the drive with those blocks as its rows and no gates,
    and the gating state after the chunk. The factors carry no gradient: dL/dx reaches
    the input times them (``network_simulators/engine.py:99-111``)."""
    if isinstance(x, PoissonInput) or drive.sparse_feedforward is not None:
        raise NotImplementedError("presynaptic dynamics on a drawn input or a compressed "
                                  "feedforward side")
    dev = x.device
    B, T, n_in = x.shape
    rows_list = [rows for rows, _ in drive.feedforward]
    blocks = _cached(("gated rows", n_in, str(dev)) + _key(*rows_list), tuple(rows_list),
                     lambda: _gated_rows(rows_list, n_in, dev))
    gating = gating.detach().to(device=dev, dtype=torch.float32).clone(
        memory_format=torch.contiguous_format)
    if gating.dim() != 2 or gating.shape[0] != B:
        raise ValueError(f"gating state of shape {tuple(gating.shape)} for {B} trials")
    R = gating.shape[1]
    xs = x.detach().float().contiguous()
    stream = torch.cuda.current_stream(dev).cuda_stream
    lib = _lib.load()
    cols, feedforward = [], []
    for k, ((rows, W), (src, own)) in enumerate(zip(drive.feedforward, blocks)):
        gate = drive.gate(drive.K_rec + k)
        xr = x[:, :, src]
        if gate is not None:
            if gate.n != src.numel() or gate.start < 0 or gate.start + gate.width > R:
                raise ValueError(f"feedforward pathway {k}: its gate does not match its "
                                 f"{src.numel()} rows and the {R} gating columns")
            f = torch.empty((B, T, gate.n), device=dev)
            params = gate.params.detach().to(device=dev, dtype=torch.float32).contiguous()
            stp_col = gate.start if gate.stp else -1
            sat_col = gate.start + 2 * gate.n * gate.stp if gate.saturates else -1
            _lib.check(lib.wt_gate_scan(xs.data_ptr(), B, T, n_in, src.data_ptr(), gate.n,
                                        params.data_ptr(), gating.data_ptr(), R, stp_col,
                                        sat_col, f.data_ptr(), stream), "wt_gate_scan")
            xr = xr * f
        cols.append(xr)
        feedforward.append((own, W))
    x = torch.cat(cols, dim=2) if cols else x[:, :, :0]
    return x, replace(drive, feedforward=feedforward, gates=[]), gating


def _last_tracked(spikes):
    node = spikes.grad_fn
    return getattr(node, "tracked", None)
