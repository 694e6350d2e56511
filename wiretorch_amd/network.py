"""Conductance-based LIF networks: connectivity, pathways, physiology tables, state.

This is the host side of the drop-in boundary. A network organises its projections
into *pathways* (one per source cell type and input side, recurrent first) and builds,
per forward call, the ``Drive`` (per-pathway rows, weights, kernel scale and synapse
types made) and the ``Physiology`` (per-neuron and per-synapse tables) that
``engine.simulate`` consumes — the same contract as the reference's
``ProjectionNetwork._simulate`` (``src/wiretorch/network_simulators/network.py:889-921``)
calling ``conductance/engine.py:71-89``.

Table values and their order follow the reference so that both engines see
bit-identical inputs:

* per-neuron tables and ``C_m = tau_mem * g_L``: ``conductance/synapses.py:18-29``;
* per-synapse tables, ``g_clip`` inf by default: ``conductance/synapses.py:32-36``;
* kernel jump ``(-g_bar, g_bar) / peak``: ``conductance/synapses.py:70-87``;
* ``alpha = exp(-dt / tau_syn)``, ``beta = exp(-dt / tau_mem)``:
  ``conductance/network.py:195-205``; ``n_ref = round(tau_ref / dt)``:
  ``network.py:553-558``;
* pathway order (per side, ascending source cell type, recurrent first) and rows:
  ``network.py:640-729``; weight assembly ``network.py:731-764``; ``Drive``:
  ``network.py:816-854``;
* learnt physiology: ``network.py:560-638``, ``conductance/network.py:210-246``;
* state at rest (``v = U_reset``, ``g = 0`` laid out ``(B, 2, S, N)``):
  ``conductance/network.py:248-255``.

The NMDA Mg block (``synapses.mg_block_tables``; ``conductance/network.py:138-141``) and
spike-frequency adaptation (``network.py:530-551``) are built. Presynaptic dynamics
(short-term plasticity, receptor saturation) are not part of this build: a network
configured with them raises ``NotImplementedError``.

``Drive`` also accepts a sparse form (``connectome.Connectome``) for connectomes too
large for the reference's dense per-pathway rows (fly scale).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch
from torch import nn

from wiretorch_amd.connectome import Connectome
from wiretorch_amd.projections import Projection, SparseProjection, projection_mask
from wiretorch_amd.stp import as_stp
from wiretorch_amd.synapses import SynapseRegistry, mg_block_tables
from wiretorch_amd.type_parameters import (
    TypeParameters,
    learnt_synapses,
    learnt_types,
)

NEURON_PARAMETERS = ("tau_mem", "theta", "U_reset", "E_L", "g_L")
SYNAPSE_PARAMETERS = ("tau_rise", "tau_decay", "E_syn", "g_bar")
#: Learnable physiology: cell parameters (default value, None if required) and
#: synapse parameters; positive ones are learnt as logarithms.
#: Cell parameters ``learn`` can train, with their defaults (None: required); the
#: adaptation's have defaults (``conductance/network.py:35-41``).
LEARNABLE = {"tau_mem": None, "theta": None, "U_reset": None, "E_L": None, "g_L": None,
             "adapt": 0.0, "tau_adapt": 100.0, "E_adapt": -90.0}
LEARNABLE_SYNAPSE = SYNAPSE_PARAMETERS
POSITIVE = {"tau_mem", "g_L", "tau_rise", "tau_decay", "g_bar", "adapt", "tau_adapt"}
STORAGE_DTYPES = (torch.float32, torch.float16)


# =====================================================================
# What the engine consumes
# =====================================================================


@dataclass
class Drive:
    """The synaptic drive of one forward call, pathway by pathway (recurrent first).

    ``made`` ``(K, S)`` bool: the synapse types each pathway makes; ``scale`` ``(K, N)``:
    its kernel's factor per target neuron. ``recurrent[k]`` / ``feedforward[k]`` are
    ``(rows, W)``: source rows (network neurons / input columns) and ``(n_rows, N)``
    weights. Alternatively ``sparse_recurrent`` / ``sparse_feedforward`` hold the
    connectome in compressed form (``connectome.Connectome``) and the dense lists are
    empty; the pathway count then comes from the connectome.
    """

    made: torch.Tensor
    scale: torch.Tensor
    recurrent: list = field(default_factory=list)
    feedforward: list = field(default_factory=list)
    differentiable_inputs: slice | None = None
    recurrent_gradients: bool = False
    gates: list = field(default_factory=list)
    sparse_recurrent: object | None = None
    sparse_feedforward: object | None = None

    @property
    def K_rec(self) -> int:
        if self.sparse_recurrent is not None:
            return self.sparse_recurrent.n_pathways
        return len(self.recurrent)

    @property
    def K_ff(self) -> int:
        if self.sparse_feedforward is not None:
            return self.sparse_feedforward.n_pathways
        return len(self.feedforward)

    def gate(self, k: int) -> "Gate | None":
        """Pathway ``k``'s presynaptic dynamics (recurrent pathways first), if any."""
        return self.gates[k] if self.gates else None

    def feedforward_activations(self, x: torch.Tensor, factors=None) -> torch.Tensor:
        """``(K_ff, B, T, N)``: each feedforward pathway's input times its weights; a
        pathway with presynaptic dynamics takes its input times its ``factors``
        ``(B, T, n_rows)`` (``network.py:143-157``)."""
        B, T = x.shape[:2]
        if not self.feedforward:
            return x.new_zeros((0, B, T, 0))
        factors = factors or [None] * len(self.feedforward)
        return torch.stack([(x[:, :, rows] if f is None else x[:, :, rows] * f) @ W
                            for (rows, W), f in zip(self.feedforward, factors)])


@dataclass(frozen=True)
class Gate:
    """A pathway's presynaptic dynamics over its ``n`` source rows
    (``network_simulators/network.py:160-183``): ``params`` ``(5,)`` — the saturation
    ``c`` and per-step decay ``d`` of the receptors' gating, the release probability at
    rest ``U`` and the per-step decays ``d_D``, ``d_F`` of the resources' deficit and of
    the facilitation; its columns of the gating state ``(B, R)`` from ``start``: with
    ``stp`` the release probabilities ``u`` then the resources ``x`` (``n`` each), then,
    if it ``saturates``, the receptors' gating ``g``."""

    params: torch.Tensor
    stp: bool
    saturates: bool
    start: int
    n: int

    @property
    def width(self) -> int:
        return self.n * (2 * self.stp + self.saturates)

    @property
    def columns(self) -> slice:
        return slice(self.start, self.start + self.width)


@dataclass
class Physiology:
    """Every parameter of the dynamics (``conductance/dynamics.py:56-92``).

    Per neuron ``(N,)``: ``theta``, ``U_reset``, ``E_L``, ``C_m``, ``beta``. Per synapse
    type ``(S,)``: ``E_syn``, ``g_clip``; ``decay`` and ``jump`` ``(2, S)`` (rise, decay
    component). ``dt`` and ``surr_scale`` are 0-d tensors; ``n_ref`` ``(N,)`` int32 or
    None when no neuron has a refractory period. ``type_of`` ``(N,)`` (optional): each
    neuron's class, such that every per-neuron table and every pathway's kernel scale is
    equal within a class (a network's cell types) — the engine then takes one row per
    class instead of searching the tables for distinct rows (a search whose size the
    host must read), and checks the claim on the device, raising at the next call or
    backward if it fails.
    """

    theta: torch.Tensor
    U_reset: torch.Tensor
    E_L: torch.Tensor
    C_m: torch.Tensor
    beta: torch.Tensor
    E_syn: torch.Tensor
    g_clip: torch.Tensor
    decay: torch.Tensor
    jump: torch.Tensor
    dt: torch.Tensor
    surr_scale: torch.Tensor
    spike_mode: str = "deterministic"
    storage_dtype: torch.dtype = torch.float32
    n_ref: torch.Tensor | None = None
    mg_c: torch.Tensor | None = None
    mg_a: torch.Tensor | None = None
    adapt: torch.Tensor | None = None
    adapt_decay: torch.Tensor | None = None
    E_adapt: torch.Tensor | None = None
    type_of: torch.Tensor | None = None


class _TypeGather(torch.autograd.Function):
    """``table[index]`` whose backward is ``grad @ onehot`` (``onehot[n, j]`` = 1 where
    ``index[n] == j``): one product instead of an accumulation over repeated indices."""

    @staticmethod
    def forward(ctx, table, index, onehot):
        ctx.save_for_backward(onehot)
        return table[index]

    @staticmethod
    def backward(ctx, grad):
        (onehot,) = ctx.saved_tensors
        return grad.to(onehot.dtype) @ onehot, None, None


@dataclass
class Run:
    """What a simulation produced (``network.py:321-351``): ``output`` ``(B, T, N)``,
    the state after the last step, and optional probabilities / tracked variables."""

    output: torch.Tensor
    v: torch.Tensor
    syn: torch.Tensor
    probabilities: torch.Tensor | None = None
    tracked: dict | None = None
    refractory: torch.Tensor | None = None
    gating: torch.Tensor | None = None
    adaptation: torch.Tensor | None = None

    @property
    def spikes(self) -> torch.Tensor:
        return self.output

    @property
    def g(self) -> torch.Tensor:
        return self.syn


def conductance_kernel(tau_rise, tau_decay, g_bar, saturating=None) -> torch.Tensor:
    """``(2, S)`` jump of the rise and decay components per unit input: ``-g_bar`` and
    ``+g_bar`` over the peak of the difference of exponentials, so the waveform peaks at
    ``g_bar`` — unnormalised for the ``saturating`` types, whose input is the fraction of
    receptors opened (``g_bar``: every receptor open) (``conductance/synapses.py:70-87``)."""
    r = tau_rise / tau_decay
    peak = r ** (r / (1 - r)) - r ** (1 / (1 - r))
    if saturating is not None:
        peak = torch.where(saturating, torch.ones_like(peak), peak)
    return torch.stack([-g_bar, g_bar], dim=0) / peak


@dataclass
class InputSide:
    """One source of synaptic input (``network.py:55-77``)."""

    projections: dict
    cell_params: list
    synapse_params: list
    cell_type_indices: np.ndarray
    recurrent: bool
    attribute: str
    mask_buffer: str
    stp: dict | None = None  # (source name, target name) -> STP (or a dict of its fields)


@dataclass(frozen=True)
class Pathway:
    """One source cell type on one input side (``network.py:80-102``). A source type
    with presynaptic dynamics has several: one per (saturating synapse type ``gate``, or
    the rest) and per group of target types sharing one ``stp`` (``targets``: the target
    cell types it reaches, None for all), all over the rows and weights of pathway
    ``source``."""

    index: int
    side: int
    cell_type: int
    mode: str
    gate: int | None = None
    stp: object | None = None
    targets: tuple | None = None
    source: int = -1

    @property
    def presynaptic(self) -> bool:
        return self.gate is not None or self.stp is not None

    @property
    def owner(self) -> int:
        """The pathway whose rows and weights this one shares (itself if none)."""
        return self.source if self.source >= 0 else self.index


def _long(values) -> torch.Tensor:
    return torch.from_numpy(np.asarray(values)).long()


def _check_ids(params, key, what):
    ids = sorted(p[key] for p in params)
    assert ids == list(range(len(ids))), f"{what}: ids {ids} are not 0, 1, 2, ..."


def validate(dt, cell_params, cell_type_indices, sides) -> None:
    """Construction checks with messages naming what is wrong (``network.py:1059-1109``)."""
    assert isinstance(dt, (int, float)) and dt > 0, f"time step {dt!r} is not a positive number"
    assert dt <= 100.0, f"time step {dt} ms exceeds 100 ms (milliseconds expected)"
    _check_ids(cell_params, "cell_id", "cell_ids in cell_params")
    assert cell_type_indices.ndim == 1 and cell_type_indices.shape[0] > 0
    assert np.all((cell_type_indices >= 0) & (cell_type_indices < len(cell_params)))
    targets = {p["name"]: p["cell_id"] for p in cell_params}
    n_target = np.bincount(cell_type_indices, minlength=len(cell_params))
    for side in sides:
        _check_ids(side.cell_params, "cell_id", f"{side.attribute} source cell_ids")
        assert side.synapse_params, f"{side.attribute}: no synapse types given"
        _check_ids(side.synapse_params, "synapse_id", f"{side.attribute} synapse_ids")
        types = side.cell_type_indices
        assert types.ndim == 1 and np.all((types >= 0) & (types < len(side.cell_params)))
        sources = {p["name"]: p["cell_id"] for p in side.cell_params}
        n_source = np.bincount(types, minlength=len(side.cell_params))
        if is_sparse(side):
            got = (side.projections.n_source, side.projections.n_target)
            want = (len(types), len(cell_type_indices))
            assert got == want, f"{side.attribute}: sparse projection {got} != {want}"
            continue
        for (src, tgt), projection in side.projections.items():
            assert src in sources, f"{side.attribute}: no source cell type {src!r}"
            assert tgt in targets, f"{side.attribute}: no target cell type {tgt!r}"
            want = (int(n_source[sources[src]]), int(n_target[targets[tgt]]))
            got = (projection.n_source, projection.n_target)
            assert got == want, f"{side.attribute} projection ({src!r}, {tgt!r}) {got} != {want}"


def is_sparse(side: InputSide) -> bool:
    """Whether a side is one ``SparseProjection`` (rather than per-type-pair blocks)."""
    return isinstance(side.projections, SparseProjection)


# =====================================================================
# The network
# =====================================================================


class ProjectionNetwork(nn.Module):
    """What every network family shares (``network.py:354-1026``): input sides of
    projections organised into pathways, the per-call ``Drive``, and the state ``v``
    ``(B, N)`` plus the family's synaptic state, continued from one ``forward`` call to
    the next until ``reset_state``.

    A family supplies its physiology through ``_register_physiology``,
    ``_set_timestep``, ``_physiology`` and ``_initial_state``, its engine as
    ``_engine``, and optionally extra engine arguments and state (``_engine_kwargs``,
    ``_extra_state``).
    """

    state_name = "syn"
    output_name = "output"
    recurrent_gradients = False

    def __init__(
        self,
        *,
        dt: float,
        cell_params: list[dict],
        cell_type_indices: np.ndarray,
        sides: list[InputSide],
        unify_synapses: bool,
        batch_size: int,
        track_variables: bool,
        track_gradients: bool,
        track_batch_idx: int | None,
        storage_dtype=torch.float32,
        learn: dict | None = None,
    ):
        super().__init__()
        validate(dt, cell_params, cell_type_indices, sides)
        self.learn = dict(learn or {})
        self.batch_size = batch_size
        self.track_variables = track_variables
        self.track_gradients = track_gradients
        self.track_batch_idx = track_batch_idx
        self.storage_dtype = storage_dtype
        self.differentiable_inputs = None
        self.cell_params = cell_params
        self.n_cell_types = len(cell_params)
        self.n_neurons = int(cell_type_indices.shape[0])
        self._sides = sides
        self._names = {c["cell_id"]: c["name"] for c in cell_params}
        self.registry = SynapseRegistry.build(
            [(s.cell_params, s.synapse_params) for s in sides], unify=unify_synapses
        )
        self.register_buffer("cell_type_indices", _long(cell_type_indices))
        for side in sides:
            if is_sparse(side):  # one module; no dense mask (the connectome is the mask)
                setattr(self, side.attribute, side.projections)
                continue
            modules = {f"{s}__{t}": p for (s, t), p in side.projections.items()}
            setattr(self, side.attribute, nn.ModuleDict(modules))
            self.register_buffer(side.mask_buffer, torch.from_numpy(self._mask(side)))
        self._register_physiology()
        self.pathways = self._build_pathways()
        # what every call's Drive shares while nothing is learnt in it (the same tensors
        # each call, so the engine's tables built from them are reused)
        order = [p.index for p in self.pathways]
        self.register_buffer("_made_in_order", self._made[order].clone(), persistent=False)
        self.register_buffer("_unit_scale", torch.ones((len(order), self.n_neurons)),
                             persistent=False)
        self.set_timestep(float(dt))

    # ------------------------------------------------------------------
    # Construction
    # ------------------------------------------------------------------

    @property
    def storage_dtype(self) -> torch.dtype:
        """What the kernels store conductances in (arithmetic stays float32)."""
        return self._storage_dtype

    @storage_dtype.setter
    def storage_dtype(self, dtype) -> None:
        dtype = getattr(torch, dtype) if isinstance(dtype, str) else dtype
        if dtype not in STORAGE_DTYPES:
            raise ValueError(f"storage dtype {dtype} not supported (supported: {STORAGE_DTYPES})")
        self._storage_dtype = dtype

    def _block(self, side: InputSide, src: str, tgt: str):
        src_id = next(c["cell_id"] for c in side.cell_params if c["name"] == src)
        tgt_id = next(c["cell_id"] for c in self.cell_params if c["name"] == tgt)
        rows = np.flatnonzero(side.cell_type_indices == src_id)
        cols = np.flatnonzero(self.cell_type_indices.cpu().numpy() == tgt_id)
        return rows, cols

    def _mask(self, side: InputSide) -> np.ndarray:
        mask = np.zeros((len(side.cell_type_indices), self.n_neurons), dtype=bool)
        for (src, tgt), projection in side.projections.items():
            rows, cols = self._block(side, src, tgt)
            if rows.size and cols.size:
                mask[np.ix_(rows, cols)] = projection_mask(projection)
        return mask

    def _per_neuron(self, name: str, default: float | None = None) -> torch.Tensor:
        lookup = np.zeros(self.n_cell_types, dtype=np.float32)
        for cell in self.cell_params:
            lookup[cell["cell_id"]] = cell[name] if default is None else cell.get(name, default)
        return torch.from_numpy(lookup[self.cell_type_indices.cpu().numpy()])

    def _saturation(self) -> torch.Tensor:
        """``(S,)``: each synapse type's saturation (0: none)."""
        return torch.zeros(len(self.registry))

    def _build_pathways(self) -> list[Pathway]:
        """Pathways by side and source cell type (``network.py:640-729``); a source type
        that makes saturating synapse types or has short-term plasticity gets one per
        (saturating type, or the rest) x (target types sharing one STP), sharing its rows
        and weights. Presynaptic dynamics are taken on feedforward sides of per-type-pair
        blocks only."""
        saturating = self._saturation() > 0
        pathways, made = [], []
        for side_no, side in enumerate(self._sides):
            side_makes = self.registry.made_by(side_no, side.synapse_params).values()
            presynaptic = bool(side.stp) or any(bool((m & saturating).any()) for m in side_makes)
            if presynaptic and (side.recurrent or is_sparse(side)):
                raise NotImplementedError(
                    f"{side.attribute}: presynaptic dynamics (short-term plasticity, saturating "
                    "synapse types) are supported on feedforward sides of per-type-pair "
                    "projections only")
            if is_sparse(side):
                self._sparse_pathways(side_no, side, pathways, made)
                continue
            names = {c["cell_id"]: c["name"] for c in side.cell_params}
            stp = {key: as_stp(value) for key, value in (side.stp or {}).items()}
            unknown = set(stp) - set(side.projections)
            if unknown:
                raise ValueError(f"{side.attribute}: short-term plasticity for "
                                 f"{sorted(unknown)}, which have no projection")
            modes: dict[str, str] = {}
            for (src, _), projection in side.projections.items():
                mode = modes.setdefault(src, projection.caching_mode)
                if mode != projection.caching_mode:
                    raise ValueError(
                        f"source cell type {src!r} has projections with mixed caching modes"
                    )
            for cell_type, synapses in self.registry.made_by(
                side_no, side.synapse_params
            ).items():
                mode = modes.get(names[cell_type])
                if mode is None:
                    continue
                source = len(pathways)
                rows = np.flatnonzero(side.cell_type_indices == cell_type)
                plain = synapses & ~saturating
                parts = [(None, plain)] if bool(plain.any()) else []
                for gate in torch.nonzero(synapses & saturating).flatten().tolist():
                    one = torch.zeros_like(synapses)
                    one[gate] = True
                    parts.append((gate, one))
                groups: dict = {}  # STP (or None) -> the target cell types it reaches
                for target, target_name in sorted(self._names.items()):
                    groups.setdefault(stp.get((names[cell_type], target_name)), []).append(target)
                for plasticity, targets in groups.items():
                    targets = None if len(groups) == 1 else tuple(targets)
                    for gate, mask in parts:
                        index = len(pathways)
                        self.register_buffer(f"_rows_{index}", _long(rows), persistent=False)
                        pathways.append(Pathway(index, side_no, cell_type, mode, gate, plasticity,
                                                targets, -1 if index == source else source))
                        made.append(mask)
                        if targets is not None:
                            reached = np.isin(self.cell_type_indices.cpu().numpy(), targets)
                            self.register_buffer(f"_targets_{index}",
                                                 torch.from_numpy(reached.astype(np.float32)),
                                                 persistent=False)
        self.register_buffer(
            "_made",
            torch.stack(made) if made else torch.zeros((0, len(self.registry)), dtype=torch.bool),
            persistent=False,
        )
        # Recurrent pathways first: the order the dynamics inject them in.
        pathways = sorted(pathways, key=lambda p: not self._sides[p.side].recurrent)
        # The gating state's columns: each presynaptic pathway's (see ``Gate``), in order,
        # and their values at rest (u = U, x = 1, g = 0).
        columns, rest = {}, []
        for p in pathways:
            if p.presynaptic:
                n = getattr(self, f"_rows_{p.index}").numel()
                columns[p.index] = (int(sum(map(len, rest))), int(n))
                if p.stp is not None:
                    rest += [np.full(n, p.stp.U), np.ones(n)]
                if p.gate is not None:
                    rest.append(np.zeros(n))
        self._gate_columns = columns
        self.register_buffer("_gating_rest", torch.from_numpy(
            np.concatenate(rest or [np.zeros(0)]).astype(np.float32)), persistent=False)
        self.n_gating = int(self._gating_rest.numel())
        return pathways

    def _gate(self, pathway: Pathway) -> Gate | None:
        """A presynaptic pathway's ``Gate`` (its parameters at this time step), else None."""
        if not pathway.presynaptic:
            return None
        return Gate(getattr(self, f"_gate_{pathway.index}"), pathway.stp is not None,
                    pathway.gate is not None, *self._gate_columns[pathway.index])

    def _set_gates(self, saturation: torch.Tensor, gate_decay: torch.Tensor) -> None:
        """Each presynaptic pathway's ``Gate.params`` at this time step, on the device: the
        saturating type's saturation and gating decay, the STP's ``U`` and decays
        (``network.py:855-874``)."""
        dt = float(self.dt)
        for p in self.pathways:
            if not p.presynaptic:
                continue
            zero = torch.zeros((), device=self.device)
            c, d = ((saturation[p.gate], gate_decay[p.gate]) if p.gate is not None
                    else (zero, zero))
            U, d_D, d_F = (p.stp.U, *p.stp.decays(dt)) if p.stp is not None else (1.0, 0.0, 0.0)
            params = torch.cat([torch.stack([c, d]).float(),
                                torch.tensor([U, d_D, d_F], device=self.device)])
            self.register_buffer(f"_gate_{p.index}", params, persistent=False)

    def _sparse_pathways(self, side_no: int, side: InputSide, pathways, made) -> None:
        """A ``SparseProjection`` side's pathways: one per distinct set of synapse types
        its source cell types make (in order of first appearance over ascending cell
        type), instead of one per source cell type — the same sum (see
        ``engine.fold_pathways``), and a handful of pathways however many cell types.
        ``_group_of_<side>`` gives each source its pathway within the side (-1: its type
        makes no synapse)."""
        groups: dict[bytes, int] = {}
        of_type = np.full(len(side.cell_params), -1, dtype=np.int64)
        for cell_type, synapses in self.registry.made_by(side_no, side.synapse_params).items():
            key = synapses.numpy().tobytes()
            if key not in groups:
                groups[key] = len(groups)
                pathways.append(Pathway(len(pathways), side_no, -1, "sparse"))
                made.append(synapses)
            of_type[cell_type] = groups[key]
        self.register_buffer(f"_group_of_{side_no}", _long(of_type[side.cell_type_indices]),
                             persistent=False)
        self._sparse_counts = getattr(self, "_sparse_counts", {})
        self._sparse_counts[side_no] = len(groups)

    def _assemble(self, pathway: Pathway, connectome: bool = False) -> torch.Tensor:
        """The pathway's ``(n_rows, N)`` weights from its projections."""
        side = self._sides[pathway.side]
        rows = getattr(self, f"_rows_{pathway.index}")
        W = torch.zeros((rows.numel(), self.n_neurons), **self._float)
        projections = getattr(self, side.attribute)
        src = next(c["name"] for c in side.cell_params if c["cell_id"] == pathway.cell_type)
        for tgt_id, tgt in self._names.items():
            key = f"{src}__{tgt}"
            if key not in projections:
                continue
            cols = (self.cell_type_indices == tgt_id).nonzero(as_tuple=True)[0]
            if cols.numel():
                projection = projections[key]
                W[:, cols] = projection.connectome if connectome else projection()
        return W

    def _cache_weights(self) -> None:
        for pathway in sorted(self.pathways, key=lambda p: p.index):  # owners first
            if pathway.mode not in ("weights", "sparse"):
                if pathway.owner != pathway.index:  # the very tensor of its source pathway
                    W = getattr(self, f"_weights_{pathway.owner}")
                else:
                    W = self._assemble(pathway, connectome=pathway.mode == "scaling_factors").detach()
                self.register_buffer(f"_weights_{pathway.index}", W, persistent=False)

    def set_timestep(self, dt: float) -> None:
        """Set the time step, recompute what depends on it, reset the state."""
        assert isinstance(dt, float) and dt > 0, "dt must be a positive float"
        self.register_buffer("dt", torch.tensor(dt, device=self.device))
        self._set_timestep()
        self._cache_weights()
        self.reset_state()

    # ------------------------------------------------------------------
    # Per call
    # ------------------------------------------------------------------

    @property
    def device(self) -> torch.device:
        return self.cell_type_indices.device

    @property
    def _float(self) -> dict:
        return {"device": self.device, "dtype": self.dt.dtype}

    def _scaling_matrix(self, side_index: int) -> torch.Tensor:
        side = self._sides[side_index]
        src_ids = {c["name"]: c["cell_id"] for c in side.cell_params}
        tgt_ids = {c["name"]: c["cell_id"] for c in self.cell_params}
        sf = torch.ones((len(side.cell_params), self.n_cell_types), **self._float)
        for key, projection in getattr(self, side.attribute).items():
            if projection.caching_mode == "scaling_factors":
                src, tgt = key.split("__", 1)
                sf[src_ids[src], tgt_ids[tgt]] = projection.kernel_factor()
        return sf

    def _edge_sides(self) -> list[int]:
        """The sides whose weights the HIP engine takes synapse by synapse: the recurrent
        side when every one of its pathways is learnt (``weights``) from blocks that form
        their entries one at a time (``Projection.edge_values``). Those entries are then
        computed for the synapses only — the blocks' values there, bit for bit — instead
        of as dense blocks assembled into rows and gathered again; the CPU oracle keeps the
        dense form (its float32 products are what the recorded fixtures hold)."""
        if getattr(self._engine, "__name__", "") != "wiretorch_amd.engine":
            return []
        out = []
        for side_no, side in enumerate(self._sides):
            if not side.recurrent or is_sparse(side):
                continue
            pathways = [p for p in self.pathways if p.side == side_no]
            projections = getattr(self, side.attribute)
            if (pathways and all(p.mode == "weights" for p in pathways)
                    and all(p.edge_mask() is not None for p in projections.values())):
                out.append(side_no)
        return out

    def _edge_plan(self, side_no: int) -> dict:
        """The compressed structure of an edge side (``_edge_sides``), cached while its
        masks and rows are unchanged: CSR by source (``indptr``, ``targets`` ascending),
        each source's pathway within the side, and per block the row-major positions of
        its synapses plus the permutation from the blocks' concatenation to CSR order."""
        side = self._sides[side_no]
        projections = getattr(self, side.attribute)
        pathways = [p for p in self.pathways if p.side == side_no]
        rows = [getattr(self, f"_rows_{p.index}") for p in pathways]
        key = tuple((t.data_ptr(), t._version) for t in rows) + tuple(
            (m.data_ptr(), m._version) for m in (q.edge_mask() for q in projections.values()))
        plans = self.__dict__.setdefault("_edge_plans", {})
        hit = plans.get(side_no)
        if hit is not None and hit["key"] == key:
            return hit
        N, dev = self.n_neurons, self.device
        pathway_of = torch.full((N,), -1, dtype=torch.int64, device=dev)
        srcs, tgts, parts = [], [], []
        for k, (pw, src_rows) in enumerate(zip(pathways, rows)):
            pathway_of[src_rows] = k
            src = next(c["name"] for c in side.cell_params if c["cell_id"] == pw.cell_type)
            for tgt_id, tgt in self._names.items():
                if f"{src}__{tgt}" not in projections:
                    continue
                block = projections[f"{src}__{tgt}"]
                cols = (self.cell_type_indices == tgt_id).nonzero(as_tuple=True)[0]
                if not cols.numel():
                    continue
                r, c = (block.edge_mask() != 0).nonzero(as_tuple=True)
                srcs.append(src_rows[r])
                tgts.append(cols[c])
                parts.append((block, r * block.n_target + c))
        src = torch.cat(srcs) if srcs else torch.zeros(0, dtype=torch.int64, device=dev)
        tgt = torch.cat(tgts) if tgts else torch.zeros(0, dtype=torch.int64, device=dev)
        order = torch.argsort(src * N + tgt)
        indptr = torch.zeros(N + 1, dtype=torch.int64, device=dev)
        indptr[1:] = torch.cumsum(torch.bincount(src, minlength=N), 0)
        plan = dict(key=key, indptr=indptr, targets=tgt[order].to(torch.int32).contiguous(),
                    pathway=pathway_of, parts=parts, order=order, K=len(pathways))
        plans[side_no] = plan
        return plan

    def _edge_connectome(self, side_no: int) -> Connectome:
        """An edge side's connectome with this call's weights (differentiable in the
        blocks' parameters)."""
        plan = self._edge_plan(side_no)
        if plan["parts"]:
            # index_select, not advanced indexing: the indices are distinct, and its
            # backward scatters without the sort an index_put with accumulation makes
            w = torch.cat([block.edge_values(flat) for block, flat in plan["parts"]])
            w = w.index_select(0, plan["order"])
        else:
            w = torch.zeros(0, **self._float)
        return Connectome(self.n_neurons, self.n_neurons, plan["indptr"], plan["targets"], w,
                          plan["pathway"], plan["K"])

    def _drive(self) -> Drive:
        """Per pathway: rows, current weights and kernel scale (``network.py:816-854``)."""
        scaling, assembled = {}, {}
        unit = self._unit_scale.to(self.dt.dtype)
        ones = unit[0] if unit.shape[0] else torch.ones(self.n_neurons, **self._float)
        scales, recurrent, feedforward = [], [], []
        sparse = {side_no: self._edge_connectome(side_no) for side_no in self._edge_sides()}
        for pathway in self.pathways:
            if pathway.side in sparse and pathway.mode == "weights":
                scales.append(ones)
                continue
            if pathway.mode == "sparse":
                scales.append(ones)
                if pathway.side not in sparse:
                    side = self._sides[pathway.side]
                    proj = getattr(self, side.attribute)
                    sparse[pathway.side] = Connectome(
                        proj.n_source, self.n_neurons, proj.indptr, proj.targets, proj(),
                        getattr(self, f"_group_of_{pathway.side}"),
                        self._sparse_counts[pathway.side])
                continue
            if pathway.mode != "weights":
                W = getattr(self, f"_weights_{pathway.index}")
            elif pathway.owner in assembled:  # the very tensor of its source pathway
                W = assembled[pathway.owner]
            else:
                W = assembled[pathway.owner] = self._assemble(pathway)
            if pathway.mode == "scaling_factors":
                if pathway.side not in scaling:
                    scaling[pathway.side] = self._scaling_matrix(pathway.side)
                scales.append(scaling[pathway.side][pathway.cell_type, self.cell_type_indices])
            else:
                scales.append(ones)
            if pathway.targets is not None:  # it reaches only these target types
                scales[-1] = scales[-1] * getattr(self, f"_targets_{pathway.index}")
            rows = getattr(self, f"_rows_{pathway.index}")
            target = recurrent if self._sides[pathway.side].recurrent else feedforward
            target.append((rows, W))
        if any(p.mode == "scaling_factors" or p.targets is not None for p in self.pathways):
            scale = torch.stack(scales)
        else:  # every kernel scale is 1: the same tensor each call
            scale = unit
        return Drive(
            made=self._made_in_order,
            scale=scale,
            recurrent=recurrent,
            feedforward=feedforward,
            differentiable_inputs=self.differentiable_inputs,
            recurrent_gradients=self.recurrent_gradients,
            gates=[self._gate(p) for p in self.pathways] if self.n_gating else [],
            sparse_recurrent=next((c for i, c in sparse.items() if self._sides[i].recurrent), None),
            sparse_feedforward=next((c for i, c in sparse.items() if not self._sides[i].recurrent),
                                    None),
        )

    @torch.compiler.disable
    def _simulate(self, input_spikes, probabilities: bool = False) -> Run:
        if isinstance(input_spikes, np.ndarray):
            input_spikes = torch.from_numpy(input_spikes).to(self.device)
        self._validate_forward(input_spikes)
        retain = [] if self.track_gradients else None
        run = self._engine.simulate(
            self.v,
            self._synaptic,
            input_spikes.to(self.dt.dtype),
            self._drive(),
            self._physiology(),
            probabilities=probabilities,
            track=self.track_variables,
            track_batch_idx=self.track_batch_idx,
            retain=retain,
            **self._engine_kwargs(),
        )
        if retain is not None:
            self._retained = retain
        self.v = run.v.detach()
        self._synaptic = run.syn.detach()
        self._after_run(run)
        return run

    def _engine_kwargs(self) -> dict:
        """Family-specific arguments of ``engine.simulate``."""
        return {}

    def _after_run(self, run: Run) -> None:
        """Keep the family's extra state from ``run``."""

    def _validate_forward(self, input_spikes: torch.Tensor) -> None:
        from wiretorch_amd.inputs import PoissonInput

        assert isinstance(input_spikes, (torch.Tensor, PoissonInput)), (
            "input_spikes must be a Tensor (or an on-device PoissonInput)")
        assert input_spikes.device == self.device, (
            f"input_spikes on {input_spikes.device}, model on {self.device}"
        )
        assert input_spikes.ndim == 3, f"input of shape {tuple(input_spikes.shape)}: expected (batch, steps, inputs)"
        assert input_spikes.shape[2] == self.n_inputs, (
            f"input has {input_spikes.shape[2]} channels, the network {self.n_inputs}"
        )
        if input_spikes.shape[0] != self.batch_size:
            raise ValueError(
                f"the input holds {input_spikes.shape[0]} trials but the state holds "
                f"{self.batch_size}: reset the state for the new batch size first"
            )

    # ------------------------------------------------------------------
    # State
    # ------------------------------------------------------------------

    @property
    def _synaptic(self) -> torch.Tensor:
        return getattr(self, self.state_name)

    @_synaptic.setter
    def _synaptic(self, value: torch.Tensor) -> None:
        setattr(self, self.state_name, value)

    def reset_state(self, batch_size: int | None = None) -> None:
        if batch_size is not None:
            self.batch_size = batch_size
        v, syn = self._initial_state()
        self.register_buffer("v", v, persistent=False)
        self.register_buffer(self.state_name, syn, persistent=False)
        self._reset_extra()

    def _reset_extra(self) -> None:
        """Reset the family's extra state."""

    def get_checkpoint_state(self) -> dict[str, np.ndarray]:
        """The state as arrays (``network.py:971-1005``)."""
        return {"v": self.v.cpu().numpy(), self.state_name: self._synaptic.cpu().numpy()}

    def load_checkpoint_state(self, state: dict[str, np.ndarray]) -> None:
        self.v = torch.from_numpy(state["v"]).to(self.device)
        self._synaptic = torch.from_numpy(state[self.state_name]).to(self.device)

    def _weight_matrix(self, side_index: int) -> torch.Tensor:
        side = self._sides[side_index]
        if is_sparse(side):
            return getattr(self, side.attribute).dense()
        W = torch.zeros((len(side.cell_type_indices), self.n_neurons), **self._float)
        for (src, tgt), _ in side.projections.items():
            rows, cols = self._block(side, src, tgt)
            if rows.size and cols.size:
                W[np.ix_(rows, cols)] = getattr(self, side.attribute)[f"{src}__{tgt}"]()
        return W


class ConductanceNetwork(ProjectionNetwork):
    """Base of the conductance-based LIF networks (``conductance/network.py:44-255`` for
    the mechanisms this build supports).

    State ``v`` ``(B, N)``, conductances ``(B, N, 2, S)`` (stored ``(B, 2, S, N)``) and
    refractory counters ``(B, N)`` int32 continue from one ``forward`` call to the next
    until ``reset_state``.
    """

    state_name = "g"
    output_name = "s"
    has_refractory = True

    def __init__(self, *, surrgrad_scale: float, spike_mode: str, **kwargs):
        assert isinstance(surrgrad_scale, (int, float)) and surrgrad_scale > 0
        if spike_mode != "deterministic":
            raise NotImplementedError("only spike_mode='deterministic' is supported")
        self.spike_mode = spike_mode
        self._surrgrad_scale = float(surrgrad_scale)
        super().__init__(**kwargs)

    def _register_physiology(self) -> None:
        for name in NEURON_PARAMETERS:
            self.register_buffer(name, self._per_neuron(name))
        self.register_buffer("C_m", self.tau_mem * self.g_L)
        for name in SYNAPSE_PARAMETERS:
            self.register_buffer(name, self.registry.table(name))
        self.register_buffer("g_clip", self.registry.table("g_clip", default=float("inf")))
        # receptor saturation (conductance/synapses.py:59-67): the fraction of a source's
        # closed receptors of a type that one of its spikes opens (0: none)
        saturation = self.registry.table("saturation", default=0.0)
        assert bool(((saturation >= 0) & (saturation <= 1)).all()), (
            "synapse params: saturation must be in [0, 1]")
        self.register_buffer("saturation", saturation, persistent=False)
        # from the synapse parameters, not saved with the module (state dicts load between
        # networks with and without a block)
        for name, table in mg_block_tables(self.registry).items():
            self.register_buffer(name, table, persistent=False)
        self._mg_block = bool(self.mg_c.any())
        tau_ref = self._per_neuron("tau_ref", 0.0)
        assert bool((tau_ref >= 0).all()), "cell_params: tau_ref must be >= 0"
        self.register_buffer("tau_ref", tau_ref, persistent=False)
        # Spike-frequency adaptation (network.py:530-551): per cell type, its rise at each
        # of the neuron's spikes (adapt, 0: none), its time constant (tau_adapt, ms) and
        # reversal potential (E_adapt, mV); from the cell parameters, not saved.
        adapt = self._per_neuron("adapt", LEARNABLE["adapt"])
        tau_adapt = self._per_neuron("tau_adapt", LEARNABLE["tau_adapt"])
        assert bool((adapt >= 0).all()), "cell_params: a negative adaptation rise (adapt)"
        assert bool((tau_adapt[adapt > 0] > 0).all()), "cell_params: tau_adapt not positive"
        self.register_buffer("adapt", adapt, persistent=False)
        self.register_buffer("tau_adapt", tau_adapt, persistent=False)
        self.register_buffer("E_adapt", self._per_neuron("E_adapt", LEARNABLE["E_adapt"]),
                             persistent=False)
        self._adapting = bool(adapt.any())
        self.register_buffer(
            "surrgrad_scale", torch.tensor(self._surrgrad_scale, dtype=torch.float32)
        )
        self._register_learnt()

    def _register_learnt(self) -> None:
        learn = self.learn
        unknown = set(learn) - set(LEARNABLE) - set(LEARNABLE_SYNAPSE)
        assert not unknown, f"nothing named {sorted(unknown)} can be learnt"
        cells = sorted(self.cell_params, key=lambda c: c["cell_id"])
        names = [c["name"] for c in cells]
        learnt = {
            name: learnt_types(learn[name], names, f"learn[{name!r}]")
            for name in LEARNABLE
            if learn.get(name)
        }
        if learnt:
            values = {name: [c[name] if LEARNABLE[name] is None else c.get(name, LEARNABLE[name])
                             for c in cells] for name in learnt}
            self.cell_parameters = TypeParameters(
                values, learnt=learnt, positive=POSITIVE & set(learnt)
            )
            for name, types in learnt.items():
                mask = torch.isin(self.cell_type_indices, torch.tensor(types))
                self.register_buffer(f"_learnt_{name}", mask, persistent=False)
        synapses = self.registry.synapses
        learnt = {
            name: learnt_synapses(learn[name], synapses, f"learn[{name!r}]")
            for name in LEARNABLE_SYNAPSE
            if learn.get(name)
        }
        if learnt:
            values = {name: self.registry.table(name).tolist() for name in learnt}
            self.synapse_parameters = TypeParameters(
                values, learnt=learnt, positive=POSITIVE & set(learnt)
            )
            for name, types in learnt.items():
                mask = torch.zeros(len(synapses), dtype=torch.bool)
                mask[types] = True
                self.register_buffer(f"_learnt_{name}", mask, persistent=False)
            tau_decay = getattr(self, "_learnt_tau_decay", None)
            if tau_decay is not None and bool((tau_decay & (self.saturation > 0)).any()):
                fixed = [synapses[i]["name"] for i in
                         torch.nonzero(tau_decay & (self.saturation > 0)).flatten().tolist()]
                raise ValueError(f"tau_decay of the saturating synapse types {fixed} cannot be "
                                 "learnt: their gating decays with it, fixed per time step")

    def _learnt(self, name: str, fixed: torch.Tensor, decay: bool = False):
        """``fixed`` with the learnt types' values in place (``decay``: as
        ``exp(-dt / value)``), ``network.py:621-634``."""
        mask = getattr(self, f"_learnt_{name}", None)
        if mask is None:
            return fixed
        if name in LEARNABLE_SYNAPSE:
            value = self.synapse_parameters.value(name)
        else:
            value = self._per_type(self.cell_parameters.value(name))
        if decay:
            value = torch.exp(-self.dt / value)
        return torch.where(mask, value, fixed)

    def _learns(self, *names: str) -> bool:
        return any(hasattr(self, f"_learnt_{n}") for n in names)

    def _per_type(self, table: torch.Tensor) -> torch.Tensor:
        """``table[cell_type_indices]``: each neuron's value of its type's entry. With
        few types (at most 2^24 neuron-type pairs) the gradient is summed per type by one
        matrix-vector product with the neurons' one-hot type matrix (cached), where
        advanced indexing's backward adds the many repeats of one type index one after
        another."""
        idx = self.cell_type_indices
        n_types = int(table.shape[0])
        if idx.numel() * n_types > 1 << 24:
            return table[idx]
        key = (idx.data_ptr(), idx._version, n_types, table.dtype)
        if getattr(self, "_onehot_key", None) != key:
            self._onehot = nn.functional.one_hot(idx, n_types).to(table.dtype)
            self._onehot_key = key
        return _TypeGather.apply(table, idx, self._onehot)

    def _saturation(self) -> torch.Tensor:
        return self.saturation

    def _set_timestep(self) -> None:
        self.register_buffer("tau_syn", torch.stack((self.tau_rise, self.tau_decay)))
        self.register_buffer("alpha", torch.exp(-self.dt / self.tau_syn))
        self.register_buffer("beta", torch.exp(-self.dt / self.tau_mem))
        self.register_buffer(
            "g_scale", conductance_kernel(self.tau_rise, self.tau_decay, self.g_bar,
                                          self.saturation > 0)
        )
        # the saturating types' gating decays as their conductances do
        self._set_gates(self.saturation, self.alpha[1])
        n_ref = torch.round(self.tau_ref / self.dt).to(torch.int32)
        self.register_buffer("n_ref", n_ref, persistent=False)
        self._refractory = bool(n_ref.any())
        self.register_buffer("adapt_decay", torch.exp(-self.dt / self.tau_adapt),
                             persistent=False)

    def _physiology(self) -> Physiology:
        """The engine's parameters for one call (``conductance/network.py:210-246``)."""
        learnt = self._learnt
        C_m, decay, jump = self.C_m, self.alpha, self.g_scale
        if self._learns("tau_mem", "g_L"):
            C_m = learnt("tau_mem", self.tau_mem) * learnt("g_L", self.g_L)
        if self._learns("tau_rise", "tau_decay", "g_bar"):
            tau_rise = learnt("tau_rise", self.tau_rise)
            tau_decay = learnt("tau_decay", self.tau_decay)
            decay = torch.exp(-self.dt / torch.stack((tau_rise, tau_decay)))
            jump = conductance_kernel(tau_rise, tau_decay, learnt("g_bar", self.g_bar),
                                      self.saturation > 0)
        return Physiology(
            theta=learnt("theta", self.theta),
            U_reset=learnt("U_reset", self.U_reset),
            E_L=learnt("E_L", self.E_L),
            C_m=C_m,
            beta=learnt("tau_mem", self.beta, decay=True),
            E_syn=learnt("E_syn", self.E_syn),
            g_clip=self.g_clip,
            decay=decay,
            jump=jump,
            dt=self.dt,
            surr_scale=self.surrgrad_scale,
            spike_mode=self.spike_mode,
            storage_dtype=self.storage_dtype,
            n_ref=self.n_ref if self._refractory else None,
            type_of=self.cell_type_indices,
            mg_c=self.mg_c if self._mg_block else None,
            mg_a=self.mg_a if self._mg_block else None,
            **(dict(adapt=learnt("adapt", self.adapt),
                    adapt_decay=learnt("tau_adapt", self.adapt_decay, decay=True),
                    E_adapt=learnt("E_adapt", self.E_adapt)) if self._adapting else {}),
        )

    def _initial_state(self):
        v = self.U_reset.expand(self.batch_size, self.n_neurons).clone()
        g = torch.zeros(
            (self.batch_size, 2, len(self.registry), self.n_neurons), device=self.device
        ).permute(0, 3, 1, 2)
        return v, g

    def _engine_kwargs(self) -> dict:
        return {"refractory": self.refractory,
                **({"gating": self.gating} if self.n_gating else {}),
                **({"adaptation": self.adaptation} if self._adapting else {})}

    def _after_run(self, run: Run) -> None:
        if run.refractory is not None:
            self.refractory = run.refractory
        if run.gating is not None and self.n_gating:
            self.gating = run.gating.detach()
        if run.adaptation is not None:  # the next chunk starts from it, without its graph
            self.adaptation = run.adaptation.detach()

    def _reset_extra(self) -> None:
        counter = torch.zeros((self.batch_size, self.n_neurons), dtype=torch.int32,
                              device=self.device)
        self.register_buffer("refractory", counter, persistent=False)
        self.register_buffer("adaptation", torch.zeros((self.batch_size, self.n_neurons),
                                                       device=self.device), persistent=False)
        self.register_buffer("gating", self._gating_rest.to(self.device).expand(
            self.batch_size, -1).clone(), persistent=False)

    def get_checkpoint_state(self) -> dict[str, np.ndarray]:
        state = super().get_checkpoint_state()
        if self._refractory:
            state["refractory"] = self.refractory.cpu().numpy()
        if self._adapting:
            state["adaptation"] = self.adaptation.cpu().numpy()
        if self.n_gating:
            state["gating"] = self.gating.cpu().numpy()
        return state

    def load_checkpoint_state(self, state: dict[str, np.ndarray]) -> None:
        super().load_checkpoint_state(state)
        self.refractory = (
            torch.from_numpy(state["refractory"]).to(self.device)
            if "refractory" in state
            else torch.zeros_like(self.v, dtype=torch.int32)
        )
        self.adaptation = (torch.from_numpy(state["adaptation"]).to(self.device)
                           if "adaptation" in state else torch.zeros_like(self.v))
        self.gating = (torch.from_numpy(state["gating"]).to(self.device) if "gating" in state
                       else self._gating_rest.to(self.device).expand(self.v.shape[0], -1).clone())


def _engine_module():
    from wiretorch_amd import engine

    return engine


class ConductanceLIFNetwork(ConductanceNetwork):
    """Recurrent conductance-based LIF network (``conductance/recurrent.py:19-208``).

    ``rec_projections`` and ``ff_projections`` map ``(source type, target type)`` to a
    ``Projection``; synapse types with the same (cell type, synapse) signature on both
    sides share one conductance. Gradients flow through the recurrent spikes only if
    ``recurrent_gradients``.

    Extensions for connectomes of many cell types (fly scale), which the reference's
    dense per-pair blocks and per-cell-type synapse types cannot hold: either side may be
    one ``SparseProjection`` instead of a dict, and a ``synapse_params`` entry may name
    several source cell types in ``cell_id`` (``synapses.SynapseRegistry``), so thousands
    of cell types share a few synapse types; ``unify_synapses`` is passed through.
    """

    def __init__(
        self,
        dt: float,
        rec_projections: dict,
        ff_projections: dict,
        cell_type_indices: np.ndarray,
        cell_type_indices_FF: np.ndarray,
        cell_params: list[dict],
        cell_params_FF: list[dict],
        synapse_params: list[dict],
        synapse_params_FF: list[dict],
        surrgrad_scale: float,
        batch_size: int,
        spike_mode: str = "deterministic",
        track_variables: bool = False,
        track_gradients: bool = False,
        track_batch_idx: int | None = None,
        storage_dtype=torch.float32,
        learn: dict | None = None,
        recurrent_gradients: bool = False,
        rec_stp: dict | None = None,
        ff_stp: dict | None = None,
        unify_synapses: bool = True,
    ):
        self.synapse_params = synapse_params
        self.cell_params_FF = cell_params_FF
        self.synapse_params_FF = synapse_params_FF
        self.n_synapse_types = len(synapse_params)
        self.n_cell_types_FF = len(cell_params_FF)
        self.n_inputs = int(cell_type_indices_FF.shape[0])
        super().__init__(
            dt=dt,
            cell_params=cell_params,
            cell_type_indices=cell_type_indices,
            sides=[
                InputSide(rec_projections, cell_params, synapse_params, cell_type_indices,
                          True, "rec_projections", "weights_mask", rec_stp),
                InputSide(ff_projections, cell_params_FF, synapse_params_FF,
                          cell_type_indices_FF, False, "ff_projections", "weights_mask_FF",
                          ff_stp),
            ],
            unify_synapses=unify_synapses,
            surrgrad_scale=surrgrad_scale,
            batch_size=batch_size,
            spike_mode=spike_mode,
            track_variables=track_variables,
            track_gradients=track_gradients,
            track_batch_idx=track_batch_idx,
            storage_dtype=storage_dtype,
            learn=learn,
        )  # fmt: skip
        self.register_buffer("cell_type_indices_FF", _long(cell_type_indices_FF))
        self.recurrent_gradients = recurrent_gradients
        self._engine = _engine_module()

    def forward(self, input_spikes):
        run = self._simulate(input_spikes)
        if not self.track_variables:
            return run.spikes
        S = len(self.registry)
        return {
            "spikes": run.spikes,
            "voltages": run.tracked["v"],
            "currents": run.tracked["I"][..., :S],
            "currents_leak": run.tracked["I"][..., S],
            "conductances": run.tracked["g"],
            **({"adaptation": run.tracked["a"]} if "a" in run.tracked else {}),
        }

    @property
    def weights(self) -> torch.Tensor:
        return self._weight_matrix(0)

    @property
    def weights_FF(self) -> torch.Tensor:
        return self._weight_matrix(1)

    @property
    def n_unified_synapse_types(self) -> int:
        return len(self.registry)


class FeedforwardConductanceLIFNetwork(ConductanceNetwork):
    """Conductance-based LIF neurons driven only by input rows
    (``conductance/feedforward.py:19-143``)."""

    state_name = "g_FF"

    def __init__(
        self,
        dt: float,
        projections: dict,
        cell_type_indices: np.ndarray,
        cell_type_indices_FF: np.ndarray,
        cell_params: list[dict],
        cell_params_FF: list[dict],
        synapse_params_FF: list[dict],
        surrgrad_scale: float,
        batch_size: int,
        spike_mode: str = "deterministic",
        track_variables: bool = False,
        track_gradients: bool = False,
        track_batch_idx: int | None = None,
        storage_dtype=torch.float32,
        return_probabilities: bool = False,
        learn: dict | None = None,
        stp: dict | None = None,
    ):
        self.cell_params_FF = cell_params_FF
        self.synapse_params_FF = synapse_params_FF
        self.n_cell_types_FF = len(cell_params_FF)
        self.n_synapse_types_FF = len(synapse_params_FF)
        self.n_inputs = int(cell_type_indices_FF.shape[0])
        self.return_probabilities = return_probabilities
        super().__init__(
            dt=dt,
            cell_params=cell_params,
            cell_type_indices=cell_type_indices,
            sides=[
                InputSide(projections, cell_params_FF, synapse_params_FF,
                          cell_type_indices_FF, False, "projections", "weights_mask_FF", stp),
            ],
            unify_synapses=False,
            surrgrad_scale=surrgrad_scale,
            batch_size=batch_size,
            spike_mode=spike_mode,
            track_variables=track_variables,
            track_gradients=track_gradients,
            track_batch_idx=track_batch_idx,
            storage_dtype=storage_dtype,
            learn=learn,
        )  # fmt: skip
        self.register_buffer("cell_type_indices_FF", _long(cell_type_indices_FF))
        self._engine = _engine_module()

    def forward(self, input_spikes):
        run = self._simulate(input_spikes, probabilities=self.return_probabilities)
        if self.track_variables:
            S = self.n_synapse_types_FF
            out = {
                "spikes": run.spikes,
                "voltages": run.tracked["v"],
                "currents_feedforward": run.tracked["I"][..., :S],
                "currents_leak": run.tracked["I"][..., S],
                "conductances_feedforward": run.tracked["g"],
                **({"adaptation": run.tracked["a"]} if "a" in run.tracked else {}),
            }
            if self.return_probabilities:
                out["probabilities"] = run.probabilities
            return out
        if self.return_probabilities:
            return run.probabilities, run.spikes
        return run.spikes

    @property
    def weights_FF(self) -> torch.Tensor:
        return self._weight_matrix(0)
