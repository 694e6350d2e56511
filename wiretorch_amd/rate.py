"""Rate networks: the current-based LIF network with a nonlinearity for the spike.

Host side of the rate family, the counterpart of the reference's
``src/wiretorch/network_simulators/rate/`` (``network.py:1-178``, ``recurrent.py``,
``feedforward.py``) on this package's ``ProjectionNetwork``: per call, a ``Drive``
(pathways, weights, kernel scale, synapse types made) and a ``RatePhysiology`` for
``rate_engine.simulate``. One step, for every neuron of every trial
(``rate/dynamics.py:1-30``):

1. output the rate of the voltage entering the step, ``r = gain f(v - theta)``;
2. filter each synaptic current towards this step's input,
   ``I <- alpha I + (1 - alpha) sum_k a_k scale_k made_k``, with ``a_k`` the recurrent
   rates times weights, or the input times weights;
3. integrate ``v <- beta v + (1 - beta) sum_s sign_s I_s``.

``alpha = exp(-dt / tau_syn)`` and ``beta = exp(-dt / tau_mem)`` are recomputed every
call (the time constants may be learnt); a time constant of 0 makes its variable follow
its input. ``storage_dtype`` is what the engine multiplies rates and recurrent weights
in (accumulating in float32): float32, or bfloat16 / float16 on the matrix cores.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from wiretorch_amd.network import InputSide, ProjectionNetwork, _long
from wiretorch_amd.type_parameters import TypeParameters, learnt_synapses, learnt_types

#: The nonlinearities ``f`` a cell type can use, by code (``rate/dynamics.py:63-69``).
NONLINEARITIES = ("relu", "softplus", "sigmoid", "tanh")
CELL_PARAMETERS = ("cell_id", "name", "tau_mem", "nonlinearity")
SYNAPSE_PARAMETERS = ("synapse_id", "cell_id", "name", "tau_syn", "type")
THETA, GAIN = 0.0, 1.0
LEARNABLE_CELL = ("tau_mem", "theta", "gain")
LEARNABLE_SYNAPSE = ("tau_syn",)
STORAGE_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


@dataclass
class RatePhysiology:
    """Every parameter of the rate dynamics (``rate/dynamics.py:72-92``).

    Per neuron ``(N,)``: ``theta``, ``gain``, ``beta``; per synapse type ``(S,)``:
    ``sign`` (+1 / -1) and ``decay``. ``groups`` lists each cell type's nonlinearity
    name and neurons; ``nonlinearity`` ``(N,)`` int8 holds each neuron's code in
    ``NONLINEARITIES``.
    """

    theta: torch.Tensor
    gain: torch.Tensor
    beta: torch.Tensor
    sign: torch.Tensor
    decay: torch.Tensor
    groups: list
    nonlinearity: torch.Tensor
    storage_dtype: torch.dtype = torch.float32


def _check_parameters(params: list[dict], required, what: str) -> None:
    for p in params:
        missing = [k for k in required if k not in p]
        assert not missing, f"{what}: {p.get('name', p)} lacks {missing}"


class RateNetwork(ProjectionNetwork):
    """Base of the rate networks (``rate/network.py:35-178``): per cell type ``tau_mem``,
    ``theta``, ``gain`` and a nonlinearity; per synapse type ``tau_syn`` and a sign
    (``type``: excitatory +1, inhibitory -1). ``learn`` trains any of ``tau_mem``,
    ``theta``, ``gain`` (per cell type) and ``tau_syn`` (per synapse type). The state
    ``v`` ``(B, N)`` and currents ``I_syn`` ``(B, N, S)`` (stored ``(B, S, N)``) continue
    across calls until ``reset_state``."""

    state_name = "I_syn"
    output_name = "r"

    def __init__(self, *, cell_params, sides, learn, storage_dtype=torch.float32, **kwargs):
        _check_parameters(cell_params, CELL_PARAMETERS, "cell_params")
        for cell in cell_params:
            assert cell["nonlinearity"] in NONLINEARITIES, (
                f"cell type {cell['name']!r}: nonlinearity must be one of "
                f"{sorted(NONLINEARITIES)}, got {cell['nonlinearity']!r}"
            )
            assert cell["tau_mem"] >= 0, f"cell type {cell['name']!r}: negative tau_mem"
        for side in sides:
            _check_parameters(side.synapse_params, SYNAPSE_PARAMETERS, side.attribute)
            for synapse in side.synapse_params:
                assert synapse["type"] in ("excitatory", "inhibitory"), (
                    f"{side.attribute}: synapse type must be 'excitatory' or "
                    f"'inhibitory', got {synapse['type']!r}"
                )
                assert synapse["tau_syn"] >= 0, (
                    f"{side.attribute}: tau_syn must be >= 0, got {synapse['tau_syn']}"
                )
        unknown = set(learn or {}) - set(LEARNABLE_CELL) - set(LEARNABLE_SYNAPSE)
        assert not unknown, (
            f"learn: unknown parameters {sorted(unknown)}; "
            f"can learn {LEARNABLE_CELL + LEARNABLE_SYNAPSE}"
        )
        super().__init__(cell_params=cell_params, sides=sides, learn=learn,
                         storage_dtype=storage_dtype, **kwargs)
        self._engine = _rate_engine_module()

    @property
    def storage_dtype(self) -> torch.dtype:
        return self._storage_dtype

    @storage_dtype.setter
    def storage_dtype(self, dtype) -> None:
        dtype = getattr(torch, dtype) if isinstance(dtype, str) else dtype
        if dtype not in STORAGE_DTYPES:
            raise ValueError(f"storage dtype {dtype} not supported (supported: {STORAGE_DTYPES})")
        self._storage_dtype = dtype

    def _register_physiology(self) -> None:
        cells = sorted(self.cell_params, key=lambda c: c["cell_id"])
        names = [c["name"] for c in cells]
        self.cell_parameters = TypeParameters(
            {
                "tau_mem": [c["tau_mem"] for c in cells],
                "theta": [c.get("theta", THETA) for c in cells],
                "gain": [c.get("gain", GAIN) for c in cells],
            },
            learnt={
                name: learnt_types(self.learn.get(name), names, f"learn[{name!r}]")
                for name in LEARNABLE_CELL
            },
            positive={"tau_mem", "gain"},
        )
        synapses = self.registry.synapses
        self.synapse_parameters = TypeParameters(
            {"tau_syn": [s["tau_syn"] for s in synapses]},
            learnt={
                "tau_syn": learnt_synapses(
                    self.learn.get("tau_syn"), synapses, "learn['tau_syn']"
                ),
            },
            positive={"tau_syn"},
        )
        self.register_buffer(
            "sign",
            torch.tensor([1.0 if s["type"] == "excitatory" else -1.0 for s in synapses]),
        )
        self.nonlinearities = [c["nonlinearity"] for c in cells]
        codes = np.array([NONLINEARITIES.index(n) for n in self.nonlinearities], dtype=np.int8)
        types = self.cell_type_indices.cpu().numpy()
        self.register_buffer("_nonlinearity", torch.from_numpy(codes[types]), persistent=False)
        for cell_type in range(len(cells)):
            neurons = (self.cell_type_indices == cell_type).nonzero(as_tuple=True)[0]
            self.register_buffer(f"_neurons_{cell_type}", neurons, persistent=False)

    def _set_timestep(self) -> None:
        pass  # the decays are computed in each call, as they may be learnt

    def _physiology(self) -> RatePhysiology:
        """``rate/network.py:151-166``."""
        types = self.cell_type_indices
        cell = self.cell_parameters
        return RatePhysiology(
            theta=cell.value("theta")[types],
            gain=cell.value("gain")[types],
            beta=torch.exp(-self.dt / cell.value("tau_mem"))[types],
            sign=self.sign,
            decay=torch.exp(-self.dt / self.synapse_parameters.value("tau_syn")),
            groups=[
                (name, getattr(self, f"_neurons_{cell_type}"))
                for cell_type, name in enumerate(self.nonlinearities)
            ],
            nonlinearity=self._nonlinearity,
            storage_dtype=self.storage_dtype,
        )

    def _initial_state(self):
        """Voltages and currents zero; currents ``(B, N, S)`` laid out ``(B, S, N)``
        (``rate/network.py:168-174``)."""
        v = torch.zeros((self.batch_size, self.n_neurons), device=self.device)
        I = torch.zeros(
            (self.batch_size, len(self.registry), self.n_neurons), device=self.device
        ).permute(0, 2, 1)
        return v, I

    def _side_currents(self, I: torch.Tensor, side: int) -> torch.Tensor:
        """The currents ``(..., S_side)`` of the synapse types one input side makes."""
        index = sorted(set(self.registry.to_index[side].values()))
        return I[..., index]


class RecurrentRateNetwork(RateNetwork):
    """Recurrent rate network (``rate/recurrent.py:13-154``): neurons receive input from
    each other through ``rec_projections`` and from outside through ``ff_projections``,
    ``{(source type, target type): Projection}``."""

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
        batch_size: int,
        learn: dict | None = None,
        track_variables: bool = False,
        track_gradients: bool = False,
        track_batch_idx: int | None = None,
        storage_dtype=torch.float32,
    ):
        self.synapse_params = synapse_params
        self.cell_params_FF = cell_params_FF
        self.synapse_params_FF = synapse_params_FF
        self.n_cell_types_FF = len(cell_params_FF)
        self.n_inputs = int(cell_type_indices_FF.shape[0])
        super().__init__(
            dt=dt,
            cell_params=cell_params,
            cell_type_indices=cell_type_indices,
            sides=[
                InputSide(rec_projections, cell_params, synapse_params, cell_type_indices,
                          True, "rec_projections", "weights_mask"),
                InputSide(ff_projections, cell_params_FF, synapse_params_FF,
                          cell_type_indices_FF, False, "ff_projections", "weights_mask_FF"),
            ],
            unify_synapses=True,
            batch_size=batch_size,
            learn=learn,
            track_variables=track_variables,
            track_gradients=track_gradients,
            track_batch_idx=track_batch_idx,
            storage_dtype=storage_dtype,
        )  # fmt: skip
        self.register_buffer("cell_type_indices_FF", _long(cell_type_indices_FF))

    def forward(self, inputs):
        """Rates ``(B, T, N)``; with ``track_variables`` a dict of ``rates``, ``voltages``,
        ``currents`` and the currents split by side (``rate/recurrent.py:108-131``)."""
        run = self._simulate(inputs)
        if not self.track_variables:
            return run.output
        I = run.tracked["I"]
        return {
            "rates": run.output,
            "voltages": run.tracked["v"],
            "currents": I,
            "currents_recurrent": self._side_currents(I, 0),
            "currents_feedforward": self._side_currents(I, 1),
        }

    @property
    def weights(self) -> torch.Tensor:
        return self._weight_matrix(0)

    @property
    def weights_FF(self) -> torch.Tensor:
        return self._weight_matrix(1)

    @property
    def scaling_factors(self) -> torch.Tensor:
        return self._scaling_matrix(0)

    @property
    def scaling_factors_FF(self) -> torch.Tensor:
        return self._scaling_matrix(1)

    @property
    def unified_synapse_params(self) -> list[dict]:
        return self.registry.synapses


class FeedforwardRateNetwork(RateNetwork):
    """Rate neurons driven only by input rows (``rate/feedforward.py:13-100``)."""

    def __init__(
        self,
        dt: float,
        projections: dict,
        cell_type_indices: np.ndarray,
        cell_type_indices_FF: np.ndarray,
        cell_params: list[dict],
        cell_params_FF: list[dict],
        synapse_params_FF: list[dict],
        batch_size: int,
        learn: dict | None = None,
        track_variables: bool = False,
        track_gradients: bool = False,
        track_batch_idx: int | None = None,
        storage_dtype=torch.float32,
    ):
        self.cell_params_FF = cell_params_FF
        self.synapse_params_FF = synapse_params_FF
        self.n_cell_types_FF = len(cell_params_FF)
        self.n_inputs = int(cell_type_indices_FF.shape[0])
        super().__init__(
            dt=dt,
            cell_params=cell_params,
            cell_type_indices=cell_type_indices,
            sides=[
                InputSide(projections, cell_params_FF, synapse_params_FF,
                          cell_type_indices_FF, False, "projections", "weights_mask_FF"),
            ],
            unify_synapses=False,
            batch_size=batch_size,
            learn=learn,
            track_variables=track_variables,
            track_gradients=track_gradients,
            track_batch_idx=track_batch_idx,
            storage_dtype=storage_dtype,
        )  # fmt: skip
        self.register_buffer("cell_type_indices_FF", _long(cell_type_indices_FF))

    def forward(self, inputs):
        run = self._simulate(inputs)
        if not self.track_variables:
            return run.output
        return {"rates": run.output, "voltages": run.tracked["v"], "currents": run.tracked["I"]}

    @property
    def weights_FF(self) -> torch.Tensor:
        return self._weight_matrix(0)

    @property
    def scaling_factors_FF(self) -> torch.Tensor:
        return self._scaling_matrix(0)


def _rate_engine_module():
    from wiretorch_amd import rate_engine

    return rate_engine
