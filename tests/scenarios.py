"""The reference's seeded fixture networks, rebuilt through this package's API.

Restates the conductance-based and rate builders of the reference's ``tests/networks.py``
(physiology ``:57-98``, random structure ``:105-213``, ``recurrent`` ``:276-355``,
``feedforward`` ``:358-429``, rate networks ``:735-880``, scenarios ``:885-957``,
``fingerprint`` ``:963-970``, ``loss_readout`` ``:973-976``) and the drive/readout code
of ``tests/harness.py:11-111``.
The numpy random streams are consumed in the same order, so a rebuilt network's
SHA-256 fingerprint equals the one its fixture records (``meta["fingerprint"]``); every
fixture test checks that first.
"""

from __future__ import annotations

import hashlib
import json
from dataclasses import dataclass
from pathlib import Path
from typing import Callable

import numpy as np
import torch

from wiretorch_amd.network import ConductanceLIFNetwork, FeedforwardConductanceLIFNetwork
from wiretorch_amd.projections import (
    FullRankProjection,
    LowRankProjection,
    ScalingFactorProjection,
    make_frozen_projections,
)
from wiretorch_amd.rate import FeedforwardRateNetwork, RecurrentRateNetwork

FIXTURES = Path(__file__).parent / "golden" / "reference"
DT = 1.0
E, I = 0, 1
CELLS = [
    dict(name="excitatory", cell_id=E, tau_mem=85.0, theta=-38.0, U_reset=-60.0,
         E_L=-60.0, g_L=1.35),
    dict(name="inhibitory", cell_id=I, tau_mem=50.0, theta=-45.0, U_reset=-60.0,
         E_L=-60.0, g_L=0.9),
]  # fmt: skip
SYNAPSES = [
    dict(name="AMPA", synapse_id=0, cell_id=E, tau_rise=0.1, tau_decay=5.0,
         E_syn=0.0, g_bar=4.0, g_clip=40.0),
    dict(name="NMDA", synapse_id=1, cell_id=E, tau_rise=10.0, tau_decay=60.0,
         E_syn=0.0, g_bar=0.5, g_clip=4.0),
    dict(name="GABA_A", synapse_id=2, cell_id=I, tau_rise=0.5, tau_decay=6.0,
         E_syn=-70.0, g_bar=8.0, g_clip=80.0),
]  # fmt: skip
MITRAL_CELLS = [dict(name="mitral", cell_id=0)]
MITRAL_SYNAPSES = [
    dict(name="AMPA", synapse_id=0, cell_id=0, tau_rise=0.1, tau_decay=5.0,
         E_syn=0.0, g_bar=6.0, g_clip=40.0),
    dict(name="NMDA", synapse_id=1, cell_id=0, tau_rise=10.0, tau_decay=70.0,
         E_syn=0.0, g_bar=0.1, g_clip=4.0),
]  # fmt: skip
W_MEAN = {"mitral": 0.18, "excitatory": 0.3, "inhibitory": 1.8}
P_CONN = {"mitral": 0.3, "excitatory": 0.15, "inhibitory": 0.3}
SF_SPREAD = 0.15
RATE_HZ = {"mitral": 10.0, "excitatory": 8.0, "inhibitory": 25.0}
N, N_FF = 150, 80
REC_NAMES = [c["name"] for c in CELLS]
SEED = 2026
BATCH_SIZE = 2
WINDOW = 10
GRAD_STEPS = 100
READOUT_SEED = 7


def mg_block(synapses, mg):
    """``synapses`` with a Mg block of ``mg`` mM on the NMDA types (unchanged for None;
    reference ``tests/networks.py:113-117``)."""
    if mg is None:
        return synapses
    return [{**s, "mg": mg} if s["name"] == "NMDA" else s for s in synapses]


def adapting(cells, adapt, tau_adapt=200.0):
    """``cells`` whose excitatory type adapts by ``adapt`` per spike (unchanged for None;
    reference ``tests/networks.py:145-155``)."""
    if adapt is None:
        return cells
    return [{**c, "adapt": adapt, "tau_adapt": tau_adapt} if c["name"] == "excitatory" else c
            for c in cells]


def saturating(synapses, saturation):
    """``synapses`` with the NMDA types saturating by ``saturation`` (unchanged if None;
    reference ``tests/networks.py:120-127``)."""
    if saturation is None:
        return synapses
    return [{**s, "saturation": saturation} if s["name"] == "NMDA" else s for s in synapses]


def stp_pairs(sources, recurrent_names=("excitatory", "inhibitory")):
    """Depressing onto excitatory cells, facilitating onto inhibitory ones, per source
    type: a source type then has two STP sets, its rows shared by two pathways
    (reference ``tests/networks.py:130-143``)."""
    from wiretorch_amd.stp import DEPRESSING, FACILITATING

    excitatory, inhibitory = recurrent_names
    pairs = {}
    for source in sources:
        pairs[(source, excitatory)] = DEPRESSING
        pairs[(source, inhibitory)] = FACILITATING
    return pairs


def combined_physiology():
    cells = [dict(c) for c in MITRAL_CELLS]
    cells += [{**c, "cell_id": c["cell_id"] + 1} for c in CELLS]
    synapses = [dict(s) for s in MITRAL_SYNAPSES]
    synapses += [
        {**s, "cell_id": s["cell_id"] + 1, "synapse_id": s["synapse_id"] + 2}
        for s in SYNAPSES
    ]
    return cells, synapses


def with_refractory(cells, tau_ref):
    return cells if tau_ref is None else [{**c, "tau_ref": tau_ref} for c in cells]


def cell_types(rng, n, frac_e=0.8):
    types = np.full(n, I, dtype=np.int64)
    types[: round(frac_e * n)] = E
    return rng.permutation(types)


def sparse_lognormal(rng, n_src, n_tgt, p, mean, cv=1.0):
    sigma2 = np.log1p(cv**2)
    w = rng.lognormal(np.log(mean) - sigma2 / 2, np.sqrt(sigma2), (n_src, n_tgt))
    return (w * (rng.random((n_src, n_tgt)) < p)).astype(np.float32)


def weights_by_source(rng, source_names, n_tgt, p_scale=1.0):
    return np.concatenate(
        [sparse_lognormal(rng, 1, n_tgt, P_CONN[s] * p_scale, W_MEAN[s]) for s in source_names]
    )


def poisson(rng, batch, n_steps, rates_hz, dt=DT):
    p = np.asarray(rates_hz) * dt / 1000.0
    return rng.random((batch, n_steps, len(p))) < p


def move_scaling_factors(rng, projections):
    values = rng.lognormal(0.0, SF_SPREAD, len(projections))
    with torch.no_grad():
        for projection, value in zip(projections, values):
            projection.log_sf.fill_(float(np.log(value)))
    return values


def per_type_blocks(weights, src_types, tgt_types, src_names, tgt_names):
    out = {}
    for a, src in enumerate(src_names):
        for b, tgt in enumerate(tgt_names):
            rows, cols = np.flatnonzero(src_types == a), np.flatnonzero(tgt_types == b)
            if rows.size and cols.size:
                out[(src, tgt)] = weights[np.ix_(rows, cols)]
    return out


@dataclass(frozen=True)
class Built:
    model: torch.nn.Module
    input_spikes: np.ndarray
    structure: dict
    output: str = "spikes"  # what the model outputs per step: "spikes" or "rates"


@dataclass(frozen=True)
class Scenario:
    name: str
    build: Callable[[int], Built]
    state_keys: tuple[str, ...] = ()
    returns_probabilities: bool = False
    rates: bool = False


def _structure(seed, n=N, n_ff=N_FF):
    rng = np.random.default_rng(seed)
    types = cell_types(rng, n)
    names = [REC_NAMES[t] for t in types]
    w_rec = weights_by_source(rng, names, n, p_scale=N / n)
    w_ff = weights_by_source(rng, ["mitral"] * n_ff, n, p_scale=N_FF / n_ff)
    return rng, types, w_rec, w_ff


def _input_rng(seed, input_seed):
    return np.random.default_rng([seed, input_seed])


def recurrent(batch_size, seed, scaling_factors=False, n=N, n_ff=N_FF, n_steps=200,
              input_seed=0, learn=None, learnt_weights=False, tau_ref=None,
              recurrent_gradients=False, dt=DT, surrgrad_scale=5.0, mg=None, adapt=None,
              saturation=None, stp=False):
    """``ConductanceLIFNetwork``: frozen weights, perturbed scaling factors, or learnt
    recurrent weights; ``mg`` mM of Mg block on the NMDA types, ``adapt`` the excitatory
    cells' adaptation, ``saturation`` the NMDA types' and ``stp`` short-term plasticity
    of the excitatory and input sources (``"feedforward"``: of the input sources only)
    (reference ``tests/networks.py:276-355``)."""
    rng, types, w_rec, w_ff = _structure(seed, n, n_ff)
    ff_types = np.zeros(n_ff, dtype=np.int64)
    rec_blocks = per_type_blocks(w_rec, types, types, REC_NAMES, REC_NAMES)
    ff_blocks = per_type_blocks(w_ff, ff_types, types, ["mitral"], REC_NAMES)
    if learnt_weights:
        rec = {k: FullRankProjection(b, mask=b != 0) for k, b in rec_blocks.items()}
        ff = {k: ScalingFactorProjection(b) for k, b in ff_blocks.items()}
    elif scaling_factors:
        rec = {k: ScalingFactorProjection(b) for k, b in rec_blocks.items()}
        ff = {k: ScalingFactorProjection(b) for k, b in ff_blocks.items()}
    else:
        rec, ff = make_frozen_projections(w_rec, w_ff, types, ff_types, REC_NAMES, ["mitral"])
    model = ConductanceLIFNetwork(
        dt=dt, rec_projections=rec, ff_projections=ff,
        cell_type_indices=types, cell_type_indices_FF=ff_types,
        cell_params=adapting(with_refractory(CELLS, tau_ref), adapt), cell_params_FF=MITRAL_CELLS,
        synapse_params=saturating(mg_block(SYNAPSES, mg), saturation),
        synapse_params_FF=saturating(mg_block(MITRAL_SYNAPSES, mg), saturation),
        surrgrad_scale=surrgrad_scale, batch_size=batch_size, learn=learn,
        recurrent_gradients=recurrent_gradients,
        rec_stp=stp_pairs(["excitatory"]) if stp is True else None,
        ff_stp=stp_pairs(["mitral"]) if stp else None,
    )  # fmt: skip
    sfs = (
        move_scaling_factors(rng, [*rec.values(), *ff.values()])
        if scaling_factors
        else np.array([])
    )
    inputs = poisson(_input_rng(seed, input_seed), batch_size, n_steps,
                     [RATE_HZ["mitral"]] * n_ff, dt)
    return Built(model, inputs, dict(types=types, w_rec=w_rec, w_ff=w_ff, sf=sfs))


def feedforward(batch_size, seed, learnt_weights=False, probabilities=False, n=N,
                n_ff=N_FF, n_steps=200, input_seed=0, learn=None, tau_ref=None, mg=None,
                adapt=None, stp=False, saturation=None):
    """``FeedforwardConductanceLIFNetwork`` on external inputs and a recurrent network's
    neurons; ``mg`` as for ``recurrent`` (reference ``tests/networks.py:358-429``)."""
    rng, types, w_rec, w_ff = _structure(seed, n, n_ff)
    cells, synapses = combined_physiology()
    synapses = saturating(mg_block(synapses, mg), saturation)
    names = [c["name"] for c in cells]
    row_types = np.concatenate([np.zeros(n_ff, dtype=np.int64), types + 1])
    weights = np.concatenate([w_ff, w_rec])
    blocks = per_type_blocks(weights, row_types, types, names, REC_NAMES)
    projections, drawn = {}, {}
    for (src, tgt), block in blocks.items():
        if learnt_weights and src == "mitral":
            init = block * rng.lognormal(0.0, 0.2, block.shape)
            drawn[f"{src}->{tgt}"] = init
            projections[(src, tgt)] = FullRankProjection(init, mask=block != 0)
        elif learnt_weights and src == "excitatory":
            n_src, n_tgt = block.shape
            U = np.stack([np.ones(n_src), rng.normal(0, 0.3, n_src)], axis=1)
            V = np.stack([np.full(n_tgt, np.log(W_MEAN[src])), rng.normal(0, 0.3, n_tgt)])
            drawn[f"{src}->{tgt}.U"], drawn[f"{src}->{tgt}.V"] = U, V
            projections[(src, tgt)] = LowRankProjection(
                n_src, n_tgt, rank=2, U_init=U, V_init=V, mask=block != 0
            )
        else:
            projections[(src, tgt)] = ScalingFactorProjection(block)
    model = FeedforwardConductanceLIFNetwork(
        dt=DT, projections=projections, cell_type_indices=types,
        cell_type_indices_FF=row_types, cell_params=adapting(with_refractory(CELLS, tau_ref), adapt),
        cell_params_FF=cells, synapse_params_FF=synapses, surrgrad_scale=5.0,
        batch_size=batch_size, return_probabilities=probabilities, learn=learn,
        stp=stp_pairs(["mitral"]) if stp else None,
    )  # fmt: skip
    scaled = [p for p in projections.values() if isinstance(p, ScalingFactorProjection)]
    drawn["sf"] = move_scaling_factors(rng, scaled)
    rates = [RATE_HZ["mitral"]] * n_ff + [RATE_HZ[REC_NAMES[t]] for t in types]
    inputs = poisson(_input_rng(seed, input_seed), batch_size, n_steps, rates)
    return Built(model, inputs, dict(types=types, weights=weights, **drawn))


# Rate networks (reference ``tests/networks.py:735-880``): each cell type has its own
# nonlinearity; excitation makes a fast and a slow synapse type, inhibition an
# instantaneous one. The input is white noise.
RATE_CELLS = [
    dict(name="excitatory", cell_id=E, tau_mem=10.0, nonlinearity="softplus",
         theta=0.5, gain=1.0),
    dict(name="inhibitory", cell_id=I, tau_mem=5.0, nonlinearity="relu",
         theta=0.0, gain=2.0),
]  # fmt: skip
RATE_SYNAPSES = [
    dict(name="fast", synapse_id=0, cell_id=E, tau_syn=5.0, type="excitatory"),
    dict(name="slow", synapse_id=1, cell_id=E, tau_syn=50.0, type="excitatory"),
    dict(name="inh", synapse_id=2, cell_id=I, tau_syn=0.0, type="inhibitory"),
]
RATE_INPUT_CELLS = [dict(name="input", cell_id=0)]
RATE_INPUT_SYNAPSES = [
    dict(name="fast", synapse_id=0, cell_id=0, tau_syn=2.0, type="excitatory")
]
RATE_WEIGHTS = {E: 0.05, I: 0.15, "input": 0.05}
RATE_INPUT = (1.0, 1.0)
RATE_LEARN = {"tau_mem": True, "theta": ["excitatory"], "gain": True, "tau_syn": ["slow"]}


def white_noise(rng, batch, n_steps, n_inputs, mean=RATE_INPUT[0], std=RATE_INPUT[1]):
    return (mean + std * rng.standard_normal((batch, n_steps, n_inputs))).astype(np.float32)


def rate_recurrent(batch_size, seed, learn=None, n=N, n_ff=N_FF, n_steps=200, input_seed=0,
                   learnt_excitatory=False, storage_dtype=torch.float32):
    """``RecurrentRateNetwork`` with perturbed scaling factors; with ``learn`` also that
    physiology and full-rank input weights (reference ``tests/networks.py:767-828``)."""
    rng = np.random.default_rng([seed, 3])
    types = cell_types(rng, n)
    p_conn = {E: 0.15, I: 0.3}
    w_rec = np.concatenate(
        [sparse_lognormal(rng, 1, n, p_conn[t] * (N / n), RATE_WEIGHTS[t]) for t in types]
    )
    w_ff = sparse_lognormal(rng, n_ff, n, 0.3 * (N_FF / n_ff), RATE_WEIGHTS["input"])
    ff_types = np.zeros(n_ff, dtype=np.int64)
    rec = {
        (src, tgt): FullRankProjection(b, mask=b != 0)
        if learnt_excitatory and src == "excitatory"
        else ScalingFactorProjection(b)
        for (src, tgt), b in per_type_blocks(w_rec, types, types, REC_NAMES, REC_NAMES).items()
    }
    ff = {}
    for key, block in per_type_blocks(w_ff, ff_types, types, ["input"], REC_NAMES).items():
        if learn:
            init = block * rng.lognormal(0.0, 0.2, block.shape)
            ff[key] = FullRankProjection(init, mask=block != 0)
        else:
            ff[key] = ScalingFactorProjection(block)
    model = RecurrentRateNetwork(
        dt=DT, rec_projections=rec, ff_projections=ff, cell_type_indices=types,
        cell_type_indices_FF=ff_types, cell_params=RATE_CELLS,
        cell_params_FF=RATE_INPUT_CELLS, synapse_params=RATE_SYNAPSES,
        synapse_params_FF=RATE_INPUT_SYNAPSES, batch_size=batch_size, learn=learn,
        storage_dtype=storage_dtype,
    )  # fmt: skip
    scaled = [p for p in (*rec.values(), *ff.values()) if hasattr(p, "log_sf")]
    sfs = move_scaling_factors(np.random.default_rng([seed, 4]), scaled)
    inputs = white_noise(_input_rng(seed, input_seed), batch_size, n_steps, n_ff)
    structure = dict(types=types, w_rec=w_rec, w_ff=w_ff, sf=sfs)
    return Built(model, inputs, structure, output="rates")


def rate_feedforward(batch_size, seed, n=N, n_ff=N_FF, n_steps=200, input_seed=0):
    """``FeedforwardRateNetwork``: rows are white-noise inputs, then a ``rate_recurrent``
    network's neurons (reference ``tests/networks.py:831-877``)."""
    source = rate_recurrent(batch_size, seed, n=n, n_ff=n_ff)
    types, w_rec, w_ff = (source.structure[k] for k in ("types", "w_rec", "w_ff"))
    cells = RATE_INPUT_CELLS + [dict(name=c["name"], cell_id=c["cell_id"] + 1) for c in RATE_CELLS]
    synapses = RATE_INPUT_SYNAPSES + [
        {**s, "cell_id": s["cell_id"] + 1, "synapse_id": s["synapse_id"] + 1}
        for s in RATE_SYNAPSES
    ]
    row_types = np.concatenate([np.zeros(n_ff, dtype=np.int64), types + 1])
    blocks = per_type_blocks(np.concatenate([w_ff, w_rec]), row_types, types,
                             [c["name"] for c in cells], REC_NAMES)
    projections = {k: ScalingFactorProjection(b) for k, b in blocks.items()}
    model = FeedforwardRateNetwork(
        dt=DT, projections=projections, cell_type_indices=types,
        cell_type_indices_FF=row_types, cell_params=RATE_CELLS, cell_params_FF=cells,
        synapse_params_FF=synapses, batch_size=batch_size,
        learn={"theta": True, "tau_syn": ["slow"]},
    )  # fmt: skip
    sfs = move_scaling_factors(np.random.default_rng([seed, 5]), list(projections.values()))
    rng = _input_rng(seed, input_seed)
    inputs = np.concatenate(
        [
            white_noise(rng, batch_size, n_steps, n_ff),
            white_noise(rng, batch_size, n_steps, n, mean=1.0, std=0.5).clip(0),
        ],
        axis=2,
    )
    structure = dict(types=types, w_rec=w_rec, w_ff=w_ff, sf=sfs)
    return Built(model, inputs, structure, output="rates")


SCENARIOS = {
    s.name: s
    for s in [
        Scenario("recurrent_frozen", lambda b: recurrent(b, SEED), ("v", "g")),
        Scenario("recurrent_scaling_factors",
                 lambda b: recurrent(b, SEED, scaling_factors=True), ("v", "g")),
        Scenario("feedforward_scaling_factors", lambda b: feedforward(b, SEED), ("v", "g_FF")),
        Scenario("feedforward_learnt_weights",
                 lambda b: feedforward(b, SEED, learnt_weights=True), ("v", "g_FF")),
        Scenario("feedforward_probabilities",
                 lambda b: feedforward(b, SEED, probabilities=True), ("v", "g_FF"),
                 returns_probabilities=True),
    ]
}  # fmt: skip
#: The rate scenarios (reference ``tests/networks.py:915-932``), kept apart: the spiking
#: tests iterate over ``SCENARIOS``.
RATE_SCENARIOS = {
    s.name: s
    for s in [
        Scenario("rate_recurrent", lambda b: rate_recurrent(b, SEED), ("v", "I_syn"), rates=True),
        Scenario("rate_recurrent_learnt", lambda b: rate_recurrent(b, SEED, learn=RATE_LEARN),
                 ("v", "I_syn"), rates=True),
        Scenario("rate_feedforward", lambda b: rate_feedforward(b, SEED), ("v", "I_syn"),
                 rates=True),
    ]
}  # fmt: skip


def fingerprint(built: Built) -> str:
    digest = hashlib.sha256()
    for key in sorted(built.structure):
        digest.update(key.encode())
        digest.update(np.ascontiguousarray(built.structure[key]).tobytes())
    digest.update(np.ascontiguousarray(built.input_spikes).tobytes())
    return digest.hexdigest()


def loss_readout(seed, shape):
    rng = np.random.default_rng(seed)
    return torch.from_numpy(rng.normal(size=shape).astype(np.float32))


def load_fixture(name: str):
    """``(arrays, meta)`` of a reference fixture, spike trains unpacked
    (the format of the reference's ``tests/fixture_io.py:131-184``)."""
    with np.load(FIXTURES / f"{name}.npz", allow_pickle=False) as data:
        raw = {k: data[k] for k in data.files}
    meta = json.loads(str(raw.pop("meta")))
    arrays = {}
    for key, value in raw.items():
        if key.endswith(".bits"):
            stem = key[: -len(".bits")]
            shape = raw[f"{stem}.shape"]
            arrays[stem] = np.unpackbits(value, axis=-1, count=int(shape[-1])).astype(bool)
        elif not key.endswith(".shape"):
            arrays[key] = value
    return arrays, meta


def unpack_output(out, output: str = "spikes") -> dict:
    if isinstance(out, torch.Tensor):
        return {output: out}
    if isinstance(out, tuple):
        probabilities, spikes = out
        return {"spikes": spikes, "probabilities": probabilities}
    keep = ("spikes", "rates", "voltages", "probabilities")
    return {k: out[k] for k in keep if k in out}


def use_engine(model, engine) -> None:
    """Point a network at an engine module (the HIP engine, or the CPU oracle)."""
    model._engine = engine


def free_run(scenario: Scenario, built: Built, device="cpu") -> dict:
    """The full input in ``WINDOW``-step chunks, recording the state before each."""
    model = built.model.to(device)
    model.track_variables = bool(scenario.state_keys)
    model.track_batch_idx = None
    x = torch.from_numpy(built.input_spikes).to(device)
    chunks, states = [], {k: [] for k in scenario.state_keys}
    with torch.no_grad():
        for start in range(0, x.shape[1], WINDOW):
            for key, value in model.get_checkpoint_state().items():
                states[key].append(np.array(value))
            out = unpack_output(model(x[:, start : start + WINDOW]), built.output)
            chunks.append({k: v.cpu().numpy() for k, v in out.items()})
        for key, value in model.get_checkpoint_state().items():
            states[key].append(np.array(value))
    record = {k: np.concatenate([c[k] for c in chunks], axis=1) for k in chunks[0]}
    if "spikes" in record:
        record["spikes"] = record["spikes"] > 0.5
    record.update({f"state.{k}": np.stack(v) for k, v in states.items()})
    return record


def readout_loss(out: dict) -> torch.Tensor:
    loss = next(iter(out.values())).new_zeros(())
    for i, key in enumerate(("spikes", "hidden_spikes", "probabilities", "rates")):
        if key in out:
            R = loss_readout(READOUT_SEED + i, tuple(out[key].shape))
            loss = loss + (out[key] * R.to(out[key].device)).sum()
    return loss


def gradients(built: Built, device="cpu", track=False, steps=GRAD_STEPS):
    """Backpropagate ``readout_loss`` through the first ``steps`` steps."""
    model = built.model.to(device)
    model.track_variables = track
    if track:
        model.track_batch_idx = 0
    x = torch.from_numpy(built.input_spikes[:, :steps]).to(device)
    loss = readout_loss(unpack_output(model(x), built.output))
    loss.backward()
    grads = {
        name: p.grad.detach().cpu().numpy()
        for name, p in model.named_parameters()
        if p.grad is not None
    }
    return float(loss.detach()), grads
