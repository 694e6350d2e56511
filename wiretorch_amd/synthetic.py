"""Seeded synthetic networks of the benchmark configurations.

Configurations 0, 1 and 3 are Erdős–Rényi conductance-LIF networks built through the
network API (``ConductanceLIFNetwork`` with per-(source type, target type)
projections). Configuration 2 — 140k neurons in 8000 cell types, ~50M synapses with a
power-law out-degree — cannot be expressed by the reference's dense per-pathway rows;
it is built directly as a compressed ``Drive`` (receptor kinds as pathways, per-type-pair
scaling factors folded into the weights) with its ``Physiology``.

Every random draw comes from ``numpy.random.default_rng`` streams seeded per
configuration (network ``[seed]``, input ``[seed, input_seed]``), as the reference's test
networks do (``tests/networks.py:263,271-273``); ``fingerprint`` hashes what defines a
network and its input (``tests/networks.py:963-970``). Physiology the configurations
leave open is fixed here:

* E_L = U_reset = -65 mV, g_L = 10 nS (C_m = tau_m g_L = 200 pF), tau_rise = 0 (a pure
  exponential conductance with peak g_bar; ``conductance_kernel`` gives peak 1);
* excitatory synapses tau_decay 5 ms, E_syn 0 mV; inhibitory 10 ms, -80 mV;
* weights are in units of g_bar = 1 nS.
"""

from __future__ import annotations

import hashlib
from dataclasses import dataclass

import numpy as np
import torch

from wiretorch_amd.connectome import Connectome, from_edges
from wiretorch_amd.network import (
    ConductanceLIFNetwork,
    Drive,
    Physiology,
    conductance_kernel,
)
from wiretorch_amd.projections import FrozenProjection, FullRankProjection, SignedProjection

E_L = -65.0
G_L = 10.0
THETA = -50.0
U_RESET = -65.0
TAU_MEM = 20.0
TAU_REF = 2.0


def lif_cells(tau_ref=TAU_REF):
    return [
        dict(name="E", cell_id=0, tau_mem=TAU_MEM, theta=THETA, U_reset=U_RESET, E_L=E_L,
             g_L=G_L, tau_ref=tau_ref),
        dict(name="I", cell_id=1, tau_mem=TAU_MEM, theta=THETA, U_reset=U_RESET, E_L=E_L,
             g_L=G_L, tau_ref=tau_ref),
    ]  # fmt: skip


SYNAPSES = [
    dict(name="exc", synapse_id=0, cell_id=0, tau_rise=0.0, tau_decay=5.0, E_syn=0.0, g_bar=1.0),
    dict(name="inh", synapse_id=1, cell_id=1, tau_rise=0.0, tau_decay=10.0, E_syn=-80.0, g_bar=1.0),
]  # fmt: skip
#: The input population makes the excitatory synapse: a type of its own (S = 3 with the
#: reference's unified registry, which keys synapse types by source cell type).
INPUT_CELLS = [dict(name="input", cell_id=0)]
INPUT_SYNAPSES = [
    dict(name="exc", synapse_id=0, cell_id=0, tau_rise=0.0, tau_decay=5.0, E_syn=0.0, g_bar=1.0),
]  # fmt: skip

#: Per (source, target) type scale of the lognormal(-1, 1) weights, for an in-degree of
#: 100 (configuration 0: about 20 Hz, irregular); other in-degrees scale it inversely.
PAIR_SCALE = {("E", "E"): 0.2, ("E", "I"): 0.2, ("I", "E"): 4.0, ("I", "I"): 4.0}


@dataclass
class Workload:
    """A built network (or drive and physiology), its input and how it was made."""

    name: str
    x: np.ndarray  # (B, T, n_in) bool
    structure: dict
    model: torch.nn.Module | None = None
    drive: Drive | None = None
    physiology: Physiology | None = None
    N: int = 0
    S: int = 0

    def fingerprint(self) -> str:
        return fingerprint(self.structure, self.x)


def fingerprint(structure: dict, x: np.ndarray) -> str:
    digest = hashlib.sha256()
    for key in sorted(structure):
        digest.update(key.encode())
        digest.update(np.ascontiguousarray(structure[key]).tobytes())
    digest.update(np.ascontiguousarray(x).tobytes())
    return digest.hexdigest()


def poisson(rng, B, T, rates_hz, dt):
    p = np.asarray(rates_hz, dtype=np.float64) * dt / 1000.0
    return rng.random((B, T, len(p))) < p


def er_network(*, N, frac_e, p, n_in, p_in, in_scale, rates_hz, B, T, dt, seed,
               input_seed=0, learnt=False, learn=None, surrgrad_scale=10.0,
               pair_scale=PAIR_SCALE) -> Workload:
    """Erdős–Rényi conductance-LIF network: lognormal(mu=-1, sigma=1) weights with
    connection probability ``p``, scaled per (source, target) type; ``n_in`` Poisson
    inputs at ``rates_hz`` connected with probability ``p_in`` and weights
    ``in_scale * lognormal(-1, 1)``."""
    rng = np.random.default_rng(seed)
    types = np.ones(N, dtype=np.int64)
    types[: round(frac_e * N)] = 0
    types = rng.permutation(types)
    names = ["E", "I"]
    w = rng.lognormal(-1.0, 1.0, (N, N)) * (rng.random((N, N)) < p)
    np.fill_diagonal(w, 0.0)
    for a, src in enumerate(names):
        for c, tgt in enumerate(names):
            w[np.ix_(types == a, types == c)] *= pair_scale[(src, tgt)]
    w = w.astype(np.float32)
    w_in = (in_scale * rng.lognormal(-1.0, 1.0, (n_in, N)) * (rng.random((n_in, N)) < p_in))
    w_in = w_in.astype(np.float32)
    rates = np.broadcast_to(np.asarray(rates_hz, dtype=np.float64), (n_in,))
    x = poisson(np.random.default_rng([seed, input_seed]), B, T, rates, dt)
    rec, ff = {}, {}
    in_types = np.zeros(n_in, dtype=np.int64)
    for a, src in enumerate(names):
        for c, tgt in enumerate(names):
            block = w[np.ix_(types == a, types == c)]
            rec[(src, tgt)] = (FullRankProjection(block, mask=block != 0) if learnt
                               else FrozenProjection(block))
    for c, tgt in enumerate(names):
        ff[("input", tgt)] = FrozenProjection(w_in[:, types == c])
    model = ConductanceLIFNetwork(
        dt=float(dt), rec_projections=rec, ff_projections=ff, cell_type_indices=types,
        cell_type_indices_FF=in_types, cell_params=lif_cells(), cell_params_FF=INPUT_CELLS,
        synapse_params=SYNAPSES, synapse_params_FF=INPUT_SYNAPSES,
        surrgrad_scale=surrgrad_scale, batch_size=B, learn=learn,
    )  # fmt: skip
    structure = dict(types=types, w=w, w_in=w_in, rates=rates.copy())
    return Workload("er", x, structure, model=model, N=N, S=len(model.registry))


def config0(seed=0, T=1000) -> Workload:
    """N 1000 (800 E / 200 I), ER p = 0.1, dt 0.1 ms, 100 Poisson inputs at 10 Hz with
    p = 0.2 input weights, batch 1."""
    wl = er_network(N=1000, frac_e=0.8, p=0.1, n_in=100, p_in=0.2, in_scale=8.0,
                    rates_hz=10.0, B=1, T=T, dt=0.1, seed=seed)
    wl.name = "config0"
    return wl


def config1(seed=1, T=5000, B=32) -> Workload:
    """N 10,000 (80/20), ER p = 0.02 (~2M synapses), 500 inputs at 5-20 Hz, batch 32."""
    rates = np.random.default_rng([seed, 99]).uniform(5.0, 20.0, 500)
    half = {k: 0.5 * v for k, v in PAIR_SCALE.items()}  # in-degree 200
    wl = er_network(N=10_000, frac_e=0.8, p=0.02, n_in=500, p_in=0.04, in_scale=8.0,
                    rates_hz=rates, B=B, T=T, dt=0.1, seed=seed, pair_scale=half)
    wl.name = "config1"
    return wl


def config3(seed=3, T=500, B=64, dt=1.0) -> Workload:
    """The training step's network: N 10,000 (80/20), ER p = 0.02 with per-synapse learnt
    weights (``FullRankProjection`` on the connectome), learnt per-type ``tau_mem`` and
    ``theta``, fast-sigmoid surrogate of slope 10, 500 inputs at 5-20 Hz, batch 64,
    T 500. dt is 1 ms (the configuration leaves it open): 500 ms, 25 bins of 20 ms for
    the rate loss (``binned_rate_loss``)."""
    rates = np.random.default_rng([seed, 99]).uniform(5.0, 20.0, 500)
    half = {k: 0.5 * v for k, v in PAIR_SCALE.items()}  # in-degree 200
    wl = er_network(N=10_000, frac_e=0.8, p=0.02, n_in=500, p_in=0.04, in_scale=8.0,
                    rates_hz=rates, B=B, T=T, dt=dt, seed=seed, pair_scale=half,
                    learnt=True, learn={"tau_mem": True, "theta": True},
                    surrgrad_scale=10.0)
    wl.name = "config3"
    return wl


def gamma_targets(seed: int, N: int, n_bins: int, shape=2.0, scale_hz=5.0) -> np.ndarray:
    """Target rates (Hz) per (bin, neuron), drawn from gamma(shape, scale)."""
    rng = np.random.default_rng([seed, 7])
    return rng.gamma(shape, scale_hz, (n_bins, N)).astype(np.float32)


def binned_rate_loss(spikes: torch.Tensor, target_hz: torch.Tensor, dt_ms: float,
                     bin_ms: float = 20.0) -> torch.Tensor:
    """Mean squared error between firing rates binned in ``bin_ms`` (Hz, averaged over the
    batch) and ``target_hz`` (n_bins, N); steps past the last whole bin are dropped."""
    B, T, N = spikes.shape
    per_bin = int(round(bin_ms / dt_ms))
    n_bins = T // per_bin
    rates = spikes[:, : n_bins * per_bin].reshape(B, n_bins, per_bin, N).mean(dim=(0, 2))
    rates = rates * (1000.0 / dt_ms)
    return ((rates - target_hz[:n_bins]) ** 2).mean()


# ---------------------------------------------------------------------------------
# Fly scale (configuration 2)
# ---------------------------------------------------------------------------------


def power_law_degrees(rng, n, exponent, k_min, k_max):
    """Discrete out-degrees from a power law ``P(k) ~ k^-exponent`` on [k_min, k_max]
    (inverse transform of the continuous law, rounded down)."""
    u = rng.random(n)
    a = 1.0 - exponent
    lo, hi = float(k_min) ** a, float(k_max + 1) ** a
    k = (lo + u * (hi - lo)) ** (1.0 / a)
    return np.floor(k).astype(np.int64)


def fly_scale(N=140_000, n_types=8000, exponent=2.1, mean_degree=357, k_max=8000,
              count_mean=4.0, frac_e_types=0.7, frac_sensory=0.05, rate_hz=10.0, B=8,
              T=2000, dt=0.1, seed=2, w_e=1.0, w_i=5.0, w_in=30.0, sf_sigma=0.5,
              device="cpu", input_seed=0) -> Workload:
    """Configuration 2: a synthetic fly-scale conductance-LIF network.

    Cell types are drawn uniformly per neuron; 70% of types are excitatory. Out-degrees
    follow the power law (``k_min`` solved so the mean is ``mean_degree``), targets are
    uniform (repeated draws of one pair merge into one synapse), synapse counts are
    geometric with mean ``count_mean``. A synapse's weight is its count times the
    scaling factor of its (source type, target type) pair — a lognormal(0, ``sf_sigma``)
    table of ``n_types``² entries, the quantity a model of this size would learn —
    times ``w_e`` / ``w_i`` by the source's receptor kind. A random 5% of neurons are
    sensory, each driven by its own Poisson channel (weight ``w_in``). The default
    weights were chosen by a sweep on the GPU for a stable, irregular state at the
    configuration's 10 Hz mean rate (9.3 Hz measured, 2% of neurons silent)."""
    cell_type, type_is_e, deg, tgt, counts, sf, sensory, x = _fly_draws(
        N, n_types, exponent, mean_degree, k_max, count_mean, frac_e_types, frac_sensory,
        rate_hz, B, T, dt, seed, input_seed, sf_sigma)
    is_e = type_is_e[cell_type]
    n_draws = int(deg.sum())

    dev = torch.device(device)
    src_t = torch.repeat_interleave(torch.arange(N, device=dev), torch.from_numpy(deg).to(dev))
    key = src_t * N + torch.from_numpy(tgt).to(dev)
    del src_t
    ct = torch.from_numpy(cell_type).to(dev)
    base = torch.where(torch.from_numpy(is_e).to(dev), torch.tensor(w_e, device=dev),
                       torch.tensor(w_i, device=dev))
    key, order = torch.sort(key)
    c = torch.from_numpy(counts).to(dev)[order]
    del order
    s_idx, t_idx = key // N, key % N
    w = c * torch.from_numpy(sf).to(dev)[ct[s_idx], ct[t_idx]] * base[s_idx]
    uniq, inverse = torch.unique_consecutive(key, return_inverse=True)
    merged = torch.zeros(uniq.numel(), dtype=torch.float64, device=dev)
    merged.index_add_(0, inverse, w.double())  # a few float32 terms: exact in float64
    del key, c, w, s_idx, t_idx, inverse
    src_u, tgt_u = uniq // N, uniq % N
    indptr = torch.zeros(N + 1, dtype=torch.int64, device=dev)
    indptr[1:] = torch.cumsum(torch.bincount(src_u, minlength=N), 0)
    rec = Connectome(N, N, indptr, tgt_u.to(torch.int32).contiguous(),
                     merged.float().contiguous(),
                     torch.from_numpy(np.where(is_e, 0, 1)).to(dev), 2)
    n_in = sensory.size
    ff = from_edges(n_in, N, np.arange(n_in), sensory, np.full(n_in, w_in, np.float32),
                    np.zeros(n_in, dtype=np.int64), 1, device=device)
    structure = dict(cell_type=cell_type, type_is_e=type_is_e, deg=deg, sensory=sensory,
                     n_draws=np.array([n_draws]), sf_row0=sf[0])
    drive, p = sparse_drive(rec, ff, N, dt, device)
    return Workload("config2", x, structure, drive=drive, physiology=p, N=N, S=2)


def _fly_draws(N, n_types, exponent, mean_degree, k_max, count_mean, frac_e_types,
               frac_sensory, rate_hz, B, T, dt, seed, input_seed, sf_sigma=0.5):
    """The random draws of configuration 2, in ``fly_scale``'s order (one stream)."""
    rng = np.random.default_rng(seed)
    cell_type = rng.integers(0, n_types, N)
    type_is_e = rng.random(n_types) < frac_e_types
    grid = np.arange(1, k_max + 1, dtype=np.float64)
    lo_k, hi_k = 1.0, float(mean_degree)
    for _ in range(60):  # k_min for the requested mean, by bisection on the law's mean
        mid = 0.5 * (lo_k + hi_k)
        ks = grid[grid >= mid]
        pk = ks ** -exponent
        if (ks * pk).sum() / pk.sum() < mean_degree:
            lo_k = mid
        else:
            hi_k = mid
    deg = power_law_degrees(rng, N, exponent, int(round(lo_k)), k_max)
    n_draws = int(deg.sum())
    tgt = rng.integers(0, N, n_draws, dtype=np.int64)
    counts = rng.geometric(1.0 / count_mean, n_draws).astype(np.float32)
    sf = rng.lognormal(0.0, sf_sigma, (n_types, n_types)).astype(np.float32)
    sensory = np.sort(rng.choice(N, int(round(frac_sensory * N)), replace=False))
    x = poisson(np.random.default_rng([seed, input_seed]), B, T, np.full(sensory.size, rate_hz), dt)
    return cell_type, type_is_e, deg, tgt, counts, sf, sensory, x


def fly_scale_network(N=140_000, n_types=8000, exponent=2.1, mean_degree=357, k_max=8000,
                      count_mean=4.0, frac_e_types=0.7, frac_sensory=0.05, rate_hz=10.0, B=8,
                      T=2000, dt=0.1, seed=2, w_e=1.0, w_i=5.0, w_in=30.0, sf_sigma=0.5,
                      learn_sf=False, device="cpu", input_seed=0) -> Workload:
    """Configuration 2 through the network API: a ``ConductanceLIFNetwork`` of ``n_types``
    cell types whose recurrent side is one ``SparseProjection`` — each synapse's count
    times the learnable scaling factor of its (source type, target type) pair — and whose
    input side connects each sensory channel to its neuron. The draws are
    ``fly_scale``'s; the receptor kinds' strengths ``w_e`` / ``w_i`` are the synapse
    types' ``g_bar`` (one ``synapse_params`` entry per kind, made by all cell types of that
    kind) instead of factors in the weights, so the dynamics equal ``fly_scale``'s up to
    rounding."""
    from wiretorch_amd.projections import SparseProjection

    cell_type, type_is_e, deg, tgt, counts, sf, sensory, x = _fly_draws(
        N, n_types, exponent, mean_degree, k_max, count_mean, frac_e_types, frac_sensory,
        rate_hz, B, T, dt, seed, input_seed, sf_sigma)
    dev = torch.device(device)
    src = torch.repeat_interleave(torch.arange(N, device=dev), torch.from_numpy(deg).to(dev))
    rec = SparseProjection(N, N, src, torch.from_numpy(tgt).to(dev),
                           torch.from_numpy(counts).to(dev), torch.from_numpy(cell_type),
                           torch.from_numpy(cell_type), sf=torch.from_numpy(sf),
                           learn_sf=learn_sf, n_source_types=n_types, n_target_types=n_types)
    del src
    n_in = sensory.size
    ff = SparseProjection(n_in, N, np.arange(n_in), sensory, np.full(n_in, w_in, np.float32),
                          np.zeros(n_in, dtype=np.int64), cell_type, sf=1.0,
                          n_source_types=1, n_target_types=n_types)
    cells = [dict(name=f"type{i}", cell_id=i, tau_mem=TAU_MEM, theta=THETA, U_reset=U_RESET,
                  E_L=E_L, g_L=G_L, tau_ref=TAU_REF) for i in range(n_types)]
    kinds = [np.flatnonzero(type_is_e).tolist(), np.flatnonzero(~type_is_e).tolist()]
    synapses = [
        dict(name="exc", synapse_id=0, cell_id=kinds[0], tau_rise=0.0, tau_decay=5.0,
             E_syn=0.0, g_bar=w_e),
        dict(name="inh", synapse_id=1, cell_id=kinds[1], tau_rise=0.0, tau_decay=10.0,
             E_syn=-80.0, g_bar=w_i),
    ]
    input_synapses = [dict(name="exc", synapse_id=0, cell_id=[0], tau_rise=0.0, tau_decay=5.0,
                           E_syn=0.0, g_bar=w_e)]
    model = ConductanceLIFNetwork(
        dt=float(dt), rec_projections=rec, ff_projections=ff, cell_type_indices=cell_type,
        cell_type_indices_FF=np.zeros(n_in, dtype=np.int64), cell_params=cells,
        cell_params_FF=[dict(name="sensory", cell_id=0)], synapse_params=synapses,
        synapse_params_FF=input_synapses, surrgrad_scale=10.0, batch_size=B,
    ).to(dev)  # fmt: skip
    structure = dict(cell_type=cell_type, type_is_e=type_is_e, deg=deg, sensory=sensory,
                     n_draws=np.array([int(deg.sum())]), sf_row0=sf[0])
    return Workload("config2", x, structure, model=model, N=N, S=len(model.registry))


def many_types(N=600, n_types=20, frac_e_types=0.7, p=0.1, n_in=60, p_in=0.2, rate_hz=20.0,
               B=2, T=200, dt=0.5, seed=11, input_seed=0, w_e=0.4, w_i=2.0, w_in=8.0,
               sparse=False, learn_sf=True) -> Workload:
    """A network of ``n_types`` cell types, more pathways than the kernels accumulate
    separately: ER connectivity ``p`` with geometric synapse counts (mean 2), one
    learnable scaling factor per (source type, target type) pair (lognormal(0, 0.3)
    start), excitatory or inhibitory by type, ``n_in`` Poisson inputs. Two receptor
    kinds, each one ``synapse_params`` entry listing its cell types (S = 2).

    ``sparse=False``: the reference's form, one ``ScalingFactorProjection`` per pair
    (``n_types`` recurrent pathways, folded by the engine); ``sparse=True``: the same
    network as one ``SparseProjection`` (folded by the network). Both forms give each
    synapse the weight ``count * sf`` (float32)."""
    from wiretorch_amd.projections import ScalingFactorProjection, SparseProjection

    rng = np.random.default_rng(seed)
    types = rng.integers(0, n_types, N)
    is_e = rng.random(n_types) < frac_e_types
    counts = (rng.geometric(0.5, (N, N)) * (rng.random((N, N)) < p)).astype(np.float32)
    np.fill_diagonal(counts, 0.0)
    sf = rng.lognormal(0.0, 0.3, (n_types, n_types)).astype(np.float32)
    w_inp = (rng.random((n_in, N)) < p_in).astype(np.float32)
    x = poisson(np.random.default_rng([seed, input_seed]), B, T, np.full(n_in, rate_hz), dt)
    names = [f"t{i}" for i in range(n_types)]
    cells = [dict(name=names[i], cell_id=i, tau_mem=TAU_MEM, theta=THETA, U_reset=U_RESET,
                  E_L=E_L, g_L=G_L, tau_ref=TAU_REF) for i in range(n_types)]
    synapses = [
        dict(name="exc", synapse_id=0, cell_id=np.flatnonzero(is_e).tolist(), tau_rise=0.0,
             tau_decay=5.0, E_syn=0.0, g_bar=w_e),
        dict(name="inh", synapse_id=1, cell_id=np.flatnonzero(~is_e).tolist(), tau_rise=0.0,
             tau_decay=10.0, E_syn=-80.0, g_bar=w_i),
    ]
    input_synapses = [dict(name="exc", synapse_id=0, cell_id=[0], tau_rise=0.0, tau_decay=5.0,
                           E_syn=0.0, g_bar=w_e)]
    if sparse:
        src, tgt = np.nonzero(counts)
        rec = SparseProjection(N, N, src, tgt, counts[src, tgt], types, types, sf=sf,
                               learn_sf=learn_sf, n_source_types=n_types,
                               n_target_types=n_types)
        s_in, t_in = np.nonzero(w_inp)
        ff = SparseProjection(n_in, N, s_in, t_in, w_in * w_inp[s_in, t_in],
                              np.zeros(n_in, dtype=np.int64), types, sf=1.0,
                              n_source_types=1, n_target_types=n_types)
    else:
        rec, ff = {}, {}
        for a in range(n_types):
            for c in range(n_types):
                block = counts[np.ix_(types == a, types == c)]
                if block.size and block.any():
                    rec[(names[a], names[c])] = ScalingFactorProjection(
                        block, init_sf=float(sf[a, c])) if learn_sf else FrozenProjection(
                        block * sf[a, c])
        for c in range(n_types):
            block = w_in * w_inp[:, types == c]
            if block.size and block.any():
                ff[("input", names[c])] = FrozenProjection(block)
    model = ConductanceLIFNetwork(
        dt=float(dt), rec_projections=rec, ff_projections=ff, cell_type_indices=types,
        cell_type_indices_FF=np.zeros(n_in, dtype=np.int64), cell_params=cells,
        cell_params_FF=[dict(name="input", cell_id=0)], synapse_params=synapses,
        synapse_params_FF=input_synapses, surrgrad_scale=10.0, batch_size=B,
    )  # fmt: skip
    structure = dict(types=types, is_e=is_e, counts=counts, sf=sf, w_inp=w_inp)
    return Workload("many_types", x, structure, model=model, N=N, S=len(model.registry))


def config2(T=2000, B=8, device="cpu", **kwargs) -> Workload:
    """Configuration 2 (fly scale) through the network API (``fly_scale_network``)."""
    return fly_scale_network(T=T, B=B, device=device, **kwargs)


def sparse_drive(rec: Connectome, ff: Connectome, N: int, dt: float, device="cpu",
                 surrgrad_scale=10.0):
    """Drive and physiology of a two-receptor network (excitatory, inhibitory) whose
    pathways are the receptor kinds: recurrent E, recurrent I, feedforward E."""
    made = torch.tensor([[True, False], [False, True], [True, False]], device=device)
    scale = torch.ones((3, N), device=device)
    drive = Drive(made=made, scale=scale, sparse_recurrent=rec, sparse_feedforward=ff)
    tau_rise = torch.zeros(2)
    tau_decay = torch.tensor([5.0, 10.0])
    g_bar = torch.ones(2)
    dt_t = torch.tensor(float(dt))
    f = lambda v: torch.full((N,), float(v), device=device)  # noqa: E731
    p = Physiology(
        theta=f(THETA), U_reset=f(U_RESET), E_L=f(E_L), C_m=f(TAU_MEM * G_L),
        beta=torch.exp(-dt_t / torch.full((N,), TAU_MEM)).to(device),
        E_syn=torch.tensor([0.0, -80.0], device=device),
        g_clip=torch.full((2,), float("inf"), device=device),
        decay=torch.exp(-dt_t / torch.stack((tau_rise, tau_decay))).to(device),
        jump=conductance_kernel(tau_rise, tau_decay, g_bar).to(device),
        dt=dt_t.to(device), surr_scale=torch.tensor(float(surrgrad_scale), device=device),
        n_ref=torch.round(torch.full((N,), TAU_REF) / dt_t).to(torch.int32).to(device),
    )  # fmt: skip
    return drive, p


def rest_state(B: int, N: int, S: int, device="cpu"):
    """``(v, g, counter)`` at rest: v = U_reset, g = 0 (``(B, N, 2, S)`` view of
    ``(B, 2, S, N)``), no refractory period left."""
    v = torch.full((B, N), U_RESET, device=device)
    g = torch.zeros((B, 2, S, N), device=device).permute(0, 3, 1, 2)
    counter = torch.zeros((B, N), dtype=torch.int32, device=device)
    return v, g, counter


# ---------------------------------------------------------------------------------
# Dense rate network (configuration 4)
# ---------------------------------------------------------------------------------

RATE_TAU_MEM = 10.0
RATE_DT = 1.0


def dense_rate(N=4096, n_in=64, B=256, T=1000, g2=1.5, dt=RATE_DT, seed=4, input_seed=0,
               storage_dtype=torch.bfloat16, learnt=True) -> Workload:
    """A dense recurrent rate network: one cell type ``r`` (``tau_mem`` 10 ms, tanh),
    synapses of time constant 0 (the voltage form: each step's current is that step's
    input), recurrent weights ``N(0, g2 / N)``, ``n_in`` Gaussian inputs (``N(0, 1)`` per
    step) through weights ``N(0, 1 / n_in)``. ``learnt``: both matrices are
    ``SignedProjection`` parameters (else fixed). ``dt`` 1 ms (the configuration leaves it
    open; 0.1 of ``tau_mem``)."""
    from wiretorch_amd.rate import RecurrentRateNetwork

    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, N)) * np.sqrt(g2 / N)).astype(np.float32)
    w_in = (rng.standard_normal((n_in, N)) * np.sqrt(1.0 / n_in)).astype(np.float32)
    x = np.random.default_rng([seed, input_seed]).standard_normal((B, T, n_in))
    x = x.astype(np.float32)
    make = SignedProjection if learnt else FrozenProjection
    cells = [dict(name="r", cell_id=0, tau_mem=RATE_TAU_MEM, nonlinearity="tanh")]
    synapses = [dict(name="exc", synapse_id=0, cell_id=0, tau_syn=0.0, type="excitatory")]
    model = RecurrentRateNetwork(
        dt=float(dt), rec_projections={("r", "r"): make(w)},
        ff_projections={("input", "r"): make(w_in)},
        cell_type_indices=np.zeros(N, dtype=np.int64),
        cell_type_indices_FF=np.zeros(n_in, dtype=np.int64), cell_params=cells,
        cell_params_FF=[dict(name="input", cell_id=0)], synapse_params=synapses,
        synapse_params_FF=[dict(synapses[0], name="exc_in")], batch_size=B,
        storage_dtype=storage_dtype,
    )  # fmt: skip
    structure = dict(w=w, w_in=w_in)
    return Workload("dense_rate", x, structure, model=model, N=N, S=len(model.registry))


def config4(seed=4, T=1000, B=256) -> Workload:
    """N 4,096 tanh rate neurons, dense bf16 recurrent weights ``N(0, 1.5/N)``, 64-dim
    Gaussian input through dense 4096 x 64 weights, batch 256, forward + backward."""
    wl = dense_rate(B=B, T=T, seed=seed)
    wl.name = "config4"
    return wl
