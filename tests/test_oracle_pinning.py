"""Checks that pin the oracle where the recorded fixtures leave it open.

The fixtures (``test_oracle_fixtures.py``) cover networks without a refractory period and
with the dense propagation form. What they leave open is fixed here by what the
mathematics or the reference's own tests fix, each chosen so that a plausible mistake in
the restatement (a dropped term, a wrong sign, a transposed index) fails:

* the exponential-Euler voltage step against the exact solution of the linear ODE
  (reference ``tests/test_membrane_step.py:36-59``) and its bounds;
* the surrogate spike's known answer (reference ``tests/test_training_utils.py:31-36``);
* refractory timing of single neurons in closed form (reference
  ``tests/test_refractory.py:85-124``);
* compressed propagation (``oracle.sparse``) against a brute-force dense float64 product;
* the rate oracle's reduced-precision product: the plain product on operands that are
  already representable, and which operands and gradients it rounds otherwise.

The refractory closed forms also run on the GPU engine (marked ``gpu``).
"""

import math

import numpy as np
import pytest
import torch

import oracle.dynamics as oracle_engine
import oracle.sparse as oracle_sparse
import scenarios as sc
from wiretorch_amd import connectome
from wiretorch_amd.network import ConductanceLIFNetwork, Physiology
from wiretorch_amd.projections import FrozenProjection

TAU, G_L, E_L, DT = 20.0, 2.0, -65.0, 0.5
E_SYN = torch.tensor([0.0, -80.0])


def _physiology(g_clip=math.inf):
    n = torch.ones(1)
    return Physiology(
        theta=n * 1e9, U_reset=n * E_L, E_L=n * E_L, C_m=n * TAU * G_L,
        beta=n * math.exp(-DT / TAU), E_syn=E_SYN, g_clip=torch.full((2,), g_clip),
        decay=torch.ones(2, 2), jump=torch.zeros(2, 2), dt=torch.tensor(DT),
        surr_scale=torch.tensor(1.0),
    )  # fmt: skip


@pytest.mark.parametrize("G", [(0.0, 0.0), (3.0, 1.0), (1e6, 0.0), (2e5, 5e5), (0.0, 7.0)])
@pytest.mark.parametrize("v0", [-50.0, -72.0])
def test_membrane_step_is_the_exact_solution(G, v0):
    """With conductances held over the step, ``C_m dv/dt = -g_tot (v - V_inf)``: ``v``
    relaxes towards ``V_inf`` by ``exp(-dt g_tot / C_m)``, never past it."""
    v = torch.tensor([[v0]])
    g = torch.zeros(1, 1, 2, 2)
    g[0, 0, 1] = torch.tensor(G)
    v_next, I, I_leak = oracle_engine.membrane(v, torch.zeros(1, 1), g, _physiology())
    g_tot = G_L + sum(G)
    V_inf = (G_L * E_L + sum(gk * e for gk, e in zip(G, E_SYN.tolist()))) / g_tot
    expected = V_inf + (v0 - V_inf) * math.exp(-DT * g_tot / (TAU * G_L))
    assert v_next.item() == pytest.approx(expected, rel=1e-6, abs=1e-4)
    assert I_leak.item() == pytest.approx(G_L * (v0 - E_L), rel=1e-6)
    np.testing.assert_allclose(I[0, 0].numpy(), [G[0] * (v0 - 0.0), G[1] * (v0 + 80.0)],
                               rtol=1e-6)
    lo, hi = sorted([v0, V_inf])
    assert lo - 1e-4 <= v_next.item() <= hi + 1e-4


def test_membrane_step_resets_and_clips():
    """A spiking neuron goes to ``U_reset``; ``g_clip`` caps each summed conductance,
    and negative sums count as zero."""
    p = _physiology(g_clip=4.0)
    p.U_reset = torch.tensor([-70.0])
    v = torch.tensor([[-50.0, -50.0]])
    p.theta, p.E_L, p.C_m, p.beta = (t.expand(2) for t in (p.theta, p.E_L, p.C_m, p.beta))
    p.U_reset = p.U_reset.expand(2)
    g = torch.zeros(1, 2, 2, 2)
    g[0, :, 1, 0] = torch.tensor([100.0, -3.0])
    v_next, I, _ = oracle_engine.membrane(v, torch.tensor([[1.0, 0.0]]), g, p)
    assert v_next[0, 0].item() == -70.0
    assert I[0, 0, 0].item() == pytest.approx(4.0 * -50.0)
    assert I[0, 1, 0].item() == 0.0
    leak_only = E_L + 15.0 * math.exp(-DT / TAU)
    assert v_next[0, 1].item() == pytest.approx(leak_only, rel=1e-6)


def test_surrogate_spike_known_answer():
    x = torch.tensor([-1.0, 0.0, 0.5], requires_grad=True)
    s = oracle_engine.SurrGradSpike.apply(x, torch.tensor(2.0))
    assert s.tolist() == [0.0, 0.0, 1.0]
    s.sum().backward()
    torch.testing.assert_close(x.grad, 1 / (2 * x.detach().abs() + 1) ** 2)


THETA, RESET = -50.0, {"below": -60.0, "above": -40.0}


def _single(regime, tau_ref, n=3, batch=2):
    """``n`` uncoupled neurons with refractory period ``tau_ref``; with the reset below
    threshold the input is strong enough to make them spike whenever they can."""
    cell = dict(name="e", cell_id=0, tau_mem=20.0, theta=THETA, U_reset=RESET[regime],
                tau_ref=tau_ref, E_L=-60.0, g_L=10.0)
    synapse = dict(tau_rise=0.1, tau_decay=1.0, E_syn=0.0, g_bar=1.0)
    model = ConductanceLIFNetwork(
        dt=1.0,
        rec_projections={("e", "e"): FrozenProjection(np.zeros((n, n)))},
        ff_projections={("in", "e"): FrozenProjection(
            np.full((1, n), 1000.0 if regime == "below" else 0.0))},
        cell_type_indices=np.zeros(n, dtype=np.int64),
        cell_type_indices_FF=np.zeros(1, dtype=np.int64),
        cell_params=[cell],
        cell_params_FF=[dict(name="in", cell_id=0)],
        synapse_params=[dict(synapse_id=0, cell_id=0, name="rec", **synapse)],
        synapse_params_FF=[dict(synapse_id=0, cell_id=0, name="ff", **synapse)],
        surrgrad_scale=5.0,
        batch_size=batch,
        track_variables=True,
    )  # fmt: skip
    return model, torch.ones((batch, 40, 1))


def _check_refractory_trains(spikes, voltages, regime, tau_ref):
    """After each spike, ``n_ref`` steps at reset without a spike; a neuron reset below
    threshold spikes again after ``n_ref + 2`` steps, one reset above it after
    ``n_ref + 1``."""
    n_ref = round(tau_ref)
    expected = n_ref + (2 if regime == "below" else 1)
    trains = spikes.permute(0, 2, 1).reshape(-1, 40)
    for train, v in zip(trains, voltages.permute(0, 2, 1).reshape(-1, 40)):
        times = torch.nonzero(train).flatten()
        assert len(times) >= 40 // expected - 1
        assert (torch.diff(times) == expected).all(), times
        for t in times[:-1]:
            held = v[t : t + n_ref + 1]
            assert (held == RESET[regime]).all(), (t, held)


def _run_single(regime, tau_ref, engine, device):
    model, x = _single(regime, tau_ref)
    model.to(device)
    sc.use_engine(model, engine)
    with torch.no_grad():
        out = model(x.to(device))
    return out["spikes"].cpu(), out["voltages"].cpu()


@pytest.mark.parametrize("tau_ref", [0.0, 1.0, 4.0])
@pytest.mark.parametrize("regime", ["below", "above"])
def test_refractory_spike_times_and_held_voltages(regime, tau_ref):
    spikes, voltages = _run_single(regime, tau_ref, oracle_engine, "cpu")
    _check_refractory_trains(spikes, voltages, regime, tau_ref)


@pytest.mark.gpu
@pytest.mark.parametrize("tau_ref", [0.0, 1.0, 4.0])
@pytest.mark.parametrize("regime", ["below", "above"])
def test_refractory_spike_times_on_gpu(regime, tau_ref):
    from wiretorch_amd import engine

    spikes, voltages = _run_single(regime, tau_ref, engine, "cuda")
    _check_refractory_trains(spikes, voltages, regime, tau_ref)
    ref_s, ref_v = _run_single(regime, tau_ref, oracle_engine, "cpu")
    assert torch.equal(spikes, ref_s)
    torch.testing.assert_close(voltages, ref_v, rtol=1e-5, atol=1e-5 * 65)


def test_tau_ref_in_whole_steps():
    """``n_ref = round(tau_ref / dt)``, recomputed with the time step; a period that
    rounds to zero steps is no period at all."""
    model, _ = _single("below", 3.0)
    assert model.n_ref.tolist() == [3, 3, 3] and model._refractory
    assert model._physiology().n_ref is not None
    model.set_timestep(0.5)
    assert model.n_ref.tolist() == [6, 6, 6]
    model, _ = _single("below", 0.4)
    assert model.n_ref.tolist() == [0, 0, 0] and not model._refractory
    assert model._physiology().n_ref is None


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_sparse_activations_equal_the_dense_product(seed):
    """Each target's activation in pathway ``k`` is the exactly rounded sum of the
    weights from that pathway's spiking sources: equal to the dense float64 product
    over those sources, rounded once (weights of one magnitude, so the float64 sums
    are exact)."""
    rng = np.random.default_rng(seed)
    n_src, n_tgt, n_path, B = 60, 30, 3, 5
    W = (rng.random((n_src, n_tgt)) < 0.3) * rng.uniform(0.5, 1.0, (n_src, n_tgt))
    W = W.astype(np.float32)
    pathway = rng.integers(0, n_path, n_src)
    conn = connectome.from_dense(torch.from_numpy(W), torch.from_numpy(pathway), n_path)
    s = (rng.random((B, n_src)) < 0.4).astype(np.float32)
    got = oracle_sparse.activations(conn, torch.from_numpy(s))
    assert got.dtype == torch.float32 and got.shape == (n_path, B, n_tgt)
    for k in range(n_path):
        rows = pathway == k
        expected = s[:, rows].astype(np.float64) @ W[rows].astype(np.float64)
        np.testing.assert_array_equal(got[k].numpy(), expected.astype(np.float32))


@pytest.mark.parametrize("seed", [0, 1])
def test_exact_dense_product_is_the_exactly_rounded_sum(seed, monkeypatch):
    """``oracle.dynamics.product`` with ``SUMS = "exact"``: each entry equals the
    exactly rounded sum of its terms — ``math.fsum`` (exact, then rounded once) on a
    brute-force loop — and the event-by-event ``oracle.sparse`` propagation bit for bit,
    on lognormal weights like the configurations'; the float32 product stays within its
    own error bound of it."""
    import math

    import oracle.dynamics as od

    monkeypatch.setattr(od, "SUMS", "exact")
    rng = np.random.default_rng(seed)
    n_src, n_tgt, B = 300, 40, 4
    W = (rng.lognormal(-1.0, 1.0, (n_src, n_tgt)) * (rng.random((n_src, n_tgt)) < 0.2))
    W = W.astype(np.float32)
    s = (rng.random((B, n_src)) < 0.3).astype(np.float32)
    got = od.product(torch.from_numpy(s), torch.from_numpy(W)).numpy()
    for b in range(B):
        for n in range(n_tgt):
            terms = [float(W[j, n]) for j in range(n_src) if s[b, j]]
            assert got[b, n] == np.float32(math.fsum(terms)), (b, n)
    conn = connectome.from_dense(torch.from_numpy(W), torch.zeros(n_src, dtype=torch.int64), 1)
    np.testing.assert_array_equal(oracle_sparse.activations(conn, torch.from_numpy(s))[0].numpy(), got)
    f32 = torch.from_numpy(s) @ torch.from_numpy(W)
    bound = n_src * np.finfo(np.float32).eps * (s @ np.abs(W))
    assert np.all(np.abs(f32.numpy().astype(np.float64) - got) <= bound + np.abs(got) * 2**-24)


# ---------------------------------------------------------------------------------
# The rate oracle's reduced-precision product (oracle/rate.py)
# ---------------------------------------------------------------------------------


def _bf16_exact(shape, gen):
    return torch.randn(shape, generator=gen).to(torch.bfloat16).float()


def test_rounded_product_is_plain_on_representable_operands():
    """Operands already in bfloat16: forward and both gradients equal the plain float32
    product's (autograd) — a transposed or swapped operand in the backward fails."""
    import oracle.rate as oracle_rate

    gen = torch.Generator().manual_seed(0)
    a, W, g = _bf16_exact((5, 7, 48), gen), _bf16_exact((48, 33), gen), _bf16_exact((5, 7, 33), gen)
    for round_grad in (False, True):
        a1, W1 = a.clone().requires_grad_(), W.clone().requires_grad_()
        a2, W2 = a.clone().requires_grad_(), W.clone().requires_grad_()
        out1 = oracle_rate.product(a1, W1, torch.bfloat16, round_grad)
        out2 = a2 @ W2
        out1.backward(g)
        out2.backward(g)
        assert torch.equal(out1, out2)
        torch.testing.assert_close(a1.grad, a2.grad, rtol=1e-6, atol=1e-6)
        torch.testing.assert_close(W1.grad, W2.grad, rtol=1e-6, atol=1e-6)


def test_rounded_product_rounds_operands_and_dl_da_only():
    """General operands: the forward is the product of the rounded operands (rounding
    is not a no-op here), ``dL/dW`` uses the unrounded ``a`` (the reference's float16
    weight gradient multiplies float32 rates), and ``dL/da`` rounds ``dL/dout`` only when
    asked to."""
    import oracle.rate as oracle_rate

    gen = torch.Generator().manual_seed(1)
    a, W, g = torch.randn((6, 40), generator=gen), torch.randn((40, 9), generator=gen), \
        torch.randn((6, 9), generator=gen)
    ra, rW, rg = (t.to(torch.bfloat16).float() for t in (a, W, g))
    assert not torch.equal(ra, a) and not torch.equal(rg, g)
    for round_grad, g_used in ((False, g), (True, rg)):
        a1, W1 = a.clone().requires_grad_(), W.clone().requires_grad_()
        out = oracle_rate.product(a1, W1, torch.bfloat16, round_grad)
        torch.testing.assert_close(out, ra @ rW, rtol=1e-6, atol=1e-6)
        out.backward(g)
        W_used = rW if round_grad else W
        torch.testing.assert_close(a1.grad, g_used @ W_used.T, rtol=1e-6, atol=1e-6)
        torch.testing.assert_close(W1.grad, a.T @ g, rtol=1e-6, atol=1e-6)
    # float32 storage is the plain product
    torch.testing.assert_close(oracle_rate.product(a, W, torch.float32, True), a @ W)


# ---------------------------------------------------------------------------------
# Pathways folded per receptor kind (oracle.dynamics.fold)
# ---------------------------------------------------------------------------------


def _random_drive(seed, K_rec=9, K_ff=4, S=3, N=40, n_src=50, n_in=30):
    from wiretorch_amd.network import Drive

    rng = np.random.default_rng(seed)
    kinds = rng.random((3, S)) < 0.6
    kinds[:, 0] |= ~kinds.any(axis=1)
    made = torch.from_numpy(kinds[rng.integers(0, 3, K_rec + K_ff)])
    scale = torch.from_numpy(rng.lognormal(0, 0.5, (K_rec + K_ff, N)).astype(np.float32))

    def pathways(n, K):
        rows = np.array_split(rng.permutation(n), K)
        return [(torch.from_numpy(r).long(),
                 torch.from_numpy((rng.lognormal(-1, 1, (len(r), N)) * (rng.random((len(r), N)) < 0.3))
                                  .astype(np.float32))) for r in rows]

    return Drive(made=made, scale=scale, recurrent=pathways(n_src, K_rec),
                 feedforward=pathways(n_in, K_ff))


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_fold_regroups_the_injection_exactly(seed):
    """In float64 arithmetic (a float64 drive) the folded drive injects what the
    per-pathway drive does (the reference's sum over pathways of a_k (jump scale_k
    made_k), with a_k the pathway's rows times its weights): one step's conductance
    increment from random spikes and inputs, 13 pathways of 3 kinds, agrees to 1e-12
    relative."""
    import oracle.dynamics as od

    drive = _random_drive(seed)
    drive.scale = drive.scale.double()  # the regrouping alone (fold's products in float64)
    drive.recurrent = [(r, W.double()) for r, W in drive.recurrent]
    drive.feedforward = [(r, W.double()) for r, W in drive.feedforward]
    folded = od.fold(drive)
    rng = np.random.default_rng(seed + 10)
    s = torch.from_numpy((rng.random((2, 50)) < 0.4).astype(np.float64))
    x = torch.from_numpy((rng.random((2, 30)) < 0.4).astype(np.float64))
    jump = torch.from_numpy(rng.normal(0, 1, (2, 3)))

    def increment(d):
        total = torch.zeros((2, 40, 2, 3), dtype=torch.float64)
        acts = ([s[:, rows] @ W.double() for rows, W in d.recurrent]
                + [x[:, rows] @ W.double() for rows, W in d.feedforward])
        assert len(acts) == d.made.shape[0]
        for k, a in enumerate(acts):
            kernel = jump[None] * d.scale[k].double()[:, None, None] * d.made[k].double()
            total += a[:, :, None, None] * kernel
        return total

    want, got = increment(drive), increment(folded)
    assert folded.made.shape[0] <= 6 and len(folded.recurrent) <= 3
    assert torch.allclose(got, want, rtol=1e-12, atol=1e-12 * float(want.abs().max()))


def test_fold_of_many_types_follows_the_per_pathway_run(monkeypatch):
    """The many-cell-type network (21 pathways): 200 steps of the folded drive against
    the per-pathway one, both with exactly rounded sums: voltages within 1e-5 relative,
    spikes identical; and the engine's own folding gives the oracle's folded weights
    bit for bit."""
    import oracle.dynamics as od
    import scenarios as sc
    from wiretorch_amd import engine, synthetic

    monkeypatch.setattr(od, "SUMS", "exact")
    wl = synthetic.many_types(T=200)
    model = wl.model
    sc.use_engine(model, od)
    drive, p = model._drive(), model._physiology()
    assert drive.K_rec + drive.K_ff == 21
    x = torch.from_numpy(wl.x).float()
    model.reset_state()
    with torch.no_grad():
        a = od.simulate(model.v, model._synaptic, x, drive, p, track=True)
        b = od.simulate(model.v, model._synaptic, x, od.fold(drive), p, track=True)
    assert a.output.sum() > 0
    assert torch.equal(a.output, b.output)
    np.testing.assert_allclose(b.tracked["v"].numpy(), a.tracked["v"].numpy(), rtol=1e-5,
                               atol=65e-5)
    mine = engine.fold_pathways(drive)
    theirs = od.fold(drive)
    assert torch.equal(mine.made, theirs.made)
    for (r1, W1), (r2, W2) in zip(mine.recurrent + mine.feedforward,
                                  theirs.recurrent + theirs.feedforward):
        assert torch.equal(r1, r2) and torch.equal(W1, W2)
