"""The Mg block on the GPU against the oracle (reference ``tests/test_nmda.py:100-153``):
spikes, final voltages and every gradient — scaling factors and all learnable
physiology, whose terms the block enters — through both backward passes, with and
without a refractory period, with learnt recurrent weights, and for the feed-forward
network with spike probabilities in the loss.

The comparison follows the reference's own kernel test (``tests/test_learnt_physiology.py:
120-176``): the learnt physiology is moved off its defaults and a warm-up chunk runs
first; spikes equal, final voltages within 1e-4; a gradient within 1e-3 of its scale, or,
where one sums terms that nearly cancel, no further from the oracle run in float64 than
twice the float32 oracle's own distance plus 1e-4 of the scale.
"""

import numpy as np
import pytest
import torch

import oracle.dynamics as oracle_engine
import scenarios as sc
from wiretorch_amd import engine

pytestmark = pytest.mark.gpu
DEV = "cuda"
MG = 1.0
LEARN = dict.fromkeys(["tau_mem", "theta", "U_reset", "E_L", "g_L", "tau_rise", "tau_decay",
                       "E_syn", "g_bar"], True)


def _gradients(builder, device, eng, warm_up=30, steps=60, float64=False):
    built = builder()
    model = built.model
    if float64:
        model = model.double()
    model = model.to(device)
    sc.use_engine(model, eng)
    model.reset_state()
    rng = np.random.default_rng(1)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.startswith(("cell_", "synapse_")):
                p += torch.from_numpy(0.1 * rng.standard_normal(p.shape).astype(np.float32)).to(p)
        x0 = torch.from_numpy(built.input_spikes[:, :warm_up]).to(device)
        model(x0.double() if float64 else x0)
    x = torch.from_numpy(built.input_spikes[:, warm_up:warm_up + steps]).to(device)
    out = sc.unpack_output(model(x.double() if float64 else x), built.output)
    rng = np.random.default_rng(3)
    loss = 0
    for key in ("spikes", "probabilities"):
        if out.get(key) is not None:
            R = torch.from_numpy(rng.standard_normal(out[key].shape).astype(np.float32))
            loss = loss + (out[key] * R.to(out[key])).sum()
    loss.backward()
    grads = {n: p.grad.detach().cpu().double() for n, p in model.named_parameters()
             if p.grad is not None}
    return out["spikes"].detach().cpu(), model.v.detach().cpu().double(), grads


def _engine_vs_oracle(builder):
    s_k, v_k, g_k = _gradients(builder, DEV, engine)
    s_r, v_r, g_r = _gradients(builder, "cpu", oracle_engine)
    assert s_r.sum() > 0
    differs = (s_k != s_r).any(dim=0).any(dim=-1)
    assert not differs.any(), f"spikes differ from step {int(differs.nonzero()[0])}"
    torch.testing.assert_close(v_k, v_r, rtol=1e-4, atol=1e-4)
    assert g_k.keys() == g_r.keys() and g_k
    g_64 = None
    for key in g_r:
        scale = g_r[key].abs().max().item() or 1.0
        if torch.allclose(g_k[key], g_r[key], rtol=0, atol=1e-3 * scale):
            continue
        if g_64 is None:
            g_64 = _gradients(builder, "cpu", oracle_engine, float64=True)[2]
        err_k = (g_k[key] - g_64[key]).abs().max().item()
        err_r = (g_r[key] - g_64[key]).abs().max().item()
        assert err_k <= 2 * err_r + 1e-4 * scale, (key, err_k, err_r, scale)
    return g_k


def _with_flag(builder, recurrent_gradients):
    def build():
        built = builder()
        built.model.recurrent_gradients = recurrent_gradients
        return built

    return build


@pytest.mark.parametrize("tau_ref", [None, 5.0], ids=["", "refractory"])
@pytest.mark.parametrize("recurrent_gradients", [False, True], ids=["off", "on"])
def test_recurrent_matches_oracle(recurrent_gradients, tau_ref):
    builder = lambda: sc.recurrent(  # noqa: E731
        sc.BATCH_SIZE, sc.SEED, scaling_factors=True, learn=LEARN, mg=MG, tau_ref=tau_ref)
    _engine_vs_oracle(_with_flag(builder, recurrent_gradients))


def test_recurrent_weights_match_oracle():
    """Learnt recurrent weights, gradients through the recurrent spikes."""
    builder = lambda: sc.recurrent(sc.BATCH_SIZE, sc.SEED, learnt_weights=True, mg=MG)  # noqa: E731
    _engine_vs_oracle(_with_flag(builder, True))


def test_feedforward_matches_oracle():
    """The feed-forward scan, with spike probabilities in the loss."""
    _engine_vs_oracle(lambda: sc.feedforward(sc.BATCH_SIZE, sc.SEED, probabilities=True,
                                             learn=LEARN, mg=MG))


def test_block_free_run_matches_oracle():
    """200 steps with the block: the raster equals the oracle's, voltages within 1e-5."""
    built = sc.recurrent(sc.BATCH_SIZE, sc.SEED, mg=MG)
    x = torch.from_numpy(built.input_spikes)
    runs = []
    for device, eng in (("cpu", oracle_engine), (DEV, engine)):
        model = built.model.to(device)
        sc.use_engine(model, eng)
        model.reset_state()
        model.track_variables, model.track_batch_idx = True, None
        with torch.no_grad():
            out = model(x.to(device))
        runs.append((out["spikes"].cpu().numpy(), out["voltages"].cpu().numpy()))
    (s_r, v_r), (s_k, v_k) = runs
    assert s_r.sum() > 0
    differs = (s_k != s_r).any(axis=(0, 2))
    assert not differs.any(), f"rasters differ from step {int(np.argmax(differs))}"
    np.testing.assert_allclose(v_k, v_r, rtol=1e-5, atol=65e-5)
