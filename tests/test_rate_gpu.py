"""The rate-network engine (MFMA) against the reference's rate fixtures and the oracle.

With float32 storage (``v_mfma_f32_32x32x2_f32``): the free run and every lockstep window
within 1e-4 of each variable's range (the reference's own GPU criterion,
``tests/test_rate.py:30``), gradients within 1e-4 of each gradient's scale. With
bfloat16 storage (``v_mfma_f32_32x32x16_bf16``, rates and weights rounded to 8-bit
mantissas, float32 accumulation) the rates stay within 2e-2 of their range of the float32
oracle's: the rounding of the products, not an error of the step.
"""

import numpy as np
import pytest
import torch

import oracle.rate as oracle_rate
import scenarios as sc

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAMES = list(sc.RATE_SCENARIOS)


def build(name, device=DEV, **kwargs):
    built = sc.RATE_SCENARIOS[name].build(sc.BATCH_SIZE) if not kwargs else \
        sc.rate_recurrent(sc.BATCH_SIZE, sc.SEED, **kwargs)
    built.model.to(device)
    return built


@pytest.mark.parametrize("name", NAMES)
def test_free_run_on_gpu(name):
    recorded, _ = sc.load_fixture(name)
    record = sc.free_run(sc.RATE_SCENARIOS[name], build(name), device=DEV)
    for key in ("rates", "voltages"):
        atol = 1e-4 * np.ptp(recorded[key])
        np.testing.assert_allclose(record[key], recorded[key], rtol=0, atol=atol, err_msg=key)


@pytest.mark.parametrize("name", NAMES)
def test_lockstep_on_gpu(name):
    scenario = sc.RATE_SCENARIOS[name]
    recorded, _ = sc.load_fixture(name)
    built = build(name)
    model = built.model
    model.track_variables, model.track_batch_idx = True, None
    x = torch.from_numpy(built.input_spikes).to(DEV)
    for w, start in enumerate(range(0, x.shape[1], sc.WINDOW)):
        stop = start + sc.WINDOW
        model.load_checkpoint_state({k: recorded[f"state.{k}"][w] for k in scenario.state_keys})
        with torch.no_grad():
            out = model(x[:, start:stop])
        for key in ("rates", "voltages"):
            atol = 1e-4 * np.ptp(recorded[key])
            np.testing.assert_allclose(out[key].cpu().numpy(), recorded[key][:, start:stop],
                                       rtol=0, atol=atol, err_msg=f"{key}, window {w}")
        for key, value in model.get_checkpoint_state().items():
            ref = recorded[f"state.{key}"][w + 1]
            np.testing.assert_allclose(value, ref, rtol=0, atol=1e-4 * (np.ptp(ref) or 1.0),
                                       err_msg=f"state {key}, window {w}")


@pytest.mark.parametrize("name", NAMES)
def test_gradients_on_gpu(name):
    recorded, _ = sc.load_fixture(name)
    loss, grads = sc.gradients(build(name), device=DEV)
    expected = {k[len("grad."):]: v for k, v in recorded.items() if k.startswith("grad.")}
    assert grads.keys() == expected.keys()
    np.testing.assert_allclose(loss, recorded["loss"], rtol=1e-4)
    for key, value in expected.items():
        scale = np.abs(value).max() or 1.0
        np.testing.assert_allclose(grads[key], value, rtol=0, atol=1e-4 * scale, err_msg=key)


def test_learnt_recurrent_weights_on_gpu():
    """Recurrent weights trained directly (full rank): the engine's plain-product weight
    gradient against the oracle's autograd."""
    results = {}
    for device, engine in (("cpu", oracle_rate), (DEV, None)):
        built = sc.rate_recurrent(sc.BATCH_SIZE, sc.SEED, learnt_excitatory=True)
        built.model.to(device)
        if engine is not None:
            sc.use_engine(built.model, engine)
        results[device] = sc.gradients(built, device=device)
    (l_cpu, g_cpu), (l_gpu, g_gpu) = results["cpu"], results[DEV]
    np.testing.assert_allclose(l_gpu, l_cpu, rtol=1e-4)
    assert g_cpu.keys() == g_gpu.keys()
    for key, value in g_cpu.items():
        scale = np.abs(value).max() or 1.0
        np.testing.assert_allclose(g_gpu[key], value, rtol=0, atol=1e-4 * scale, err_msg=key)


def test_bfloat16_storage_close_to_float32():
    built = sc.rate_recurrent(sc.BATCH_SIZE, sc.SEED, storage_dtype=torch.bfloat16)
    built.model.to(DEV)
    x = torch.from_numpy(built.input_spikes)
    with torch.no_grad():
        r_bf16 = built.model(x.to(DEV)).cpu().numpy()
    ref = sc.rate_recurrent(sc.BATCH_SIZE, sc.SEED)
    sc.use_engine(ref.model, oracle_rate)
    with torch.no_grad():
        r_ref = ref.model(x).numpy()
    np.testing.assert_allclose(r_bf16, r_ref, rtol=0, atol=2e-2 * np.ptp(r_ref))
