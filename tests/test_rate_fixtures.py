"""The rate-network oracle against the reference's recorded fixtures.

``tests/golden/reference/rate_*.npz`` were recorded from the reference's PyTorch CPU
rate step (``rate/dynamics.py``). The networks are rebuilt through this package's API
(``wiretorch_amd.rate``) and run on the oracle (``oracle.rate``); the reference's own
criteria apply (``tests/test_rate.py:30-88``): fingerprints equal, rates and voltages
within 1e-5 of each variable's range in a free run and restarted from every recorded
state, gradients within 1e-4 of each gradient's scale (``tests/test_gradients.py``).
"""

import numpy as np
import pytest
import torch

import oracle.rate as oracle_rate
import scenarios as sc

NAMES = list(sc.RATE_SCENARIOS)


def build(name, engine=oracle_rate, device="cpu"):
    built = sc.RATE_SCENARIOS[name].build(sc.BATCH_SIZE)
    built.model.to(device)
    sc.use_engine(built.model, engine)
    return built


@pytest.mark.parametrize("name", NAMES)
def test_fingerprint(name):
    _, meta = sc.load_fixture(name)
    assert sc.fingerprint(build(name)) == meta["fingerprint"]


@pytest.mark.parametrize("name", NAMES)
def test_free_run(name):
    recorded, _ = sc.load_fixture(name)
    record = sc.free_run(sc.RATE_SCENARIOS[name], build(name))
    for key in ("rates", "voltages"):
        atol = 1e-5 * np.ptp(recorded[key])
        np.testing.assert_allclose(record[key], recorded[key], rtol=0, atol=atol, err_msg=key)
    for key in ("v", "I_syn"):
        np.testing.assert_allclose(record[f"state.{key}"], recorded[f"state.{key}"],
                                   rtol=1e-4, atol=1e-5 * np.ptp(recorded[f"state.{key}"]))


@pytest.mark.parametrize("name", NAMES)
def test_lockstep(name):
    scenario = sc.RATE_SCENARIOS[name]
    recorded, _ = sc.load_fixture(name)
    built = build(name)
    model = built.model
    model.track_variables, model.track_batch_idx = True, None
    x = torch.from_numpy(built.input_spikes)
    for w, start in enumerate(range(0, x.shape[1], sc.WINDOW)):
        stop = start + sc.WINDOW
        model.load_checkpoint_state({k: recorded[f"state.{k}"][w] for k in scenario.state_keys})
        with torch.no_grad():
            out = model(x[:, start:stop])
        for key in ("rates", "voltages"):
            atol = 1e-5 * np.ptp(recorded[key])
            np.testing.assert_allclose(out[key].numpy(), recorded[key][:, start:stop], rtol=0,
                                       atol=atol, err_msg=f"{key}, window {w}")


@pytest.mark.parametrize("name", NAMES)
def test_gradients(name):
    recorded, _ = sc.load_fixture(name)
    loss, grads = sc.gradients(build(name))
    expected = {k[len("grad."):]: v for k, v in recorded.items() if k.startswith("grad.")}
    assert grads.keys() == expected.keys()
    np.testing.assert_allclose(loss, recorded["loss"], rtol=1e-4)
    for key, value in expected.items():
        scale = np.abs(value).max() or 1.0
        np.testing.assert_allclose(grads[key], value, rtol=0, atol=1e-4 * scale, err_msg=key)
