"""The double-exponential filter's oracle, pinned without a GPU.

The reference's own tests define the filter as the literal sum over past inputs with a
chunk carry (``tests/test_losses.py:26-52``); that definition is restated here in
float64 on the same trains those tests draw (``tests/test_losses.py:55-64``: seed 0,
(3, 120, 7) Bernoulli(0.05), tau 10 / 100 ms, dt 1 ms, chunks of 40). The float32
recursion must agree within the reference's CPU tolerance (1e-5 relative). An impulse
pins the closed forms of both stages and the undecayed entry of the carried state; the
adjoint identity pins the reverse recursion. The host module's CPU behaviour (it
raises) is checked here too.
"""

import numpy as np
import pytest
import torch

import oracle.filtering as of

TAU_RISE, TAU_DECAY, DT, CHUNK = 10.0, 100.0, 1.0, 40


def decays():
    """``kernel[1]`` as the reference's loss computes it: float32 ``exp(-dt / tau)``."""
    t = torch.arange(2, dtype=torch.float32) * DT
    return float(torch.exp(-t / TAU_RISE)[1]), float(torch.exp(-t / TAU_DECAY)[1])


def literal(x, tau, carried):
    """``y[t] = sum_{k<=t} exp(-k dt/tau) x[t-k] + carried exp(-t dt/tau)``, float64."""
    T = x.shape[1]
    kernel = np.exp(-np.arange(T) * DT / tau)
    y = np.stack([(kernel[: t + 1][::-1][None, :, None] * x[:, : t + 1]).sum(1)
                  for t in range(T)], axis=1)  # fmt: skip
    return y if carried is None else y + carried * kernel[None, :, None]


def reference_trains():
    rng = np.random.default_rng(0)
    return [(rng.random((3, 3 * CHUNK, 7)) < 0.05).astype(np.float32) for _ in range(2)]


def test_matches_the_reference_tests_definition_with_chunk_carry():
    a_r, a_d = decays()
    for train in reference_trains():
        rise = smooth = rise64 = smooth64 = None
        for c in range(0, train.shape[1], CHUNK):
            x = train[:, c : c + CHUNK]
            r, s = of.forward(x, a_r, a_d, rise, smooth)
            r64 = literal(x.astype(np.float64), TAU_RISE, rise64)
            s64 = literal(r64, TAU_DECAY, smooth64)
            np.testing.assert_allclose(r, r64, rtol=1e-5, atol=1e-7)
            np.testing.assert_allclose(s, s64, rtol=1e-5, atol=1e-7)
            rise, smooth = r[:, -1:], s[:, -1:]
            rise64, smooth64 = r64[:, -1:], s64[:, -1:]


def test_impulse_and_carried_state_closed_forms():
    a_r, a_d = decays()
    T = 100
    t = np.arange(T, dtype=np.float64)
    ar, ad = np.float64(np.float32(a_r)), np.float64(np.float32(a_d))
    both = (ar ** (t + 1) - ad ** (t + 1)) / (ar - ad)
    x = np.zeros((1, T, 1), np.float32)
    x[0, 0, 0] = 1.0
    r, s = of.forward(x, a_r, a_d)
    np.testing.assert_allclose(r[0, :, 0], ar ** t, rtol=2e-5)
    np.testing.assert_allclose(s[0, :, 0], both, rtol=2e-5)
    # carried state alone: it enters undecayed at t = 0, then decays
    c_r, c_s = np.float32(0.75), np.float32(-2.5)
    r, s = of.forward(np.zeros((1, T, 1), np.float32), a_r, a_d,
                      np.full((1, 1, 1), c_r), np.full((1, 1, 1), c_s))  # fmt: skip
    np.testing.assert_allclose(r[0, :, 0], c_r * ar ** t, rtol=2e-5)
    np.testing.assert_allclose(s[0, :, 0], c_s * ad ** t + c_r * both, rtol=2e-5, atol=1e-6)


@pytest.mark.parametrize("T", [1, 9, 64])
def test_backward_is_the_adjoint_of_forward(T):
    a_r, a_d = decays()
    rng = np.random.default_rng(T)
    x = rng.standard_normal((2, T, 5)).astype(np.float32)
    g = rng.standard_normal((2, T, 5)).astype(np.float32)
    _, s = of.forward(x, a_r, a_d)
    lhs = float((g.astype(np.float64) * s).sum())
    rhs = float((of.backward(g, a_r, a_d).astype(np.float64) * x).sum())
    assert abs(lhs - rhs) <= 1e-5 * (abs(lhs) + np.abs(g).sum())


def test_backward_matches_autograd_through_the_literal_sum():
    a_r, a_d = decays()
    rng = np.random.default_rng(1)
    x = torch.from_numpy(rng.standard_normal((2, 30, 4))).requires_grad_(True)
    g = rng.standard_normal((2, 30, 4)).astype(np.float32)
    T = x.shape[1]
    lag = torch.arange(T)[:, None] - torch.arange(T)[None, :]
    def toeplitz(y, a):
        return torch.where(lag >= 0, torch.tensor(a, dtype=torch.float64) ** lag.clamp(min=0), 0.0) @ y
    s = toeplitz(toeplitz(x, a_r), a_d)
    (grad,) = torch.autograd.grad((s * torch.from_numpy(g).double()).sum(), x)
    np.testing.assert_allclose(of.backward(g, a_r, a_d), grad.numpy(), rtol=1e-5, atol=1e-5)


def test_host_module_has_no_cpu_path():
    from wiretorch_amd.filtering import VanRossumLoss, double_exponential

    k = torch.tensor([1.0, 0.9])
    with pytest.raises(RuntimeError, match="GPU"):
        double_exponential(torch.zeros(1, 3, 2), k, k, None, None)
    with pytest.raises(RuntimeError, match="GPU"):
        VanRossumLoss(TAU_RISE, TAU_DECAY, DT, CHUNK, device="cpu")(
            torch.zeros(1, 3, 2), torch.zeros(1, 3, 2))
