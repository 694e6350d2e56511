"""The double-exponential filter's HIP kernels against the oracle, bit for bit.

``wt_filter_forward`` / ``wt_filter_backward`` round every multiply and add separately,
as the float32 oracle recursion does, so rise, smooth and dL/dx must be identical:
binary and real-valued trains, carried state, time lengths that are and are not a
multiple of the kernel's 8-step load chunk, a single column, an empty time axis, and a
training-sized batch. ``VanRossumLoss`` is checked against the reference's own test
definition (``tests/test_losses.py:67-90``: literal sums, chunk carry, gradients) with
the reference's GPU tolerance, 1e-4.
"""

import numpy as np
import pytest
import torch

import oracle.filtering as of
from wiretorch_amd.filtering import VanRossumLoss, double_exponential

pytestmark = pytest.mark.gpu
DEV = "cuda"
TAU_RISE, TAU_DECAY, DT, CHUNK = 10.0, 100.0, 1.0, 40


def kernels(T=2):
    t = torch.arange(max(T, 2), dtype=torch.float32, device=DEV) * DT
    return torch.exp(-t / TAU_RISE), torch.exp(-t / TAU_DECAY)


def decays():
    kr, kd = kernels()
    return float(kr[1]), float(kd[1])


@pytest.mark.parametrize("shape,binary,carry", [
    ((3, 120, 7), True, False),
    ((3, 120, 7), True, True),
    ((4, 37, 300), False, True),
    ((1, 1, 1), False, True),
    ((2, 0, 5), False, False),
    ((64, 500, 2000), True, True),
])  # fmt: skip
def test_forward_and_backward_bit_exact(shape, binary, carry):
    print(f"filter shape={shape} binary={binary} carry={carry}", flush=True)
    rng = np.random.default_rng(sum(shape))
    B, T, N = shape
    x = (rng.random(shape) < 0.05).astype(np.float32) if binary else \
        rng.standard_normal(shape).astype(np.float32)
    cr = rng.random((B, 1, N)).astype(np.float32) if carry else None
    cs = rng.random((B, 1, N)).astype(np.float32) if carry else None
    a_r, a_d = decays()
    r_ref, s_ref = of.forward(x, a_r, a_d, cr, cs)
    xd = torch.from_numpy(x).to(DEV).requires_grad_(True)
    dev = lambda c: None if c is None else torch.from_numpy(c).to(DEV)  # noqa: E731
    r, s = double_exponential(xd, *kernels(T), dev(cr), dev(cs))
    assert not r.requires_grad
    np.testing.assert_array_equal(r.cpu().numpy(), r_ref)
    np.testing.assert_array_equal(s.detach().cpu().numpy(), s_ref)
    if T == 0:
        return
    g = rng.standard_normal(shape).astype(np.float32)
    (grad,) = torch.autograd.grad(s, xd, torch.from_numpy(g).to(DEV))
    np.testing.assert_array_equal(grad.cpu().numpy(), of.backward(g, a_r, a_d))


def literal(x, tau, carried):
    T = x.shape[1]
    kernel = torch.exp(-torch.arange(T, dtype=x.dtype, device=x.device) * DT / tau)
    y = torch.stack([(kernel[: t + 1].flip(0)[None, :, None] * x[:, : t + 1]).sum(1)
                     for t in range(T)], dim=1)  # fmt: skip
    return y if carried is None else y + carried * kernel[None, :, None]


def reference_smooth(chunks):
    rise = smooth = None
    out = []
    for x in chunks:
        r = literal(x, TAU_RISE, rise)
        y = literal(r, TAU_DECAY, smooth)
        rise, smooth = r[:, -1:].detach(), y[:, -1:].detach()
        out.append(y)
    return out


def test_van_rossum_loss_matches_definition():
    rng = np.random.default_rng(0)
    output, target = (torch.from_numpy((rng.random((3, 3 * CHUNK, 7)) < 0.05)
                                       .astype(np.float32)).to(DEV) for _ in range(2))  # fmt: skip
    output.requires_grad_(True)
    loss_fn = VanRossumLoss(TAU_RISE, TAU_DECAY, DT, CHUNK, device=DEV)
    chunks = [slice(c, c + CHUNK) for c in range(0, output.shape[1], CHUNK)]
    o_ref = reference_smooth([output[:, c] for c in chunks])
    t_ref = reference_smooth([target[:, c] for c in chunks])
    for c, o, t in zip(chunks, o_ref, t_ref):
        loss = loss_fn(output[:, c], target[:, c])
        expected = ((o - t) ** 2).mean()
        torch.testing.assert_close(loss, expected, rtol=1e-4, atol=1e-7)
        (grad,) = torch.autograd.grad(loss, output, retain_graph=True)
        (expected_grad,) = torch.autograd.grad(expected, output, retain_graph=True)
        torch.testing.assert_close(
            grad, expected_grad, rtol=1e-4, atol=1e-4 * float(expected_grad.abs().max()))
    loss_fn.reset_state()
    first = VanRossumLoss(TAU_RISE, TAU_DECAY, DT, CHUNK, device=DEV)(
        output[:, :CHUNK], target[:, :CHUNK])
    torch.testing.assert_close(loss_fn(output[:, :CHUNK], target[:, :CHUNK]), first)
