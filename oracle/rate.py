"""The rate-network step restated on the CPU — TEST INFRASTRUCTURE ONLY (see
``oracle/__init__.py``).

Op for op the reference's PyTorch rate step, so that its recorded CPU fixtures
(``rate_recurrent``, ``rate_recurrent_learnt``, ``rate_feedforward``) reproduce:

* ``NONLINEARITIES`` — ``src/wiretorch/network_simulators/rate/dynamics.py:63-69``;
* ``kernels`` — ``rate/dynamics.py:95-97``;
* ``rates`` — ``rate/dynamics.py:100-106``;
* ``simulate`` — ``rate/dynamics.py:109-160``.

With a reduced-precision ``storage_dtype`` (``RatePhysiology.storage_dtype``; the
reference has float16, ``network.py:52``, this build bfloat16) the products multiply
operands rounded to it (round to nearest even, ``Tensor.to``) and accumulate in float32;
every product of two bfloat16 or float16 numbers is exact in float32, so only the order
of the float32 sums can differ from a GPU's. The gradients follow the reference's
float16 recurrent product (``rate/engine.py:157-210,367-376``): ``dL/dr = round(dL/da)
@ round(W)^T`` and ``dL/dW = r^T dL/da`` in float32, with ``r`` as computed (not
rounded). Two deliberate differences from the reference's float16 input product, which
runs under autocast (``rate/engine.py:386-393``): its output stays float32 (autocast
rounds it to the storage dtype), and its gradients are float32 products of the unrounded
operands.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from wiretorch_amd.network import Run

NONLINEARITIES = {
    "relu": F.relu,
    "softplus": F.softplus,
    "sigmoid": torch.sigmoid,
    "tanh": torch.tanh,
}


def stack_steps(tensors):
    return torch.stack([t.contiguous() for t in tensors], dim=1)


def kernels(drive):
    """Per pathway, the ``(N, S)`` input to each synapse type per unit activation."""
    return [drive.scale[k][:, None] * drive.made[k] for k in range(drive.made.shape[0])]


def rates(v, p):
    """``gain f(v - theta)``, each cell type with its own ``f``."""
    x = v - p.theta
    r = torch.zeros_like(x)
    for name, neurons in p.groups:
        r = r.index_copy(-1, neurons, NONLINEARITIES[name](x.index_select(-1, neurons)))
    return p.gain * r


def rounded(t, dtype):
    """``t`` rounded to ``dtype`` and back to float32 (unchanged for float32)."""
    return t if dtype == torch.float32 else t.to(dtype).float()


class _Product(torch.autograd.Function):
    """``round(a) @ round(W)`` over the last axis of ``a``, with the gradients described
    in the module docstring (``round_grad``: the recurrent product's rounding of
    ``dL/da``)."""

    @staticmethod
    def forward(ctx, a, W, dtype, round_grad):
        ctx.save_for_backward(a, W)
        ctx.dtype, ctx.round_grad = dtype, round_grad
        return rounded(a, dtype) @ rounded(W, dtype)

    @staticmethod
    def backward(ctx, g):
        a, W = ctx.saved_tensors
        if ctx.round_grad:
            da = rounded(g, ctx.dtype) @ rounded(W, ctx.dtype).T
        else:
            da = g @ W.T
        dW = a.reshape(-1, a.shape[-1]).T @ g.reshape(-1, g.shape[-1])
        return da, dW, None, None


def product(a, W, dtype, round_grad):
    if dtype == torch.float32:
        return a @ W
    return _Product.apply(a, W, dtype, round_grad)


def feedforward_activations(x, drive, dtype):
    """``(K_ff, B, T, N)``: ``x[:, :, rows] @ W`` per input pathway
    (``network.py:142-157``), operands in ``dtype``."""
    B, T = x.shape[:2]
    if not drive.feedforward:
        return x.new_zeros((0, B, T, 0))
    return torch.stack([product(x[:, :, rows], W, dtype, False) for rows, W in drive.feedforward])


def simulate(v, I, x, drive, p, *, probabilities=False, track=False, track_batch_idx=None,
             retain=None):
    """``x.shape[1]`` steps from state ``(v, I)`` (``(B, N)``, ``(B, N, S)``)."""
    assert not probabilities, "rate networks have no spike probabilities"
    dtype = getattr(p, "storage_dtype", torch.float32)
    A_ff = feedforward_activations(x, drive, dtype)
    jumps = kernels(drive)
    keep = slice(None) if track_batch_idx is None else slice(track_batch_idx, track_batch_idx + 1)
    outputs, tracked = [], {"v": [], "I": []}
    for t in range(x.shape[1]):
        r = rates(v, p)
        activations = [product(r[:, rows], W, dtype, True) for rows, W in drive.recurrent]
        activations += list(A_ff[:, :, t])
        target = sum(a[:, :, None] * jump for a, jump in zip(activations, jumps))
        I = p.decay * I + (1 - p.decay) * target
        I_syn = sum(I[..., j] * p.sign[j] for j in range(I.shape[-1]))
        v = p.beta * v + (1 - p.beta) * I_syn
        outputs.append(r)
        if retain is not None:
            for tensor in (v, I, r):
                if tensor.requires_grad:
                    tensor.retain_grad()
            retain.append((v, I, r))
        if track:
            tracked["v"].append(v[keep].detach())
            tracked["I"].append(I[keep].detach())
    return Run(
        output=torch.stack(outputs, dim=1),
        v=v,
        syn=I,
        tracked={k: stack_steps(val) for k, val in tracked.items()} if track else None,
    )
