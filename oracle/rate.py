"""The rate-network step restated on the CPU — TEST INFRASTRUCTURE ONLY (see
``oracle/__init__.py``).

Op for op the reference's PyTorch rate step, so that its recorded CPU fixtures
(``rate_recurrent``, ``rate_recurrent_learnt``, ``rate_feedforward``) reproduce:

* ``NONLINEARITIES`` — ``src/wiretorch/network_simulators/rate/dynamics.py:63-69``;
* ``kernels`` — ``rate/dynamics.py:95-97``;
* ``rates`` — ``rate/dynamics.py:100-106``;
* ``simulate`` — ``rate/dynamics.py:109-160``.
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


def simulate(v, I, x, drive, p, *, probabilities=False, track=False, track_batch_idx=None,
             retain=None):
    """``x.shape[1]`` steps from state ``(v, I)`` (``(B, N)``, ``(B, N, S)``)."""
    assert not probabilities, "rate networks have no spike probabilities"
    A_ff = drive.feedforward_activations(x)
    jumps = kernels(drive)
    keep = slice(None) if track_batch_idx is None else slice(track_batch_idx, track_batch_idx + 1)
    outputs, tracked = [], {"v": [], "I": []}
    for t in range(x.shape[1]):
        r = rates(v, p)
        activations = [r[:, rows] @ W for rows, W in drive.recurrent]
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
