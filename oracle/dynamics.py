"""The conductance-LIF step restated on the CPU — TEST INFRASTRUCTURE ONLY (see
``oracle/__init__.py``).

Op for op the reference's PyTorch step, so that recorded CPU fixtures reproduce
bit for bit (same torch CPU kernels, same association order):

* ``SurrGradSpike`` — ``src/wiretorch/training_utils/surrogate_gradients.py:9-33``;
* ``jumps`` — ``conductance/dynamics.py:95-100``;
* ``spike`` — ``conductance/dynamics.py:103-107``;
* ``mg_block`` — ``conductance/dynamics.py:110-113``;
* ``membrane`` — ``conductance/dynamics.py:116-143`` (the Mg block and the adaptation
  conductance);
* ``simulate`` — ``conductance/dynamics.py:146-237`` (adaptation; presynaptic dynamics
  on feedforward pathways, not on recurrent ones);
* ``gate_step`` / ``gate_feedforward`` — ``network_simulators/network.py:186-250``
  (short-term plasticity and receptor saturation of a feedforward pathway's inputs);
* ``refractory_mask`` / ``held_at_reset`` / ``count_down`` —
  ``network_simulators/network.py:294-318``;
* ``recurrent_activations`` — ``network_simulators/network.py:260-271``;
* ``Drive.feedforward_activations`` — ``network_simulators/network.py:142-157``;
* ``fold`` — the injection's sum regrouped by the synapse types pathways make
  (``conductance/dynamics.py:95-100,206-208``), the form the engine evaluates for drives
  of many pathways.

A drive given in compressed form (``sparse_recurrent`` / ``sparse_feedforward``)
propagates through ``oracle.sparse.activations`` instead of the dense products.

``SUMS`` picks how a dense pathway's product ``s[:, rows] @ W`` is summed:

* ``"float32"`` (default) — torch CPU's float32 matrix product, the reference's own
  call; its rounding depends on the BLAS's blocking, and the reference's recorded
  fixtures were made with it;
* ``"exact"`` — the same products summed in float64 and rounded to float32 once: for
  0/1 spikes times float32 weights the exactly rounded sum (float64 holds every partial
  sum of a few thousand float32 weights within 2^29 of each other exactly), the value
  ``oracle.sparse`` computes and the GPU kernels compute. Parity tests at sizes where
  float32 BLAS rounding alone flips spikes use it (gradients then flow through the float64
  product, rounded to float32).
"""

from __future__ import annotations

import torch

from oracle import sparse as _sparse


class SurrGradSpike(torch.autograd.Function):
    """Heaviside forward; fast-sigmoid surrogate ``g / (k |x| + 1)^2`` backward."""

    @staticmethod
    def forward(x, scale):
        return (x > 0).to(x.dtype)

    @staticmethod
    def setup_context(ctx, inputs, output):
        x, scale = inputs
        ctx.save_for_backward(x)
        ctx.scale = scale

    @staticmethod
    def backward(ctx, grad):
        (x,) = ctx.saved_tensors
        return grad / (ctx.scale * torch.abs(x) + 1.0) ** 2, None


def jumps(drive, jump):
    """Per pathway, the ``(N, 2, S)`` conductance jump per unit activation."""
    return [
        jump[None] * drive.scale[k][:, None, None] * drive.made[k]
        for k in range(drive.made.shape[0])
    ]


def refractory_mask(counter, n_ref):
    return None if n_ref is None else (counter > 0).float()


def held_at_reset(s, held):
    return s.detach() if held is None else torch.maximum(s.detach(), held)


def count_down(s, counter, n_ref):
    if n_ref is None:
        return counter
    return torch.where(s.detach() > 0, n_ref, (counter - 1).clamp(min=0))


def spike(v, p, held=None):
    s = SurrGradSpike.apply(v - p.theta, p.surr_scale)
    return s if held is None else s * (1 - held)


def mg_block(v, mg_c, mg_a):
    """``(B, N, S)``: each synapse type's Mg block at ``v``, ``1 / (1 + mg_c exp(-mg_a
    v))`` evaluated as ``sigmoid(mg_a v - log mg_c)`` (exactly 1 where ``mg_c = 0``)."""
    return torch.sigmoid(mg_a * v[:, :, None] - torch.log(mg_c))


def membrane(v, s, g, p, g_a=None):
    """Currents and the voltage after the exponential-Euler step, reset where ``s``;
    ``g_a`` ``(B, N)`` the adaptation conductance (by ``E_adapt``), if any."""
    g_total = torch.minimum(g.sum(dim=2).clamp(min=0.0), p.g_clip)
    if getattr(p, "mg_c", None) is not None:  # the block scales each type's conductance
        g_total = g_total * mg_block(v, p.mg_c, p.mg_a)
    I = g_total * (v[:, :, None] - p.E_syn)
    rate = -torch.log1p(p.beta - 1) / p.dt
    g_L = p.C_m * rate
    I_leak = g_L * (v - p.E_L)
    G = g_total.sum(dim=2)
    J = I.sum(dim=2) + I_leak
    if g_a is not None:
        G = G + g_a
        J = J + g_a * (v - p.E_adapt)
    x = p.dt * rate + p.dt * G / p.C_m
    step = -torch.expm1(-x) / (g_L + G)
    s = s.detach()
    v_next = (v - step * J) * (1 - s) + p.U_reset * s
    return v_next, I, I_leak


SUMS = "float32"


def product(a, W):
    """``a @ W`` for a dense pathway, summed as ``SUMS`` says."""
    if SUMS == "exact":
        return (a.double() @ W.double()).float()
    if SUMS != "float32":
        raise ValueError(f"SUMS must be 'float32' or 'exact', got {SUMS!r}")
    return a @ W


def recurrent_activations(drive, s):
    if drive.sparse_recurrent is not None:
        return list(_sparse.activations(drive.sparse_recurrent, s))
    return [product(s[:, rows], W) for rows, W in drive.recurrent]


def feedforward_activations(drive, x, factors=None):
    """``(K_ff, B, T, N)``; a pathway with presynaptic dynamics takes its rows' input
    times its ``factors`` (``network.py:143-157``)."""
    if drive.sparse_feedforward is not None:
        if factors is not None:
            raise NotImplementedError("presynaptic dynamics on a compressed side")
        B, T, n_in = x.shape
        A = _sparse.activations(drive.sparse_feedforward, x.reshape(B * T, n_in))
        return A.reshape(A.shape[0], B, T, -1)
    if SUMS == "float32":
        return drive.feedforward_activations(x, factors)
    B, T = x.shape[:2]
    if not drive.feedforward:
        return x.new_zeros((0, B, T, 0))
    factors = factors or [None] * len(drive.feedforward)
    return torch.stack([product(x[:, :, rows] if f is None else x[:, :, rows] * f, W)
                        for (rows, W), f in zip(drive.feedforward, factors)])


def gate_step(state, s, gate):
    """One step of a pathway's presynaptic variables ``state`` ``(B, width)`` given its
    source rows' activity ``s`` ``(B, n)`` (``network_simulators/network.py:186-223``):
    returns ``(f, state)``, ``s f`` being the pathway's input in place of ``s``.
    Short-term plasticity (Markram, Wang & Tsodyks 1998): ``x <- 1 - (1 - x) d_D``,
    ``u <- U + (u - U) d_F``, ``f = u x / U``, ``x <- x - s u x``, ``u <- u + s U (1 - u)``;
    saturation: ``g <- g d``, ``f <- min(c f (1 - g), 1 - g)`` (``c (1 - g)`` without
    STP), ``g <- min(g + s f, 1)``. Nothing carries a gradient."""
    c, d, U, d_D, d_F = gate.params.unbind()
    n = gate.n
    s = s.detach()
    f, parts = None, []
    if gate.stp:
        u, r = state[:, :n], state[:, n : 2 * n]
        r = 1 - (1 - r) * d_D
        u = U + (u - U) * d_F
        release = u * r
        f = release / U
        r = r - s * release
        u = u + s * U * (1 - u)
        parts += [u, r]
    if gate.saturates:
        g = state[:, -n:] * d
        closed = 1 - g
        f = c * closed if f is None else torch.minimum(c * f * closed, closed)
        parts.append(torch.clamp(g + s * f, max=1.0))
    return f, torch.cat(parts, dim=1)


def gate_feedforward(drive, x, gating):
    """The factors ``(B, T, n_rows)`` of the feedforward pathways with presynaptic
    dynamics (None for the others) over the chunk ``x``, and the gating state after it
    (``network_simulators/network.py:226-250``): a step at a time."""
    K_rec = len(drive.recurrent)
    gates = [drive.gate(K_rec + k) for k in range(len(drive.feedforward))]
    if not any(gates):
        return None, gating
    gating = gating.clone()
    factors = []
    x = x.detach()
    for (rows, _), gate in zip(drive.feedforward, gates):
        if gate is None:
            factors.append(None)
            continue
        state, fs = gating[:, gate.columns], []
        for t in range(x.shape[1]):
            f, state = gate_step(state, x[:, t, rows], gate)
            fs.append(f)
        gating[:, gate.columns] = state
        factors.append(torch.stack(fs, dim=1))
    return factors, gating


def fold(drive):
    """The drive with its dense pathways merged per (side, synapse types made): the
    pathways of a group keep their source rows, each row's weights multiplied by its
    pathway's kernel scale (a float32 product), and the group's scale is 1.

    This restates the identity ``sum_k a_k (jump scale_k made_k) = sum_g (sum_{k in g}
    sum_j s_j W_k[j] scale_k) (jump made_g)`` of the reference's injection
    (``conductance/dynamics.py:95-100,206-208``), which holds for pathways that make the
    same synapse types; the engine evaluates a drive of more pathways than its kernels
    hold this way. Groups keep the order of first appearance, recurrent first. A
    compressed side is left as it is."""
    from wiretorch_amd.network import Drive

    made = drive.made.bool()
    K_rec, K = drive.K_rec, drive.K_rec + drive.K_ff
    out_made, sides = [], []
    for lo, hi, pathways, sparse in ((0, K_rec, drive.recurrent, drive.sparse_recurrent),
                                     (K_rec, K, drive.feedforward, drive.sparse_feedforward)):
        if sparse is not None:
            out_made += [made[k] for k in range(lo, hi)]
            sides.append([])
            continue
        rows_of = {}
        for k in range(lo, hi):
            key = tuple(made[k].tolist())
            rows_of.setdefault(key, []).append(k)
        merged = []
        for key, members in rows_of.items():
            out_made.append(made[members[0]])
            rows = torch.cat([pathways[k - lo][0] for k in members])
            W = torch.cat([pathways[k - lo][1] * drive.scale[k] for k in members], dim=0)
            merged.append((rows, W))
        sides.append(merged)
    N = drive.scale.shape[1]
    return Drive(made=torch.stack(out_made), scale=torch.ones((len(out_made), N)),
                 recurrent=sides[0], feedforward=sides[1],
                 differentiable_inputs=drive.differentiable_inputs,
                 recurrent_gradients=drive.recurrent_gradients,
                 sparse_recurrent=drive.sparse_recurrent,
                 sparse_feedforward=drive.sparse_feedforward)


def stack_steps(tensors):
    return torch.stack([t.contiguous() for t in tensors], dim=1)


def simulate(
    v, g, x, drive, p, *, refractory=None, gating=None, adaptation=None,
    probabilities=False, track=False, track_batch_idx=None, retain=None,
):  # fmt: skip
    """Simulate ``x.shape[1]`` steps from ``(v, g)``; returns a ``Run``."""
    from wiretorch_amd.network import Run

    if any(drive.gate(k) is not None for k in range(len(drive.recurrent))):
        raise NotImplementedError("presynaptic dynamics on recurrent pathways")
    factors, gating = gate_feedforward(drive, x, gating)
    A_ff = feedforward_activations(drive, x, factors)
    kernels = jumps(drive, p.jump)
    keep = (
        slice(None)
        if track_batch_idx is None
        else slice(track_batch_idx, track_batch_idx + 1)
    )
    spikes, probs, tracked = [], [], {"v": [], "I": [], "g": [], "a": []}
    g_a = adaptation if getattr(p, "adapt", None) is not None else None
    if g_a is None and getattr(p, "adapt", None) is not None:
        g_a = torch.zeros_like(v)
    if refractory is None:
        refractory = torch.zeros(v.shape, dtype=torch.int32, device=v.device)
    for t in range(x.shape[1]):
        held = refractory_mask(refractory, p.n_ref)
        s = spike(v, p, held)
        if probabilities:
            prob = torch.sigmoid(p.surr_scale * (v - p.theta))
            probs.append(prob if held is None else prob * (1 - held))
        v_next, I, I_leak = membrane(v, held_at_reset(s, held), g, p, g_a)
        refractory = count_down(s, refractory, p.n_ref)
        if g_a is not None:  # the neuron's own spike raises it (no gradient, as reset)
            g_a = g_a * p.adapt_decay + p.adapt * s.detach()
        s_rec = s if drive.recurrent_gradients else s.detach()
        activations = recurrent_activations(drive, s_rec)
        activations += list(A_ff[:, :, t])
        g = g * p.decay
        for a, kernel in zip(activations, kernels):
            g = g + a[:, :, None, None] * kernel
        v = v_next
        spikes.append(s)
        if retain is not None:
            for tensor in (v, g, s):
                if tensor.requires_grad:
                    tensor.retain_grad()
            retain.append((v, g, s))
        if track:
            tracked["v"].append(v[keep].detach())
            tracked["I"].append(torch.cat([I, I_leak[..., None]], dim=-1)[keep].detach())
            tracked["g"].append(g[keep].detach())
            if g_a is not None:
                tracked["a"].append(g_a[keep].detach())
    return Run(
        output=torch.stack(spikes, dim=1),
        v=v,
        syn=g,
        probabilities=torch.stack(probs, dim=1) if probabilities else None,
        tracked={k: stack_steps(val) for k, val in tracked.items() if val} if track else None,
        refractory=refractory,
        gating=gating,
        adaptation=g_a,
    )
