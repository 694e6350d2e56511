"""The double-exponential spike-train filter on the CPU — TEST INFRASTRUCTURE ONLY
(see ``oracle/__init__.py``).

``forward`` restates the reference's linear-time recursion
(``src/wiretorch/training_utils/filtering.py:103-123``): per (trial, neuron) column,
``r[t] = a_r r[t-1] + x[t]``, ``s[t] = a_d s[t-1] + r[t]``, the carried state entering
undecayed at ``t = 0``. ``backward`` restates its reverse recursion
(``filtering.py:125-135``). Both run in float32 with every multiply and add rounded
separately (numpy rounds each operation), vectorised over the columns and serial in
time, so the HIP kernels reproduce them bit for bit.

Pinned (``tests/test_filter_oracle.py``): against the reference's own definition in its
tests (``tests/test_losses.py:26-52``, the literal sum ``sum_k a^k x[t-k] + carried a^t``
with chunk carry) evaluated in float64; against the closed form of a single impulse
(``r[t] = a_r^t``, ``s[t] = (a_r^{t+1} - a_d^{t+1}) / (a_r - a_d)``); and the backward
against the adjoint identity ``<g, F x> = <F^T g, x>`` with ``F`` the forward's linear
map, plus torch autograd through the float64 literal sum.
"""

from __future__ import annotations

import numpy as np


def forward(x, a_rise, a_decay, carried_rise=None, carried_smooth=None):
    """``(rise, smooth)`` float32 ``(B, T, N)`` from ``x`` ``(B, T, N)``; carried ``(B, 1, N)``."""
    x = np.asarray(x, dtype=np.float32)
    B, T, N = x.shape
    a_r, a_d = np.float32(a_rise), np.float32(a_decay)
    r = np.zeros((B, N), np.float32) if carried_rise is None else \
        np.asarray(carried_rise, np.float32).reshape(B, N).copy()
    s = np.zeros((B, N), np.float32) if carried_smooth is None else \
        np.asarray(carried_smooth, np.float32).reshape(B, N).copy()
    rise, smooth = np.empty_like(x), np.empty_like(x)
    one = np.float32(1.0)
    for t in range(T):
        kr, kd = (one, one) if t == 0 else (a_r, a_d)
        r = kr * r + x[:, t]
        s = kd * s + r
        rise[:, t], smooth[:, t] = r, s
    return rise, smooth


def backward(grad_smooth, a_rise, a_decay):
    """``dL/dx`` float32 ``(B, T, N)`` from ``dL/dsmooth`` (no gradient through rise)."""
    g = np.asarray(grad_smooth, dtype=np.float32)
    B, T, N = g.shape
    a_r, a_d = np.float32(a_rise), np.float32(a_decay)
    gs = np.zeros((B, N), np.float32)
    gr = np.zeros((B, N), np.float32)
    out = np.empty_like(g)
    for t in range(T - 1, -1, -1):
        gs = g[:, t] + a_d * gs
        gr = gs + a_r * gr
        out[:, t] = gr
    return out
