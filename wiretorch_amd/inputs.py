"""On-device Poisson input: input spikes drawn inside the forward instead of read from a
dense ``(B, T, n_in)`` tensor.

The reference draws Poisson input with ``torch.rand(n_steps, n_neurons) < rate * dt *
1e-3`` per item (``dataloaders/unsupervised.py:80-90``) and hands the network the dense
spike tensor. ``PoissonInput`` stands in for that tensor: a network called with one runs
``wt_cond_run`` with the input drawn on the device from a counter-based generator
(Philox4x32-10, Salmon et al. 2011; ``csrc/wt_philox.h``), so neither the host nor HBM
holds the spikes. Channel ``j`` of trial ``b`` fires at absolute step ``t`` when the top 24
bits of the first word of the generator's output for counter ``(j, t, b, 0)`` under key
``seed``, scaled by 2^-24, are below ``p_j = rate_j * dt * 1e-3`` (float32, as the
reference computes it). Every draw is a pure function of ``(seed, b, t, j)``:

* ``materialize()`` writes the same spikes as a tensor on the device (``wt_poisson_fill``),
  for whatever needs them dense (weight gradients of the input side);
* ``replay()`` recomputes them on the host with numpy — the stream the CPU oracle is
  given, bit for bit the GPU's.

``window(start, stop)`` is the same stream over steps ``start .. stop`` (chunked runs
continue the stream).
"""

from __future__ import annotations

import numpy as np
import torch

from wiretorch_amd import _lib

_M0, _M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
_W0, _W1 = np.uint32(0x9E3779B9), np.uint32(0xBB67AE85)
_LOW = np.uint64(0xFFFFFFFF)


def philox4x32_10(c0, c1, c2, c3, k0, k1):
    """The four output words of Philox4x32-10 for counters ``(c0, c1, c2, c3)`` (uint32
    arrays, broadcast) under key ``(k0, k1)`` — the published algorithm, in numpy."""
    c0, c1, c2, c3 = (np.asarray(c, dtype=np.uint32) for c in (c0, c1, c2, c3))
    k0, k1 = np.uint32(k0), np.uint32(k1)
    with np.errstate(over="ignore"):
        for _ in range(10):
            p0 = _M0 * c0.astype(np.uint64)
            p1 = _M1 * c2.astype(np.uint64)
            hi0, lo0 = (p0 >> np.uint64(32)).astype(np.uint32), (p0 & _LOW).astype(np.uint32)
            hi1, lo1 = (p1 >> np.uint64(32)).astype(np.uint32), (p1 & _LOW).astype(np.uint32)
            c0, c1, c2, c3 = hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0
            k0 = np.uint32(k0 + _W0)
            k1 = np.uint32(k1 + _W1)
    return c0, c1, c2, c3


def firing_probability(rates_hz, dt: float) -> torch.Tensor:
    """``rate * dt * 1e-3`` in float32, as the reference's dataset forms it."""
    return torch.as_tensor(np.asarray(rates_hz, dtype=np.float32)).float() * dt * 1e-3


class PoissonInput:
    """Poisson input spikes of ``batch_size`` trials x ``n_steps`` steps x ``len(rates)``
    channels, drawn on the device where a forward needs them (see the module doc).

    Stands in for the input tensor of a network's ``forward``: it has ``shape``, ``ndim``,
    ``device`` and ``dtype`` (float32) like the dense spike tensor it replaces.
    """

    dtype = torch.float32
    ndim = 3

    def __init__(self, rates_hz, dt: float, batch_size: int, n_steps: int, seed: int,
                 t0: int = 0, device="cuda"):
        self.prob = firing_probability(rates_hz, dt).to(device).contiguous()
        self.dt = float(dt)
        self.seed = int(seed) & 0xFFFFFFFFFFFFFFFF
        self.t0 = int(t0)
        self.shape = torch.Size((int(batch_size), int(n_steps), int(self.prob.numel())))
        if self.t0 < 0 or self.t0 + self.shape[1] > 0xFFFFFFFF:
            raise ValueError("steps must lie in [0, 2^32)")

    @property
    def device(self) -> torch.device:
        return self.prob.device

    @property
    def is_cuda(self) -> bool:
        return self.prob.is_cuda

    @property
    def requires_grad(self) -> bool:
        return False

    def to(self, *args, **kwargs) -> "PoissonInput":
        """Itself (the spikes are float32 wherever they are drawn)."""
        return self

    def window(self, start: int, stop: int) -> "PoissonInput":
        """Steps ``start .. stop`` of the same stream."""
        out = object.__new__(PoissonInput)
        out.prob, out.dt, out.seed = self.prob, self.dt, self.seed
        out.t0 = self.t0 + int(start)
        out.shape = torch.Size((self.shape[0], int(stop) - int(start), self.shape[2]))
        return out

    def materialize(self, stream=None) -> torch.Tensor:
        """The spikes as a ``(B, T, n_in)`` float32 tensor on the device."""
        B, T, n_in = self.shape
        x = torch.empty((B, T, n_in), dtype=torch.float32, device=self.device)
        if stream is None:
            stream = torch.cuda.current_stream(self.device).cuda_stream
        _lib.check(_lib.load().wt_poisson_fill(self.prob.data_ptr(), n_in, self.seed, self.t0,
                                               B, T, x.data_ptr(), stream), "wt_poisson_fill")
        return x

    def replay(self) -> np.ndarray:
        """The spikes recomputed on the host, ``(B, T, n_in)`` bool (numpy)."""
        B, T, n_in = self.shape
        b = np.arange(B, dtype=np.uint32)[:, None, None]
        t = (self.t0 + np.arange(T, dtype=np.uint64)).astype(np.uint32)[None, :, None]
        j = np.arange(n_in, dtype=np.uint32)[None, None, :]
        w0, _, _, _ = philox4x32_10(np.broadcast_to(j, (B, T, n_in)), t, b, np.uint32(0),
                                    self.seed & 0xFFFFFFFF, self.seed >> 32)
        u = (w0 >> np.uint32(8)).astype(np.float32) * np.float32(2.0**-24)
        return u < self.prob.cpu().numpy()[None, None, :]
