"""The rate-network engine on MI355X (HIP kernels through ``libwiretorch_amd.so``)."""

from __future__ import annotations


def simulate(v, I, x, drive, p, *, probabilities=False, track=False, track_batch_idx=None,
             retain=None):
    raise NotImplementedError("the rate-network kernels are not built yet")
