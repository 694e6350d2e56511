"""Short-term plasticity of release, per (source cell type, target cell type) connection
(the reference's ``network_simulators/stp.py``): each source neuron keeps, per connection
type with STP, its resources ``x`` (1 at rest) and its release probability ``u`` (``U`` at
rest); ``x`` recovers with ``tau_D`` and ``u`` relaxes with ``tau_F`` between spikes, a
spike releases ``u x`` and raises ``u`` by ``U (1 - u)``, and its input is the release
over ``U`` (Markram, Wang & Tsodyks 1998). The step itself is ``gate_step`` of the
engine's oracle and ``wt_gate_scan`` on the GPU."""

from __future__ import annotations

import math
from dataclasses import dataclass


@dataclass(frozen=True)
class STP:
    """One connection type's plasticity: ``U`` in (0, 1], ``tau_D`` > 0 ms, ``tau_F`` >= 0
    ms (0: depression only)."""

    U: float
    tau_D: float
    tau_F: float = 0.0

    def __post_init__(self):
        if not 0 < self.U <= 1:
            raise ValueError(f"STP: U must be in (0, 1], got {self.U}")
        if not self.tau_D > 0:
            raise ValueError(f"STP: tau_D must be > 0 ms, got {self.tau_D}")
        if not self.tau_F >= 0:
            raise ValueError(f"STP: tau_F must be >= 0 ms, got {self.tau_F}")

    def decays(self, dt: float) -> tuple[float, float]:
        """Per-step decays of the resources' deficit and of the facilitation."""
        return math.exp(-dt / self.tau_D), math.exp(-dt / self.tau_F) if self.tau_F > 0 else 0.0


#: Depressing connections (pyramidal onto pyramidal; Tsodyks & Markram 1997).
DEPRESSING = STP(U=0.5, tau_D=800.0, tau_F=0.0)
#: Facilitating connections (pyramidal onto interneuron; Tsodyks, Pawelzik & Markram 1998).
FACILITATING = STP(U=0.03, tau_D=130.0, tau_F=530.0)


def as_stp(value) -> STP:
    """An ``STP``, from one or from a dict of its fields."""
    return value if isinstance(value, STP) else STP(**value)
