"""MI355X-native conductance-LIF hot path of wiretorch.

Host side (``network``, ``projections``, ``synapses``, ``type_parameters``,
``connectome``) mirrors the reference's network API; ``engine.simulate`` runs the
hand-written HIP kernels (``csrc/``) through the C-ABI library ``libwiretorch_amd.so``.
"""

from wiretorch_amd.network import (  # noqa: F401
    ConductanceLIFNetwork,
    Drive,
    FeedforwardConductanceLIFNetwork,
    Physiology,
    Run,
)
