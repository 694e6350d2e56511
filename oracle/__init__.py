"""CPU oracle for the conductance-LIF hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithm the HIP kernels must
reproduce. It is the checker: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and never as the thing measured or
shipped. The product path (``wiretorch_amd``) never imports it and has no CPU fallback.

Modules:

* ``oracle.dynamics`` — ``simulate`` restated op for op from the reference's PyTorch
  step ``src/wiretorch/network_simulators/conductance/dynamics.py:95-237``, with the
  surrogate spike of ``src/wiretorch/training_utils/surrogate_gradients.py:9-33``.
  Gradients come from torch autograd through the restated step, as in the reference.
  Pinned by the reference's recorded fixtures (``tests/golden/reference/*.npz``:
  lockstep, free run, gradients), see ``tests/test_oracle_fixtures.py``. Its optional
  terms, which no fixture exercises: the Mg block (``dynamics.py:110-129``) by the
  tracked currents against ``B G (v - E)`` in float64 and the block-free network bit for
  bit (``tests/test_nmda.py``); adaptation (``dynamics.py:116-143,200-202``) by the
  exact solution of the membrane with the adaptation conductance held over a step, the
  tracked adaptation against its recursion from the spikes, and the non-adapting network
  bit for bit (``tests/test_adaptation.py``); presynaptic dynamics of feedforward
  pathways (``gate_step`` / ``gate_feedforward``, ``network_simulators/network.py:
  186-250``) by short-term plasticity's factors against the event-by-event map of
  Markram, Wang & Tsodyks (1998) and saturation against its recursion, both in float64
  (``tests/test_gating.py``).
* ``oracle.sparse`` — the compressed-connectome propagation used at fly scale, where
  the reference's dense per-pathway rows cannot be built. Pinned against the dense
  product on small networks (``tests/test_oracle_pinning.py``,
  ``test_sparse_activations_equal_the_dense_product``).
* ``oracle.filtering`` — the spike-train losses' double-exponential filter and its
  reverse (``src/wiretorch/training_utils/filtering.py:103-135``). Pinned against the
  reference tests' literal-sum definition, an impulse's closed form and the adjoint
  identity (``tests/test_filter_oracle.py``).
"""
