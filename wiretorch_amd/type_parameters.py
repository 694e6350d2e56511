"""Physiology values with one entry per type, any of them learnt.

Per cell type (membrane time constant, threshold, ...) or per synapse type (synaptic
time constants, reversal potential, peak conductance). Learnt entries are parameters;
positive quantities are learnt as their logarithm so they stay positive. Follows
``src/wiretorch/network_simulators/type_parameters.py:28-79``.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch
from torch import nn


class TypeParameters(nn.Module):
    """``{name: per-type values}``; ``learnt[name]`` lists the type ids trained."""

    def __init__(
        self,
        values: dict[str, Sequence[float]],
        learnt: dict[str, Sequence[int]] | None = None,
        positive=frozenset(),
    ):
        super().__init__()
        learnt = dict(learnt or {})
        unknown = set(learnt) - set(values)
        assert not unknown, f"cannot learn unknown parameters {sorted(unknown)}"
        self.names = tuple(values)
        self.positive = frozenset(positive)
        self.learnt: dict[str, list[int]] = {}
        for name, raw in values.items():
            full = torch.tensor([float(v) for v in raw], dtype=torch.float32)
            types = sorted(set(learnt.get(name, ())))
            if not types:
                self.register_buffer(name, full)
                continue
            self.learnt[name] = types
            which = torch.tensor(types, dtype=torch.long)
            self.register_buffer(f"_{name}_learnt", which, persistent=False)
            self.register_buffer(f"_{name}_fixed", full)
            start = full[which]
            if name in self.positive:
                assert bool((start > 0).all()), (
                    f"a learnt {name} must be positive, got {start.tolist()}"
                )
                self.register_parameter(f"log_{name}", nn.Parameter(start.log()))
            else:
                self.register_parameter(name, nn.Parameter(start))

    def value(self, name: str) -> torch.Tensor:
        """``(n_types,)``: fixed values with the learnt types' current values in place."""
        if name not in self.learnt:
            return getattr(self, name)
        trained = (
            getattr(self, f"log_{name}").exp()
            if name in self.positive
            else getattr(self, name)
        )
        base = getattr(self, f"_{name}_fixed")
        return base.index_put((getattr(self, f"_{name}_learnt"),), trained)


def learnt_types(spec, names: Sequence[str], what: str) -> list[int]:
    """Type ids from a ``learn`` entry: True (all), a list of names, or falsy."""
    if not spec:
        return []
    if spec is True:
        return list(range(len(names)))
    missing = set(spec) - set(names)
    assert not missing, f"{what}: unknown types {sorted(missing)} (have {list(names)})"
    return [i for i, n in enumerate(names) if n in spec]


def learnt_synapses(spec, synapses: list[dict], what: str = "learn") -> list[int]:
    """Registry indices from a ``learn`` entry naming synapse types by name."""
    if not spec:
        return []
    if spec is True:
        return list(range(len(synapses)))
    known = {s["name"] for s in synapses}
    missing = set(spec) - known
    assert not missing, f"{what}: unknown synapses {sorted(missing)}"
    return [i for i, s in enumerate(synapses) if s["name"] in spec]
