"""Per-type physiology tables (one entry per cell type or per synapse type), any entry
of any table trainable.

Role of ``src/wiretorch/network_simulators/type_parameters.py:28-79`` in the reference.
The names under which a table lives in a module's state dict are the reference's, so
that checkpoints carry over; everything else is this module's own:

* a table nothing trains is the buffer ``<name>`` ``(n_types,)``;
* a table with trained entries is the buffer ``_<name>_fixed`` (all entries, as given),
  the trained type ids ``_<name>_learnt`` (rebuilt, not saved) and a parameter holding the
  trained entries only — ``log_<name>`` (their logarithms) for a quantity that must stay
  positive, else ``<name>``.

``value(name)`` rebuilds the full table each call (an out-of-place scatter of the trained
entries into the fixed table: differentiable, no host synchronisation).
"""

from __future__ import annotations

from collections.abc import Iterable, Sequence
from dataclasses import dataclass

import torch
from torch import nn


@dataclass(frozen=True)
class _Trained:
    """How one table is trained: which entries, and whether through their logarithm."""

    ids: tuple[int, ...]
    via_log: bool


class TypeParameters(nn.Module):
    """Named per-type tables; ``learnt[name]`` are the type ids trained in ``name``.

    Args:
        values: ``{name: one value per type}`` (index = type id).
        learnt: ``{name: type ids}`` to train; a name given no ids stays fixed.
        positive: names whose trained entries are kept positive (trained as logarithms).
    """

    def __init__(
        self,
        values: dict[str, Sequence[float]],
        learnt: dict[str, Iterable[int]] | None = None,
        positive: Iterable[str] = frozenset(),
    ):
        super().__init__()
        requested = {name: sorted(set(ids)) for name, ids in (learnt or {}).items()}
        stray = sorted(set(requested) - set(values))
        if stray:
            raise AssertionError(f"no table given for the trained parameters {stray}")
        self.names = tuple(values)
        self.positive = frozenset(positive)
        self._plans: dict[str, _Trained] = {}
        for name in self.names:
            table = torch.as_tensor([float(v) for v in values[name]], dtype=torch.float32)
            ids = requested.get(name) or []
            if not ids:
                self.register_buffer(name, table)
                continue
            plan = _Trained(tuple(ids), name in self.positive)
            self._plans[name] = plan
            self.register_buffer(f"_{name}_learnt", torch.tensor(ids, dtype=torch.long),
                                 persistent=False)
            self.register_buffer(f"_{name}_fixed", table)
            start = table[list(ids)]
            if plan.via_log:
                if not bool(torch.all(start > 0)):
                    raise AssertionError(
                        f"{name} is trained as a logarithm and needs positive starting "
                        f"values; got {start.tolist()}"
                    )
                start = torch.log(start)
            self.register_parameter(self._parameter_name(name), nn.Parameter(start))

    @property
    def learnt(self) -> dict[str, list[int]]:
        """``{name: trained type ids}`` for the tables with trained entries."""
        return {name: list(plan.ids) for name, plan in self._plans.items()}

    def _parameter_name(self, name: str) -> str:
        return f"log_{name}" if self._plans[name].via_log else name

    def value(self, name: str) -> torch.Tensor:
        """The full ``(n_types,)`` table of ``name``, differentiable in its trained
        entries."""
        plan = self._plans.get(name)
        if plan is None:
            return getattr(self, name)
        trained = getattr(self, self._parameter_name(name))
        if plan.via_log:
            trained = torch.exp(trained)
        fixed = getattr(self, f"_{name}_fixed")
        return fixed.scatter(0, getattr(self, f"_{name}_learnt"), trained.to(fixed.dtype))


def learnt_types(spec, names: Sequence[str], what: str) -> list[int]:
    """Type ids a ``learn`` entry asks for: ``True`` (every type), an iterable of type
    names, or anything falsy (none)."""
    if not spec:
        return []
    if spec is True:
        return list(range(len(names)))
    wanted = set(spec)
    absent = sorted(wanted - set(names))
    if absent:
        raise AssertionError(f"{what} names types this network lacks: {absent}; its types "
                             f"are {list(names)}")
    return [index for index, name in enumerate(names) if name in wanted]


def learnt_synapses(spec, synapses: list[dict], what: str = "learn") -> list[int]:
    """Registry indices a ``learn`` entry asks for, naming synapse types by ``name``
    (every index carrying that name)."""
    if not spec:
        return []
    if spec is True:
        return list(range(len(synapses)))
    wanted = set(spec)
    absent = sorted(wanted - {syn["name"] for syn in synapses})
    if absent:
        raise AssertionError(f"{what} names synapse types this network lacks: {absent}")
    return [index for index, syn in enumerate(synapses) if syn["name"] in wanted]
