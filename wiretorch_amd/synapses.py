"""Synapse types of every input side, under one index.

A conductance-based network keeps one conductance per synapse type per neuron, each
with a rise and a decay component. Synapse types are made by the source cell types of
each input side (the network's own neurons, external inputs). With ``unify=True`` two
types with the same signature ``(source cell type name, synapse name)`` share one
index, so e.g. AMPA made by excitatory neurons on both sides is one conductance.

Follows ``src/wiretorch/network_simulators/synapses.py:18-86`` (index order: sides in
order, each side's types in the order given; unification by signature).

Extension for networks of many cell types: an entry's ``cell_id`` may list several
source cell types, all of which make that synapse type (the reference needs one entry
per cell type, hence one synapse type per cell type at fly scale). An entry whose
``cell_id`` is a list has the signature ``(None, synapse name)``: unified, two sides'
listed entries of one name share one index.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class SynapseRegistry:
    """Every side's synapse types under one index.

    ``synapses`` holds one parameter dict per index (with ``unified_synapse_id`` and
    ``signature`` added); ``to_index[side]`` maps that side's ``synapse_id`` to it.
    """

    synapses: list[dict]
    to_index: list[dict[int, int]]

    @classmethod
    def build(cls, sides, unify: bool) -> "SynapseRegistry":
        """Index the synapse types of each ``(cell_params, synapse_params)`` side."""
        entries: list[dict] = []
        index_of: dict[tuple, int] = {}
        maps: list[dict[int, int]] = []
        for side_no, (cells, side_synapses) in enumerate(sides):
            cell_name = {c["cell_id"]: c["name"] for c in cells}
            order = (
                list(side_synapses)
                if unify
                else sorted(side_synapses, key=lambda syn: syn["synapse_id"])
            )
            mapping: dict[int, int] = {}
            for syn in order:
                maker = None if _listed(syn) else cell_name[syn["cell_id"]]
                signature = (maker, syn["name"])
                key = signature if unify else (side_no, syn["synapse_id"])
                if key not in index_of:
                    index_of[key] = len(entries)
                    entries.append(
                        dict(syn, unified_synapse_id=len(entries), signature=signature)
                    )
                mapping[syn["synapse_id"]] = index_of[key]
            maps.append(mapping)
        return cls(entries, maps)

    def __len__(self) -> int:
        return len(self.synapses)

    def table(self, name: str, default: float | None = None) -> torch.Tensor:
        """One parameter per index as float32 (``default`` where a type omits it)."""
        values = [
            syn[name] if default is None else syn.get(name, default)
            for syn in self.synapses
        ]
        return torch.tensor(values, dtype=torch.float32)

    def made_by(self, side: int, synapse_params: list[dict]) -> dict[int, torch.Tensor]:
        """Per source cell type of ``side`` (ascending id), which indices it makes."""
        out: dict[int, torch.Tensor] = {}
        for syn in synapse_params:
            for cell in _makers(syn):
                mask = out.get(cell)
                if mask is None:
                    mask = out[cell] = torch.zeros(len(self), dtype=torch.bool)
                mask[self.to_index[side][syn["synapse_id"]]] = True
        return {k: out[k] for k in sorted(out)}


def _listed(syn: dict) -> bool:
    """Whether an entry names its source cell types as a list (the extension)."""
    return isinstance(syn["cell_id"], (list, tuple, range))


def _makers(syn: dict) -> list[int]:
    """The source cell types an entry names: one ``cell_id``, or a list of them."""
    return [int(c) for c in syn["cell_id"]] if _listed(syn) else [int(syn["cell_id"])]


#: The Mg block's parameter defaults: no block (``mg``, mM), the Jahr-Stevens voltage
#: slope (``mg_slope``, 1/mV) and dissociation constant (``mg_k``, mM)
#: (``conductance/synapses.py:39-41``).
MG, MG_SLOPE, MG_K = 0.0, 0.062, 3.57


def mg_block_tables(registry: "SynapseRegistry") -> dict[str, torch.Tensor]:
    """Per synapse type the voltage-dependent Mg block ``B(v) = 1 / (1 + mg_c exp(-mg_a
    v))`` that scales its current: ``mg_c = mg / mg_k``, ``mg_a = mg_slope``; ``mg = 0``
    (a type without one) gives ``B = 1`` (``conductance/synapses.py:44-56``)."""
    mg = registry.table("mg", default=MG)
    if bool((mg < 0).any()):
        raise ValueError("synapse params: a negative Mg concentration")
    return {"mg_c": mg / registry.table("mg_k", default=MG_K),
            "mg_a": registry.table("mg_slope", default=MG_SLOPE)}
