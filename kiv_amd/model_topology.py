"""Head geometry and layer roles of a model, as the tiered cache sees them.

Same fields, invariants and ``manual`` constructor as the reference's
``ModelTopology`` (kiv/model_topology.py:9-84).
"""

from __future__ import annotations

from dataclasses import dataclass, field


def _extras(found: set, allowed: set) -> list:
    return sorted(found - allowed)


@dataclass(frozen=True)
class ModelTopology:
    """Which layers attend globally, which own a cold store, and head sizes.

    Invariants checked at construction:
      * independent_kv_layers is a subset of global_layer_indices;
      * every kv_sharing_map key is a global layer;
      * every kv_sharing_map value is an independent layer (owns a store).
    """

    model_family: str
    num_hidden_layers: int
    global_layer_indices: tuple[int, ...]
    independent_kv_layers: tuple[int, ...]
    kv_sharing_map: dict[int, int] = field(default_factory=dict)
    num_query_heads: int = 0
    num_kv_heads: int = 0
    head_dim: int = 0

    def __post_init__(self) -> None:
        glob = set(self.global_layer_indices)
        indep = set(self.independent_kv_layers)
        bad = _extras(indep, glob)
        if bad:
            raise ValueError(
                f"independent_kv_layers must be a subset of global_layer_indices; extras: {bad}"
            )
        bad = _extras(set(self.kv_sharing_map), glob)
        if bad:
            raise ValueError(
                f"kv_sharing_map keys must all appear in global_layer_indices; extras: {bad}"
            )
        bad = _extras(set(self.kv_sharing_map.values()), indep)
        if bad:
            raise ValueError(
                f"kv_sharing_map values must all appear in independent_kv_layers; extras: {bad}"
            )

    @property
    def num_kv_groups(self) -> int:
        return self.num_query_heads // self.num_kv_heads if self.num_kv_heads else 0

    @staticmethod
    def manual(
        *,
        global_layer_indices: tuple[int, ...],
        num_query_heads: int,
        num_kv_heads: int,
        head_dim: int,
        num_hidden_layers: int,
        independent_kv_layers: tuple[int, ...] | None = None,
        kv_sharing_map: dict[int, int] | None = None,
        model_family: str = "unknown",
    ) -> "ModelTopology":
        """Build a topology by hand; independents default to all globals."""
        return ModelTopology(
            model_family=model_family,
            num_hidden_layers=num_hidden_layers,
            global_layer_indices=tuple(global_layer_indices),
            independent_kv_layers=tuple(
                global_layer_indices if independent_kv_layers is None else independent_kv_layers
            ),
            kv_sharing_map=dict(kv_sharing_map or {}),
            num_query_heads=num_query_heads,
            num_kv_heads=num_kv_heads,
            head_dim=head_dim,
        )
