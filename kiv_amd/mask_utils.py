"""Attention-mask widening for retrieved cold tokens.

Behaviour of ``extend_mask_for_cold`` (kiv/mask_utils.py:8-38): cold columns
are prepended along the last axis and are always attendable (``True`` for
boolean masks, ``0.0`` for additive float masks).
"""

from __future__ import annotations

import torch


def extend_mask_for_cold(mask: torch.Tensor, num_cold: int) -> torch.Tensor:
    fill = True if mask.dtype == torch.bool else 0.0
    lead = list(mask.shape[:-1])
    cold_cols = mask.new_full(lead + [num_cold], fill)
    return torch.cat([cold_cols, mask], dim=-1)
