"""Algorithm and budget parameters for the tiered KV cache.

Mirrors ``KIVConfig`` of the reference (kiv/config.py:6-26): the first five
fields keep their names, order and defaults so that positional and keyword
construction behave the same.  The trailing fields are MI355X placement
knobs with defaults that keep the reference's behaviour.
"""

from __future__ import annotations

from dataclasses import dataclass


@dataclass
class KIVConfig:
    """Tiered-cache parameters.

    hot_budget       exact K/V tokens kept in HBM per global layer.
    top_p            cold tokens handed to attention per decode step.
    page_size        tokens per cold page (one mean-K summary per page).
    top_pages        pages picked per query head by the coarse pass.
    prefetch_stream  accepted for API compatibility; the HIP path reads cold
                     rows in-kernel, so there is no separate copy stream.
    cold_tier        where evicted K/V rows live: "host" (pinned, mapped host
                     memory read zero-copy by the kernels, the reference's
                     placement), "hbm" (device memory) or "split" (K rows in
                     HBM, where the fine scan reads every union page; V rows
                     in host memory, of which only the selected rows are read).
    score_rounding   "activation": round scores to the activation dtype after
                     the dot product and again after scaling, as the
                     reference's dtype matmul does (kiv/cold_store.py:206-208);
                     "fp32": rank on the fp32 scores.
    reserve_tokens   optional capacity hint; the store pre-sizes its page
                     arrays for this many cold tokens.
    fine_pruning     host tier, opt-in: the coarse scan also bounds each
                     page's token scores (from the page's summary and
                     radius), and the fine scan reads only the union pages
                     whose bound can reach the top P, which cuts host-link
                     reads (NS shape: 20 MB -> 1.3 MB per step).  Selected
                     tokens, their order and the returned rows are the same
                     as without it; the fine telemetry's mean_score then
                     averages the scored candidates only, so the default
                     (off) keeps the reference's telemetry exactly.
    """

    hot_budget: int = 2048
    top_p: int = 256
    page_size: int = 128
    top_pages: int = 32
    prefetch_stream: bool = True
    cold_tier: str = "host"
    score_rounding: str = "activation"
    reserve_tokens: int = 0
    fine_pruning: bool = False

    def __post_init__(self) -> None:
        if self.cold_tier not in ("host", "hbm", "split"):
            raise ValueError(f"cold_tier must be 'host', 'hbm' or 'split', got {self.cold_tier!r}")
        if self.score_rounding not in ("activation", "fp32"):
            raise ValueError(
                f"score_rounding must be 'activation' or 'fp32', got {self.score_rounding!r}"
            )
        if self.page_size < 1:
            raise ValueError("page_size must be >= 1")
