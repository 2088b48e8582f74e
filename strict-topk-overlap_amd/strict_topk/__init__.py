"""Strict-set speculative sparse attention on hand-written gfx950 HIP kernels."""
from .kernels import (PartialState, Prediction, RepairResult, block_partials,
                      merge_partials, exact_attention, speculate, repair,
                      touch_kv)

__all__ = ["PartialState", "Prediction", "RepairResult", "block_partials",
           "merge_partials", "exact_attention", "speculate", "repair", "touch_kv"]
