"""Signed repair whose corrections share one launch and whose fallback is inline.

Drop-in for the reference ``strict_topk/signed_fused.py``
(``repair_signed_fused`` :148-193). Saved and hybrid predictions in bf16 /
fp16 with D in {64, 128, 256}, B a multiple of 16, at most 256 selected and
predicted slots, SP * D <= 32768 and 16-byte aligned tensors run in one
launch (``k_srepair``: schedule, signed corrections and the guarded merge
with the strict fallback, one workgroup per query head). Other cases take
three launches: the job schedule, one parallel signed K/V kernel (hybrid
negatives evaluated block-locally and rescaled to the low frame, compact
negatives in the low frame), and a guarded finalize with the strict fallback
in the same launch.
"""
from .signed_repair import SignedRepairResult, _signed  # noqa: F401


def repair_signed_fused(q, k, v, selected, predicted, prediction, min_remaining=1.e-3,
                        cancellation_tol=1.e-5, max_extra_mass=0.):
    """Repair by signed block corrections: the added (missed) and subtracted
    (wrong low) blocks' states, then the guarded merge, which also recomputes
    the strict selected set for heads whose guards fail; one launch where
    the shape allows it, otherwise three (module docstring)."""
    return _signed(q, k, v, selected, predicted, prediction, min_remaining, cancellation_tol,
                   max_extra_mass, True, "max_extra_mass must be in [0,1]")
