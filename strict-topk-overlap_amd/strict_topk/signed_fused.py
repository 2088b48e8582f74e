"""Signed block correction with a shared low-group scale and inline fallback.

Drop-in for the reference ``strict_topk/signed_fused.py``
(``repair_signed_fused`` :148-193): three launches — job schedule, one
parallel signed K/V kernel (hybrid negatives evaluated block-locally and
rescaled to the low frame, compact negatives evaluated in the low frame),
and a guarded finalize with the strict fallback in the same launch.
"""
from .signed_repair import SignedRepairResult, _signed  # noqa: F401


def repair_signed_fused(q, k, v, selected, predicted, prediction, min_remaining=1.e-3,
                        cancellation_tol=1.e-5, max_extra_mass=0.):
    """One shared add/erase KV kernel, followed by guarded finalization.

    Uses three launches: queue metadata; parallel signed KV computation;
    output merge and optional strict fallback.
    """
    return _signed(q, k, v, selected, predicted, prediction, min_remaining, cancellation_tol,
                   max_extra_mass, True, "max_extra_mass must be in [0,1]")
