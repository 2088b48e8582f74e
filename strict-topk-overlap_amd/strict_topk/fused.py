"""The whole repair of a kernels.speculate prediction in one launch.

Drop-in for the reference ``strict_topk/fused.py`` (``repair_fused``
:176-220, kernel semantics :48-173): one workgroup per query head performs
membership, retained-state merge, the optional wrong-low subtraction with
its extra-mass budget, late misses, the guards and the inline recompute.
"""
import torch

from . import _lib
from .kernels import RepairResult, _args, _shape, prediction_args


def repair_fused(q, k, v, selected, predicted, prediction,
                 min_remaining=1.e-3, cancellation_tol=1.e-5,
                 max_extra_mass=0.):
    """One workgroup per query head repairs the prediction to the selected set.

    Inputs: finite Q/K/V, ID rows of unique in-range blocks.  The guards
    (remaining low mass, per-coordinate cancellation) are evaluated in the
    low group's own exponent frame, before any rescaling to the final
    maximum.  With max_extra_mass > 0, wrong low blocks may stay in the
    output when their bounded share of the softmax mass is at most that
    value (the head is then reported as approximate).
    """
    h, n, b, d, sa = _shape(q, k, v, selected)
    _, _, _, _, sp = _shape(q, k, v, predicted)
    hybrid = prediction.mode in ("hybrid", "compact")
    if not 0 <= max_extra_mass <= 1:
        raise ValueError("max_extra_mass must be in [0, 1]")
    if hybrid and max_extra_mass > 0 and (prediction.mass_m is None or prediction.mass_l is None):
        raise ValueError("positive max_extra_mass requires speculate(..., keep_mass=True)")
    out = torch.empty((h, d), device=q.device, dtype=torch.float32)
    fallback = torch.empty((h,), device=q.device, dtype=torch.bool)
    remaining = torch.empty((h,), device=q.device, dtype=torch.float32)
    approximate = None
    extra_mass_bound = None
    if max_extra_mass > 0:
        approximate = torch.empty_like(fallback)
        extra_mass_bound = torch.empty_like(remaining)
    _lib.call("stk_repair_fused", *_args(q, k, v), _lib.ptr(selected), _lib.id_code(selected), sa,
              _lib.ptr(predicted), _lib.id_code(predicted), sp, *prediction_args(prediction, q),
              _lib.ptr(prediction.mass_m), _lib.ptr(prediction.mass_l), float(min_remaining),
              float(cancellation_tol), float(max_extra_mass), _lib.ptr(out), _lib.ptr(fallback),
              _lib.ptr(remaining), _lib.ptr(approximate), _lib.ptr(extra_mass_bound),
              _lib.stream(q.device))
    return RepairResult(out, fallback, remaining, approximate, extra_mass_bound)
