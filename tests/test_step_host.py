"""Host-side checks of the fused step's Python layer (no GPU): the outputs
an allocation-free call writes into are validated before any launch, and
every operand's alignment decides between the fused and the composed path."""
import pytest
import torch


def test_step_into_is_checked_before_any_launch():
    """speculative_step_noalloc's ``into``: every tensor's shape, dtype,
    device and layout is checked (ValueError) before the C call."""
    from strict_topk import step
    from strict_topk.kernels import PartialState
    hq, sp, topk, d = 4, 8, 6, 64
    dev = torch.device("cpu")

    def good():
        return step.StepResult(torch.zeros((hq, topk), dtype=torch.int32),
                               PartialState(torch.zeros((hq, sp)), torch.zeros((hq, sp)),
                                            torch.zeros((hq, sp, d))),
                               torch.zeros((hq, d)))
    step.check_into(good(), hq, sp, topk, d, dev)
    bad = []
    r = good(); r.selected = torch.zeros((hq, topk + 1), dtype=torch.int32); bad.append(r)
    r = good(); r.selected = torch.zeros((hq, topk), dtype=torch.int64); bad.append(r)
    r = good(); r.state.m = torch.zeros((hq, sp - 1)); bad.append(r)
    r = good(); r.state.l = torch.zeros((hq, sp), dtype=torch.float64); bad.append(r)
    r = good(); r.state.u = torch.zeros((hq, d, sp)).transpose(1, 2); bad.append(r)
    r = good(); r.state.u = torch.zeros((hq, sp, d + 1)); bad.append(r)
    r = good(); r.output = torch.zeros((hq + 1, d)); bad.append(r)
    for r in bad:
        with pytest.raises(ValueError):
            step.check_into(r, hq, sp, topk, d, dev)
    with pytest.raises(ValueError):
        step.check_into(good(), hq, sp, topk, d, torch.device("meta"))


def test_step_supported_checks_every_operand_alignment():
    """A misaligned V or HI view makes ``supported`` false, so the step takes
    its composed path instead of failing in the fused one."""
    from strict_topk import step
    hq, hkv, n, b, d = 8, 2, 64, 32, 128
    q = torch.zeros((hq, d), dtype=torch.bfloat16)
    k = torch.zeros((hkv, n, b, d), dtype=torch.bfloat16)
    lo = torch.zeros((hkv, n, d), dtype=torch.bfloat16)
    p = torch.zeros((hq, 16), dtype=torch.int32)
    v_bad = torch.zeros(k.numel() + 1, dtype=torch.bfloat16)[1:].view(k.shape)
    hi_bad = torch.zeros(lo.numel() + 1, dtype=torch.bfloat16)[1:].view(lo.shape)
    assert step.supported(q, k, lo, 16, p, k.clone(), lo.clone())
    assert not step.supported(q, k, lo, 16, p, v_bad, lo.clone())
    assert not step.supported(q, k, lo, 16, p, k.clone(), hi_bad)
