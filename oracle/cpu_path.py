"""Host-CPU torch restatement of the reference's decode step (CPU baseline).

TEST INFRASTRUCTURE ONLY.  Only ``bench.py``'s ``cpu_baseline`` leg and
``tests/`` use this module; the product path never imports it.

It restates, in float32 torch on the CPU, the reference's torch path for one
decode step:
  * selector: ``torch.where(q >= 0, hi * q, lo * q).sum(-1)`` then
    ``topk(sorted=False)`` (``benchmarks/run_benchmark.py:50-51``), with the
    native GQA mapping of ``strict_topk/gqa.py:15-26`` (query head h reads KV
    head h // G);
  * attention over the selected blocks: gather, ``einsum`` logits scaled by
    D**-0.5, softmax over all selected tokens, ``einsum`` with V
    (``benchmarks/critical_path.py:16-25``, computed in float32 here).
The full speculative step on one CPU has no concurrency to exploit, so the
baseline is this serial step.
"""
from __future__ import annotations

import math
import os
import time

import torch


def select(q, lo, hi, topk):
    hq, d = q.shape
    hkv, n, _ = lo.shape
    g = hq // hkv
    qf = q.float().view(hkv, g, 1, d)
    scores = torch.where(qf >= 0, hi[:, None] * qf, lo[:, None] * qf).sum(-1)
    return scores.view(hq, n).topk(topk, sorted=False).indices.to(torch.int32)


def attend(q, k, v, ids):
    hq, d = q.shape
    g = hq // k.shape[0]
    heads = torch.arange(hq) // g
    keys = k[heads[:, None], ids.long()].float()       # [hq, s, b, d]
    values = v[heads[:, None], ids.long()].float()
    logits = torch.einsum("hd,hsbd->hsb", q.float(), keys) / math.sqrt(d)
    w = logits.flatten(1).softmax(-1).view_as(logits)
    return torch.einsum("hsb,hsbd->hd", w, values)


def serial_step(q, k, v, lo, hi, topk):
    return attend(q, k, v, select(q, lo, hi, topk))


def time_serial(q, k, v, lo, hi, topk, budget_s=10.0, max_steps=2000):
    """Time serial steps on all host cores this process may use.

    Runs whole steps until ``budget_s`` seconds have passed (at least one).
    Returns (microseconds per step, steps, threads).
    """
    threads = len(os.sched_getaffinity(0))
    old = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        serial_step(q, k, v, lo, hi, topk)    # warm the allocator
        steps = 0
        t0 = time.perf_counter()
        while True:
            serial_step(q, k, v, lo, hi, topk)
            steps += 1
            el = time.perf_counter() - t0
            if el >= budget_s or steps >= max_steps:
                break
        return el * 1e6 / steps, steps, threads
    finally:
        torch.set_num_threads(old)


def time_oracle(q, k, v, lo, hi, topk, budget_s=5.0, max_steps=50):
    """Time the FP64 oracle's serial step (bound scores in the fixed order,
    top-K, FP64 attention over the selected blocks), the reference's own
    FP64 torch path restated in numpy.  Returns (microseconds per step,
    steps)."""
    from . import stk_oracle as O
    qn = q.double().numpy()
    kn, vn = k.double().numpy(), v.double().numpy()
    lon, hin = lo.double().numpy(), hi.double().numpy()
    steps = 0
    t0 = time.perf_counter()
    while True:
        ids = O.select_blocks(qn, lon, hin, topk)
        O.attention(qn, kn, vn, ids)
        steps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or steps >= max_steps:
            break
    return el * 1e6 / steps, steps
