"""Two-stream speculative decode step, HIP graph capture and paired timing.

Counterpart of the reference harness: ``overlap_run``
(``benchmarks/run_benchmark.py:99-118``), graph capture and batched replay
timing (``benchmarks/critical_path.py:28-62``) and randomized ABBA paired
intervals with a warm-up (``benchmarks/paired_confirm.py:17-157``).

The full decode step is select (stream S) concurrently with speculation on
the already-known predicted list (stream P); the main stream joins both and
runs the repair.  Every kernel is launched by the C ABI on torch's current
stream, so one ``torch.cuda.graph`` capture records the fork/join exactly.
Streams are created at the default priority.
"""
from __future__ import annotations

import random
import statistics
import time

import torch


def _record(obj, stream):
    if isinstance(obj, torch.Tensor):
        obj.record_stream(stream)
    elif isinstance(obj, (list, tuple)):
        for x in obj:
            _record(x, stream)
    elif hasattr(obj, "__dict__"):
        for x in vars(obj).values():
            _record(x, stream)


def overlap_run(selector, speculative, finish, select_stream, predict_stream):
    """select || speculate, join, then finish(selected, prediction)."""
    main = torch.cuda.current_stream()
    select_stream.wait_stream(main)
    predict_stream.wait_stream(main)
    with torch.cuda.stream(select_stream):
        a = selector()
    with torch.cuda.stream(predict_stream):
        state = speculative()
    main.wait_stream(select_stream)
    main.wait_stream(predict_stream)
    # the caching allocator must know that the main stream consumes these
    _record(a, main)
    _record(state, main)
    return finish(a, state)


def across_streams(fns, streams):
    """Run independent requests fns[i]() on streams[i % len(streams)] (one
    fork from the current stream, one join at the end), so that one
    request's latency-bound kernels can overlap the next one's bandwidth-
    bound kernels; returns the outputs in order."""
    main = torch.cuda.current_stream()
    for s in streams:
        s.wait_stream(main)
    outs = []
    for i, fn in enumerate(fns):
        with torch.cuda.stream(streams[i % len(streams)]):
            outs.append(fn())
    for s in streams:
        main.wait_stream(s)
    _record(outs, main)
    return outs


def capture(fn, warmup=3):
    """Warm fn on a side stream, then capture one call into a HIP graph."""
    main = torch.cuda.current_stream()
    side = torch.cuda.Stream()
    side.wait_stream(main)
    with torch.cuda.stream(side):
        for _ in range(warmup):
            fn()
    main.wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    graph.replay()
    torch.cuda.synchronize()
    return graph, out


def warm(graphs, ms=200.0):
    """Replay every graph for at least ``ms`` milliseconds of wall time."""
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for g in graphs:
            for _ in range(20):
                g.replay()
        torch.cuda.synchronize()


def interval_us(graph, replays):
    """Mean microseconds per replay over one batch (events on the current stream)."""
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        graph.replay()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e3 / replays


def paired(graphs: dict, replays=100, rounds=5, seed=20261103, warm_ms=200.0):
    """Randomized ABBA/BAAB paired intervals; median per name (µs/replay)."""
    names = list(graphs)
    rng = random.Random(seed)
    warm(graphs.values(), warm_ms)
    raw = {n: [] for n in names}
    for _ in range(rounds):
        order = names[:]
        rng.shuffle(order)
        for n in order + order[::-1]:
            raw[n].append(interval_us(graphs[n], replays))
    return {n: statistics.median(v) for n, v in raw.items()}, raw


def launch_us(fn, launches=200, warmup=20):
    """Mean microseconds per call of an eager launcher, events around a loop."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(launches):
        fn()
    e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e3 / launches
