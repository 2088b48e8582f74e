"""GQA attention over many small blocks, states reduced in two levels.

Drop-in for the reference ``strict_topk/gqa_hierarchical.py`` (``partials``
:55-61, ``exact`` :111-112, ``repair_saved`` :133-134,
``repair_saved_shared`` :137-144): per-block states, a level-1 merge of 32
positions and a final LSE merge.  The LSE merge is associative, so the
library merges in the order its kernels like: ``exact`` computes one state
per pack of 32 tokens for a whole KV group on the matrix cores
(``k_hier_mfma``, 8-16 query heads per KV head at D = 128) or on the vector
units (``k_states_pack_comb``), four packs merged in LDS, then one merge
over the packs; the repairs take the hits' states from the prediction and
recompute the rest the same way; ``partials`` returns per-block states.
"""
import torch

from . import _lib, gqa
from .kernels import _args


def partials(q, k, v, selected):
    return gqa.partials(q, k, v, selected)


def exact(q, k, v, selected):
    h, n, b, d, group, sa = gqa._shape(q, k, v, selected)
    out = torch.empty((h, d), device=q.device, dtype=torch.float32)
    ws = _lib.workspace(_lib.size("stk_hier_exact_workspace_bytes", h, sa, d), q.device)
    _lib.call("stk_hier_exact", *_args(q, k, v), _lib.ptr(selected), _lib.id_code(selected), sa,
              _lib.ptr(out), _lib.ptr(ws), ws.numel(), _lib.stream(q.device))
    return out


def _repair(q, k, v, selected, predicted, state, shared):
    h, n, b, d, group, sa = gqa._shape(q, k, v, selected)
    gqa._validate_ids(q, predicted)
    sp = predicted.shape[1]
    if state.u.shape != (h, sp, d) or state.m.shape != (h, sp) or state.l.shape != (h, sp):
        raise ValueError('prediction state shape does not match predicted blocks')
    out = torch.empty((h, d), device=q.device, dtype=torch.float32)
    ws = _lib.workspace(_lib.size("stk_hier_repair_workspace_bytes", h, sa, d, int(shared)),
                        q.device)
    _lib.call("stk_hier_repair", *_args(q, k, v), _lib.ptr(selected), _lib.id_code(selected), sa,
              _lib.ptr(predicted), _lib.id_code(predicted), sp, _lib.ptr(state.m),
              _lib.ptr(state.l), _lib.ptr(state.u), 1 if shared else 0, _lib.ptr(out),
              _lib.ptr(ws), ws.numel(), _lib.stream(q.device))
    return out


def repair_saved(q, k, v, selected, predicted, state):
    return _repair(q, k, v, selected, predicted, state, False)


def repair_saved_shared(q, k, v, selected, predicted, state):
    """repair_saved for a selection shared by all heads (an indexer's).

    The caller guarantees that every row of ``selected`` is the same list in
    the same order, and likewise for ``predicted``; this is not checked.
    Hits and misses are looked up from row 0 only, while each query head
    still has its own states and output.
    """
    return _repair(q, k, v, selected, predicted, state, True)
