"""Paged sparse top-k forward: CPU restatement (test infrastructure only).

Reference ``st/ops/sparse.py:15-174``. Over a logically contiguous KV
``[B,N,H,D]`` (pages are a storage detail and do not change results):

1. exact block scores ``s_j = logsumexp_{i in j} a_i`` for visible blocks
   (``j < p//b - 1``, the block complete inside the KV), ``-inf`` elsewhere
   (``st/ops/sparse.py:15-30``);
2. ``log Z_R`` = logsumexp over ALL visible blocks (``st/ops/sparse.py:132``);
3. top-k block ids per (batch, query, head) in descending score order, ``-1``
   where the score is ``-inf`` (``st/ops/sparse.py:133-139,154``);
4. softmax over the local window (logit ``a_i``) and the selected blocks
   (logit ``a_i + s_j - log Z_R``), output in ``q.dtype``
   (``st/ops/sparse.py:33-65,157-174``).

Tie order: the reference merges pages with ``torch.topk`` whose order among
exactly equal scores is unspecified (``st/ops/sparse.py:134-138``). This
restatement and the HIP kernels both break ties by ascending block id.
"""
import math

import torch
import torch.nn.functional as F

from .dense import _heads, _scores, work_dtype


def block_scores(q, k, positions, block_size, offset=0):
    """``[B,Q,H,G]`` block scores of a KV slab that starts at absolute token
    ``offset`` (``st/ops/sparse.py:15-30``, ``st/ops/kernels/sparse.py:24-33``)."""
    dtype = work_dtype(q)
    b, n = block_size, k.shape[1]
    a = _scores(q, k, dtype)
    groups = -(-n // b)
    padded = F.pad(a, (0, groups * b - n), value=-math.inf)
    s = padded.reshape(*a.shape[:-1], groups, b).logsumexp(-1).transpose(1, 2)
    blocks = torch.arange(groups, device=q.device) + offset // b
    pos = positions[:, :, None, None]
    visible = ((blocks < torch.div(pos, b, rounding_mode="floor") - 1)
               & ((blocks + 1) * b <= offset + n) & (pos >= 0))
    return s.masked_fill(~visible, -math.inf)


def select_topk(scores, topk):
    """Global top-k of ``[B,Q,H,G]`` scores plus ``log Z_R``.

    Returns ``(values, ids, log_zr)``: values descending, ties by ascending
    block id, ``ids = -1`` where the value is ``-inf``; ``log_zr`` is the
    logsumexp over all blocks (``st/ops/sparse.py:121-139,154``)."""
    values, order = torch.sort(scores, dim=-1, descending=True, stable=True)
    values, order = values[..., :topk], order[..., :topk]
    if values.shape[-1] < topk:
        short = topk - values.shape[-1]
        values = F.pad(values, (0, short), value=-math.inf)
        order = F.pad(order, (0, short), value=-1)
    ids = torch.where(torch.isfinite(values), order, torch.full_like(order, -1))
    return values, ids, scores.logsumexp(-1)


def pop(q, k, v, positions, ids, scores, log_zr, block_size):
    """Softmax over the local window and the selected blocks
    (``st/ops/sparse.py:33-65``). Returns ``(out, lse)`` in the work dtype."""
    dtype = work_dtype(q)
    batch, nq, heads, dim = q.shape
    b, n = block_size, k.shape[1]
    topk = ids.shape[-1]
    pos = positions[:, :, None]
    local_block = torch.div(pos, b, rounding_mode="floor") - 1
    slot = torch.arange(b, device=q.device)
    # local slots: blocks p//b-1 and p//b, then the selected blocks
    local_tokens = (local_block[..., None] * b + torch.arange(2 * b, device=q.device))
    local_tokens = local_tokens.expand(batch, nq, heads, 2 * b)
    sel_tokens = (ids[..., None] * b + slot).reshape(batch, nq, heads, topk * b)
    tokens = torch.cat((local_tokens, sel_tokens), -1)
    zr_safe = torch.where(torch.isfinite(log_zr), log_zr, torch.zeros_like(log_zr))
    bias = torch.cat((torch.zeros(batch, nq, heads, 2 * b, dtype=dtype, device=q.device),
                      (scores.to(dtype) - zr_safe[..., None].to(dtype))
                      .repeat_interleave(b, -1)), -1)
    chosen_ok = torch.cat((torch.ones(batch, nq, heads, 2 * b, dtype=torch.bool, device=q.device),
                           ((ids >= 0) & torch.isfinite(scores)).repeat_interleave(b, -1)), -1)
    valid = (chosen_ok & (tokens >= 0) & (tokens < n) & (tokens <= pos[..., None])
             & (pos[..., None] >= 0))
    safe_tokens = tokens.clamp(0, n - 1)
    rows = torch.arange(batch, device=q.device)[:, None, None, None]
    hs = torch.arange(heads, device=q.device)[None, None, :, None]
    kr = k[rows, safe_tokens, hs].to(dtype)
    vr = v[rows, safe_tokens, hs].to(dtype)
    a = (kr * q.to(dtype)[..., None, :]).sum(-1) / math.sqrt(dim) + bias
    a = a.masked_fill(~valid, -math.inf)
    lse = a.logsumexp(-1)
    safe = torch.where(torch.isfinite(lse), lse, torch.zeros_like(lse))
    w = torch.exp(a - safe[..., None])
    out = (w[..., None] * vr).sum(-2)
    return out, lse


def sparse_attention(q, k, v, positions, block_size, topk):
    """Whole sparse forward over a logically contiguous KV.

    Returns ``(out in q.dtype, {"indices", "scores", "log_zr"})`` like
    ``sparse_attention(..., return_selection=True)`` (``st/ops/sparse.py:172-173``)."""
    s = block_scores(q, k, positions, block_size)
    values, ids, log_zr = select_topk(s, topk)
    out, _ = pop(q, k, v, positions, ids, values, log_zr, block_size)
    return out.to(q.dtype), {"indices": ids, "scores": values, "log_zr": log_zr}


def sparse_bytes(heads, dim, elem_bytes, positions, block_size, ids):
    """Algorithmic HBM bytes of one sparse forward: every visible K block is
    scanned once per head, then the K and V of the union of selected and
    local blocks per (batch, head) are read once."""
    b = block_size
    total = 0
    batch = positions.shape[0]
    for bi in range(batch):
        pmax = int(positions[bi].max())
        visible = max(0, pmax // b - 1)
        total += heads * visible * b * dim * elem_bytes
        for h in range(heads):
            chosen = set(int(x) for x in ids[bi, :, h].reshape(-1).tolist() if x >= 0)
            for p in positions[bi].tolist():
                if p >= 0:
                    chosen.update({p // b - 1, p // b})
            chosen.discard(-1)
            total += len(chosen) * b * dim * elem_bytes * 2
    return total
