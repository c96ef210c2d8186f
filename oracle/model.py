"""Stack model read rounds: per-position loop restatement (test infrastructure only).

The reference checks its model's global read rounds against a per-position
loop (``tests/test_stack_model.py:24-81``): encode once, then for each
supervised position ``t`` and each round, ``q = wq(q_norm(z))``, gated
attention of that one row over raw K/V with at most ``min(topk, groups)``
remote blocks, ``z += read_out(ctx)``, ``z += ffn(ffn_norm(z))``, then
``lm_head(final_norm(z))``. This restatement uses the model's own encoder
and weights and ``dense.loop_attention`` for the attention (itself pinned by
``tests/test_oracle.py``), so it checks the read plumbing (position gathers,
chunking, ``sup``, the dense/sparse dispatch) and the operator integration.

``attention_ops`` gives drop-in replacements of the package's operators,
backed by this oracle, for running the model where no HIP library is loaded
(CPU tests) or as the reference side of a GPU comparison.
"""
import torch

from .dense import eager_attention, loop_attention


def oracle_logits(model, ids, positions):
    """Logits ``[B, len(positions), V]`` at the given positions."""
    b = model.block_size
    batch, n = ids.shape
    groups = -(-n // b)
    keep = None if model.topk >= groups else min(model.topk, groups)
    x, raw_k, raw_v = model.encode(ids)
    outs = []
    for t in positions:
        z = x[:, t:t + 1]
        pos = torch.full((batch, 1), t, dtype=torch.long, device=ids.device)
        for rd in model.reads:
            q = rd.wq(rd.q_norm(z)).reshape(batch, 1, model.heads, model.hd)
            ctx = loop_attention(q, raw_k, raw_v, pos, b, topk=keep)
            z = z + rd.read_out(ctx.reshape(batch, 1, model.dim))
            z = z + rd.ffn(rd.ffn_norm(z))
        outs.append(model.lm_head(model.final_norm(z)))
    return torch.cat(outs, 1)


def dense_op(q, k, v, positions, block_size, backend="auto", q_chunk=32, kv_chunk=1024):
    """``dense_attention`` signature over the vectorised oracle (work dtype
    float32/float64, result in q.dtype)."""
    return eager_attention(q, k, v, positions, block_size)


def sparse_op(q, cache, positions, block_size, topk, backend="auto", **_):
    """``sparse_attention`` signature over the loop oracle (contiguous K/V of
    a ``TensorPages`` cache)."""
    work = torch.float64 if q.dtype == torch.float64 else torch.float32
    out = loop_attention(q.to(work), cache.k.to(work), cache.v.to(work), positions, block_size, topk=topk)
    return out.to(q.dtype)
