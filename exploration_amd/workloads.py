"""Seeded synthetic workloads of the benchmark configurations and their
algorithmic work counts (FLOP for the dense operator, HBM bytes for the
sparse one). Used by ``bench.py`` and the tests; nothing here is timed.
"""
import math

import torch


def _gen(seed, device):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def dense_inputs(batch, queries, length, heads, dim, dtype, seed=0, scale=1.0, device="cpu",
                 positions=None):
    """q [B,Q,H,D], k/v [B,N,H,D] ~ N(0,1)*scale and dO ~ N(0,1), drawn in this
    order from one generator; positions default to the last ``queries``
    positions of ``length`` (``arange`` when queries == length)."""
    g = _gen(seed, device)
    shape_q, shape_k = (batch, queries, heads, dim), (batch, length, heads, dim)
    q = torch.randn(shape_q, generator=g, device=device, dtype=torch.float32) * scale
    k = torch.randn(shape_k, generator=g, device=device, dtype=torch.float32) * scale
    v = torch.randn(shape_k, generator=g, device=device, dtype=torch.float32) * scale
    do = torch.randn(shape_q, generator=g, device=device, dtype=torch.float32)
    if positions is None:
        positions = torch.arange(length - queries, length, device=device)[None].expand(batch, -1)
    positions = torch.as_tensor(positions, device=device, dtype=torch.int64).contiguous()
    return q.to(dtype), k.to(dtype), v.to(dtype), positions, do.to(dtype)


# BASELINE.json configurations (dense)
CFG1 = dict(batch=2, queries=512, length=512, heads=4, dim=64, block=64, dtype=torch.float32, seed=0, scale=1.0)
CFG2 = dict(batch=1, queries=4096, length=4096, heads=8, dim=128, block=128, dtype=torch.bfloat16, seed=0,
            scale=1.0 / math.sqrt(128))
CFG3 = dict(batch=1, queries=5, length=385, heads=4, dim=128, block=128, dtype=torch.float32, seed=0, scale=1.0)


def dense_config(cfg, device="cpu"):
    c = dict(cfg)
    block = c.pop("block")
    q, k, v, pos, do = dense_inputs(device=device, **c)
    return q, k, v, pos, do, block


def dense_flops(positions, n_keys, heads, dim):
    """Algorithmic FLOP of one dense forward+backward: ``14 H D sum(p+1)``
    over valid rows (2 forward and 5 backward matmuls over each row's causal
    prefix; recomputation excluded)."""
    lengths = (positions.clamp(max=n_keys - 1) + 1).clamp(min=0)
    return 14 * heads * dim * int(lengths.sum())


def dense_forward_flops(positions, n_keys, heads, dim):
    lengths = (positions.clamp(max=n_keys - 1) + 1).clamp(min=0)
    return 4 * heads * dim * int(lengths.sum())


# ---------------------------------------------------------------------------
# sparse: cfg4 with planted blocks

CFG4 = dict(batch=1, heads=8, length=1 << 20, queries=16, dim=128, block=128, topk=64, page_tokens=128,
            dtype=torch.bfloat16, seed=0)


def planted_alphas(topk):
    """Strictly decreasing plant strengths, one per rank."""
    return torch.linspace(2.5, 1.25, topk)


def planted_sparse(batch, heads, length, queries, dim, block, topk, page_tokens, dtype, seed=0,
                   device="cuda", noise=0.05, paged=True):
    """KV ~ N(0,1) with ``topk`` planted blocks per (query, head).

    Queries sit at the last ``queries`` positions. For every (batch, head) the
    planted blocks of different queries are distinct visible blocks; block r
    of query t holds keys ``alpha_r sqrt(D) q_hat + noise N(0,1)`` so its
    score exceeds every unplanted block by a wide margin and the expected
    selection is the planted ids in rank order. Pages of ``page_tokens``
    tokens are placed in the pool by a seeded random permutation.

    Returns ``(q, cache, positions, expected_ids)`` with ``cache`` a PagedKV
    (or ``(k, v)`` when ``paged=False``) and expected ids ``[B,Q,H,topk]``.
    """
    from .sparse import PagedKV

    g = _gen(seed, device)
    k = torch.randn((batch, length, heads, dim), generator=g, device=device, dtype=dtype)
    v = torch.randn((batch, length, heads, dim), generator=g, device=device, dtype=dtype)
    q = torch.randn((batch, queries, heads, dim), generator=g, device=device, dtype=torch.float32)
    positions = torch.arange(length - queries, length, device=device)[None].expand(batch, -1).contiguous()
    n_visible = (length - queries) // block - 1
    if queries * topk > n_visible:
        raise ValueError("not enough visible blocks to plant disjoint selections")
    alphas = planted_alphas(topk).to(device)
    qhat = q / q.norm(dim=-1, keepdim=True)
    expected = torch.empty((batch, queries, heads, topk), device=device, dtype=torch.int64)
    for bi in range(batch):
        for h in range(heads):
            perm = torch.randperm(n_visible, generator=g, device=device)[:queries * topk]
            ids = perm.reshape(queries, topk)
            expected[bi, :, h] = ids
            keys = (alphas[None, :, None, None] * math.sqrt(dim) * qhat[bi, :, h][:, None, None, :]
                    + noise * torch.randn((queries, topk, block, dim), generator=g, device=device))
            tokens = (ids[..., None] * block + torch.arange(block, device=device)).reshape(-1)
            k[bi, tokens, h] = keys.reshape(-1, dim).to(dtype)
    q = q.to(dtype)
    if not paged:
        return q, (k, v), positions, expected
    pages = -(-length // page_tokens)
    table = torch.randperm(batch * pages, generator=g, device=device).reshape(batch, pages).to(torch.int32)
    cache = PagedKV.from_dense(k, v, page_tokens, table)
    del k, v
    return q, cache, positions, expected


def plant_blocks(q, k, positions, block, topk, queries, generator, noise=0.05):
    """Plant ``topk`` well-separated key blocks for the query indices
    ``queries`` (every batch row and head) into ``k [B, N, H, D]`` in place.

    Block r of query t holds keys ``alpha_r sqrt(D) q_hat_t + noise N(0,1)``
    (strictly decreasing ``alpha_r``), chosen among the blocks visible to all
    of ``queries`` and distinct across them within a head. Returns the
    expected ids ``[B, len(queries), H, topk]`` in rank order."""
    batch, _, heads, dim = q.shape
    device = k.device
    pos = positions[:, list(queries)]
    n_visible = int(pos.min()) // block - 1
    if len(queries) * topk > n_visible:
        raise ValueError("not enough visible blocks to plant disjoint selections")
    alphas = planted_alphas(topk).to(device)
    qf = q.float()
    qhat = qf / qf.norm(dim=-1, keepdim=True)
    expected = torch.empty((batch, len(queries), heads, topk), device=device, dtype=torch.int64)
    for bi in range(batch):
        for h in range(heads):
            ids = torch.randperm(n_visible, generator=generator, device=device)[:len(queries) * topk]
            ids = ids.reshape(len(queries), topk)
            expected[bi, :, h] = ids
            qh = qhat[bi, list(queries), h]
            keys = (alphas[None, :, None, None] * math.sqrt(dim) * qh[:, None, None, :]
                    + noise * torch.randn((len(queries), topk, block, dim), generator=generator, device=device))
            tokens = (ids[..., None] * block + torch.arange(block, device=device)).reshape(-1)
            k[bi, tokens, h] = keys.reshape(-1, dim).to(k.dtype)
    return expected


def sparse_bytes(positions, ids, heads, dim, block, elem_bytes):
    """Algorithmic HBM bytes of one sparse forward: every visible key block is
    read once per (batch, head) by the scan, then the keys and values of the
    union of selected and local blocks of each (batch, head)."""
    b = block
    total = 0
    pos = positions.cpu()
    sel = ids.cpu()
    for bi in range(pos.shape[0]):
        valid = pos[bi][pos[bi] >= 0]
        if valid.numel() == 0:
            continue
        visible = max(0, int(valid.max()) // b - 1)
        total += heads * visible * b * dim * elem_bytes
        local = set()
        for p in valid.tolist():
            local.update(j for j in (p // b - 1, p // b) if j >= 0)
        for h in range(heads):
            chosen = set(int(x) for x in sel[bi, :, h].reshape(-1).tolist() if x >= 0) | local
            total += len(chosen) * b * dim * elem_bytes * 2
    return total
