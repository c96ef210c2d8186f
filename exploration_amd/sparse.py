"""Paged sparse top-k inference forward on gfx950: the drop-in for ``st.ops``.

``sparse_attention`` keeps the reference signature (``st/ops/sparse.py:100``)
and semantics: exact block scores over every visible block, ``log Z_R`` over
all visible blocks, global top-k selection (descending score, ties broken by
ascending block id, ``-1`` for ``-inf``), then the gated softmax read of the
local window and the selected blocks. All of it runs on the device in one
call of ``st_sparse_fwd`` with no host synchronisation.

KV sources:
* ``TensorPages`` (reference ``st/ops/sparse.py:75-96``): contiguous device
  ``k, v [B, N, H, D]`` holding absolute tokens ``[offset, offset + N)``;
  ``page_tokens`` only shapes the ``pages()`` protocol here, since the kernels
  read the resident cache directly.
* ``PagedKV``: a page pool ``[P, H, page_tokens, D]`` addressed through a page
  table ``[B, pages]`` (logical page -> pool page). New in this package; it
  keeps the ``pages()`` / ``touched_pages()`` protocol of ``TensorPages``.
* ``HostPages``: ``k, v`` in (pinned) host memory, for caches larger than HBM
  (the reference's CPU tier, ``st/runtime/inference.py:19-43`` with the page
  loop of ``st/ops/sparse.py:81-96,121-139``). The score scan streams K
  through two device buffers on a copy stream while the previous chunk is
  scored; after the selection (one host synchronisation for the touched
  block set) the K/V blocks the read needs are copied into a block-paged
  device pool and read through the paged kernels.
"""
import torch

from . import _lib
from .attention import BACKENDS, hip_supported

_records = {}


def _record(kernel, q, block_size, paged):
    key = (kernel, q.device.index, str(q.dtype), q.shape[-1], block_size, paged)
    if key not in _records:
        _records[key] = {"kernel": kernel, "path": "hip", "device": q.device.index, "dtype": str(q.dtype),
                         "head_dim": q.shape[-1], "block_size": block_size,
                         "kv": "paged" if paged else "contiguous"}


def launch_report():
    return list(_records.values())


class TensorPages:
    """In-core KV adapter with the reference's protocol (``st/ops/sparse.py:75-96``)."""

    def __init__(self, k, v, page_tokens=65536, offset=0):
        self.k, self.v, self.page_tokens, self.offset = k, v, page_tokens, offset
        self.length = k.shape[1]

    def pages(self, device, indices=None, keys_only=False):
        if indices is None:
            indices = range((self.length + self.page_tokens - 1) // self.page_tokens)
        for page in indices:
            lo = page * self.page_tokens
            hi = min(lo + self.page_tokens, self.length)
            if hi > lo:
                key = self.k[:, lo:hi].to(device).contiguous()
                value = None if keys_only else self.v[:, lo:hi].to(device).contiguous()
                yield self.offset + lo, key, value

    def touched_pages(self, ids, pos, b):
        blocks = torch.cat((ids.reshape(-1), (pos // b - 1).reshape(-1), (pos // b).reshape(-1)))
        tokens = blocks * b
        local = tokens[(tokens >= self.offset) & (tokens < self.offset + self.length)] - self.offset
        return (local // self.page_tokens).unique().cpu().tolist()


class PagedKV:
    """KV cache in fixed-size pages addressed through a page table.

    ``k_pool, v_pool``: ``[P, H, page_tokens, D]`` (one page of one head is a
    contiguous ``page_tokens x D`` slab); ``page_table``: ``[B, pages]`` int32
    mapping logical page ``t // page_tokens`` of batch row ``b`` to a pool page.
    ``length`` tokens (absolute ``[offset, offset + length)``) are valid.
    """

    def __init__(self, k_pool, v_pool, page_table, length, offset=0):
        if k_pool.shape != v_pool.shape or k_pool.ndim != 4:
            raise ValueError("expected k_pool/v_pool [P, H, page_tokens, D]")
        if page_table.ndim != 2:
            raise ValueError("expected page_table [B, pages]")
        self.k_pool, self.v_pool = k_pool, v_pool
        self.page_table = page_table.to(torch.int32).contiguous()
        self.page_tokens = k_pool.shape[2]
        self.length, self.offset = int(length), int(offset)
        if self.page_table.shape[1] * self.page_tokens < self.length:
            raise ValueError("page table does not cover the cache length")
        # every entry the kernels can dereference must name a pool page
        used = self.page_table[:, :-(-self.length // self.page_tokens)]
        if used.numel() and (int(used.min()) < 0 or int(used.max()) >= k_pool.shape[0]):
            raise ValueError("page table entries must index the page pool")

    @property
    def batch(self):
        return self.page_table.shape[0]

    @classmethod
    def empty(cls, batch, length, heads, dim, dtype, device, page_tokens=128, offset=0):
        """A zero-filled cache for ``length`` tokens: ``batch * ceil(length /
        page_tokens)`` pool pages, batch row ``b``'s logical pages at pool
        pages ``b * pages ...`` in order. Fill it with ``write``."""
        pages = -(-int(length) // page_tokens)
        table = torch.arange(batch * pages, dtype=torch.int32, device=device).reshape(batch, pages)
        k_pool = torch.zeros(batch * pages, heads, page_tokens, dim, dtype=dtype, device=device)
        return cls(k_pool, torch.zeros_like(k_pool), table, length, offset)

    def write(self, start, k, v):
        """Store ``k, v [B, T, H, D]`` (device, the pool's dtype) at absolute
        tokens ``[start, start + T)`` through the page table, in one kernel
        on the current stream (``st_paged_kv_write``; the reference's
        ``KVCache.write``, ``st/runtime/inference.py:45-52``)."""
        lo = start - self.offset
        if lo < 0 or lo + k.shape[1] > self.length:
            raise ValueError("KV write outside owned shard")
        pool = self.k_pool
        if k.shape != v.shape or k.ndim != 4 or k.shape[0] != self.batch or k.shape[2] != pool.shape[1] \
                or k.shape[3] != pool.shape[3]:
            raise ValueError("expected k, v [B, T, H, D] matching the cache")
        if k.dtype != pool.dtype or v.dtype != pool.dtype or k.device != pool.device or v.device != pool.device:
            raise ValueError("k, v must have the cache's dtype and device")
        lib = _lib.load()
        k, v = k.contiguous(), v.contiguous()
        _lib.check(lib.st_paged_kv_write(_lib.DTYPE_CODES[pool.dtype], k.shape[0], k.shape[1], k.shape[2],
                                         k.shape[3], _lib.ptr(k), _lib.ptr(v), _lib.ptr(self.page_table),
                                         self.page_tokens, self.page_table.shape[1], lo, _lib.ptr(pool),
                                         _lib.ptr(self.v_pool), pool.shape[0], _lib.stream_of(k)), lib)

    @classmethod
    def from_dense(cls, k, v, page_tokens, page_table=None, offset=0):
        """Build a paged cache from contiguous ``k, v [B, N, H, D]``. With
        ``page_table=None`` pages are laid out in order."""
        batch, n, heads, dim = k.shape
        pages = -(-n // page_tokens)
        if page_table is None:
            page_table = torch.arange(batch * pages, device=k.device, dtype=torch.int32).reshape(batch, pages)
        page_table = page_table.to(device=k.device, dtype=torch.int64)
        total = int(page_table.max()) + 1
        k_pool = k.new_zeros(total, heads, page_tokens, dim)
        v_pool = v.new_zeros(total, heads, page_tokens, dim)
        pad = pages * page_tokens - n
        for src, pool in ((k, k_pool), (v, v_pool)):
            full = torch.nn.functional.pad(src, (0, 0, 0, 0, 0, pad)) if pad else src
            pool[page_table.reshape(-1)] = (full.reshape(batch, pages, page_tokens, heads, dim)
                                            .permute(0, 1, 3, 2, 4).reshape(batch * pages, heads, page_tokens, dim))
        return cls(k_pool, v_pool, page_table, n, offset)

    def gather(self, lo=0, hi=None):
        """Contiguous ``(k, v) [B, hi-lo, H, D]`` of range-relative tokens [lo, hi)."""
        hi = self.length if hi is None else hi
        first, last = lo // self.page_tokens, -(-hi // self.page_tokens)
        idx = self.page_table[:, first:last].to(torch.int64)
        out = []
        for pool in (self.k_pool, self.v_pool):
            g = pool[idx.reshape(-1)]  # [B*pages, H, T, D]
            g = g.reshape(idx.shape[0], -1, *pool.shape[1:]).permute(0, 1, 3, 2, 4)
            g = g.reshape(idx.shape[0], -1, pool.shape[1], pool.shape[3])
            start = lo - first * self.page_tokens
            out.append(g[:, start:start + (hi - lo)].contiguous())
        return out[0], out[1]

    def pages(self, device, indices=None, keys_only=False):
        if indices is None:
            indices = range(-(-self.length // self.page_tokens))
        for page in indices:
            lo = page * self.page_tokens
            hi = min(lo + self.page_tokens, self.length)
            if hi > lo:
                k, v = self.gather(lo, hi)
                yield self.offset + lo, k.to(device), None if keys_only else v.to(device)

    def touched_pages(self, ids, pos, b):
        blocks = torch.cat((ids.reshape(-1), (pos // b - 1).reshape(-1), (pos // b).reshape(-1)))
        tokens = blocks * b
        local = tokens[(tokens >= self.offset) & (tokens < self.offset + self.length)] - self.offset
        return (local // self.page_tokens).unique().cpu().tolist()


class HostPages:
    """Host-resident raw K/V ``[B, N, H, D]`` (absolute tokens
    ``[offset, offset + N)``) streamed to ``device`` in chunks of
    ``chunk_tokens`` tokens. Pinned tensors are copied to the device
    directly; pageable ones (a file mapping) are first copied into pinned
    staging buffers, so the device copies stay asynchronous."""

    def __init__(self, k, v, device, chunk_tokens=65536, offset=0):
        if k.shape != v.shape or k.ndim != 4 or k.device.type != "cpu":
            raise ValueError("expected host k, v [B, N, H, D]")
        self.k, self.v, self.device = k, v, torch.device(device)
        self.chunk_tokens = self.page_tokens = int(chunk_tokens)
        self.offset, self.length = int(offset), k.shape[1]


def _sparse_host(q, cache, positions, b, topk, return_selection):
    """Scan (streamed K), selection, then the paged read of the touched blocks."""
    lib = _lib.load()
    if cache.k.dtype != q.dtype or cache.k.shape[0] != q.shape[0] or cache.k.shape[2:] != q.shape[2:]:
        raise ValueError("q and the host KV cache differ in dtype or batch/head dimensions")
    batch, queries, heads, dim = q.shape
    n, off = cache.length, cache.offset
    chunk = max(b, cache.chunk_tokens // b * b)
    n_blocks = -(-n // b)
    scores = torch.empty((batch, queries, heads, n_blocks), device=q.device, dtype=torch.float32)
    main = torch.cuda.current_stream(q.device)
    copier = torch.cuda.Stream(q.device)
    copier.wait_stream(main)  # device->host writes of the cache issued on the main stream come first
    size = batch * min(chunk, n) * heads * dim
    bufs = [torch.empty(size, device=q.device, dtype=q.dtype) for _ in range(2)]
    # pageable source: the CPU fills pinned buffer i%2 with chunk i while the
    # device still copies and scores chunk i-1
    stage = None if cache.k.is_pinned() else [torch.empty(size, dtype=q.dtype, pin_memory=True) for _ in range(2)]
    ready = [torch.cuda.Event() for _ in range(2)]
    free = [torch.cuda.Event() for _ in range(2)]
    for i, lo in enumerate(range(0, n, chunk)):
        hi, slot = min(n, lo + chunk), i % 2
        part = bufs[slot][:batch * (hi - lo) * heads * dim].view(batch, hi - lo, heads, dim)
        src = cache.k[:, lo:hi]
        if stage is not None:
            if i >= 2:
                ready[slot].synchronize()  # the device copy out of this buffer (chunk i-2) is done
            src = stage[slot][:part.numel()].view(part.shape).copy_(src)
        with torch.cuda.stream(copier):
            if i >= 2:
                copier.wait_event(free[slot])
            part.copy_(src, non_blocking=True)
            ready[slot].record(copier)
        main.wait_event(ready[slot])
        g0, g1 = lo // b, -(-hi // b)
        scores[..., g0:g1] = block_scores(q, part, positions, b, offset=off + lo)
        free[slot].record(main)
    values, ids, log_zr = select_blocks(scores, topk, id_base=off // b)
    # blocks the read touches per batch row: the selection and the two local
    # blocks of every query (host synchronisation)
    pos = positions.to(q.device, torch.int64)
    local = torch.stack((pos // b - 1, pos // b), -1)[:, :, None, :].expand(batch, queries, heads, 2)
    wanted = torch.cat((ids, local), -1).reshape(batch, -1) - off // b
    wanted = wanted.cpu()
    table = torch.zeros((batch, n_blocks), dtype=torch.int32)
    rows, blocks, placed = [], [], 0
    for r in range(batch):
        w = wanted[r]
        uniq = w[(w >= 0) & (w < n_blocks)].unique()
        table[r, uniq] = torch.arange(placed, placed + len(uniq), dtype=torch.int32)
        placed += len(uniq)
        rows.append(torch.full_like(uniq, r))
        blocks.append(uniq)
    rows, blocks = torch.cat(rows), torch.cat(blocks)
    tok = (blocks[:, None] * b + torch.arange(b)).clamp(max=n - 1)       # [T, b]
    pools = []
    for src in (cache.k, cache.v):
        staged = src[rows[:, None], tok].permute(0, 2, 1, 3).contiguous()  # [T, H, b, D]
        pools.append(staged.pin_memory().to(q.device, non_blocking=True))
    table = table.to(q.device, non_blocking=True)
    ws_bytes = lib.st_sparse_workspace_bytes(batch, queries, heads, dim, topk, 0)
    ws = torch.empty(max(ws_bytes, 256), device=q.device, dtype=torch.uint8)
    out = torch.empty_like(q)
    _lib.check(lib.st_sparse_pop(_lib.DTYPE_CODES[q.dtype], batch, queries, heads, dim, b, _lib.ptr(q),
                                 _lib.ptr(pos), _lib.ptr(pools[0]), _lib.ptr(pools[1]), _lib.ptr(table), b,
                                 n_blocks, n, off, _lib.ptr(ids), _lib.ptr(values), _lib.ptr(log_zr), topk,
                                 _lib.DTYPE_CODES[q.dtype], _lib.ptr(out), None, _lib.ptr(ws), ws.numel(),
                                 _lib.stream_of(q)), lib)
    _record("sparse_pop", q, b, True)
    if return_selection:
        return out, {"indices": ids, "scores": values, "log_zr": log_zr}
    return out


def sparse_workspace_bytes(batch, queries, heads, head_dim, topk, n_blocks):
    """Device workspace of one ``st_sparse_fwd`` call, as the library computes
    it (``st_sparse_workspace_bytes``): the float32 block scores of every
    row, then the read's float32 partials (``ceil((topk + 2) / 4)`` chunks of
    ``Dp + 2`` floats per row, ``Dp`` = 64, 128 or 256), each rounded up to
    256 bytes. Host arithmetic only, so planners can use it without a GPU."""
    rows = batch * queries * heads
    dp = 64 if head_dim <= 64 else (128 if head_dim <= 128 else 256)
    chunks = (topk + 2 + 3) // 4
    up = lambda x: (x + 255) // 256 * 256
    return up(4 * rows * n_blocks) + up(4 * rows * chunks * (dp + 2))


def _host_resident(cache):
    k, v = getattr(cache, "k", None), getattr(cache, "v", None)
    return (isinstance(k, torch.Tensor) and isinstance(v, torch.Tensor) and k.device.type == "cpu"
            and v.device.type == "cpu")


def _kv_view(cache, q, block_size):
    """(k, v, page_table, page_tokens, pages_per_seq, n_tokens, offset) of a
    device-resident cache, or ValueError."""
    if isinstance(cache, PagedKV):
        if cache.k_pool.device != q.device or cache.page_table.device != q.device:
            raise ValueError("paged KV cache must live on the query's device")
        if cache.k_pool.dtype != q.dtype:
            raise ValueError("q and the KV cache must use the same dtype")
        if cache.batch != q.shape[0] or cache.k_pool.shape[1] != q.shape[2] or cache.k_pool.shape[3] != q.shape[3]:
            raise ValueError("query and KV batch/head dimensions differ")
        return (cache.k_pool.contiguous(), cache.v_pool.contiguous(), cache.page_table, cache.page_tokens,
                cache.page_table.shape[1], cache.length, cache.offset)
    k, v = getattr(cache, "k", None), getattr(cache, "v", None)
    if not (isinstance(k, torch.Tensor) and isinstance(v, torch.Tensor) and k.device == q.device
            and v.device == q.device):
        raise ValueError("the HIP sparse kernels read a device-resident cache (TensorPages or PagedKV "
                         "on the query's device)")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q and the KV cache must use the same dtype")
    if k.ndim != 4 or k.shape != v.shape or k.shape[0] != q.shape[0] or k.shape[2:] != q.shape[2:]:
        raise ValueError("query and KV batch/head dimensions differ")
    return (k.contiguous(), v.contiguous(), None, cache.page_tokens, 0, k.shape[1], cache.offset)


@torch.inference_mode()
def sparse_attention(q, cache, positions, block_size, topk, backend="auto", group=None,
                     score_page_tokens=65536, return_selection=False):
    """Exact score/top-k + gate + sparse read (``st/ops/sparse.py:99-174``).

    ``score_page_tokens`` tiles the reference's host loop and is validated
    only. ``group`` must be ``None`` or a single-rank group: sequence-sharded
    inference across GPUs is not implemented here.
    """
    b = block_size
    if backend not in BACKENDS:
        raise ValueError(f"unknown attention backend {backend!r}")
    if isinstance(getattr(cache, "paged", None), PagedKV):
        cache = cache.paged  # an inference session's HBM-tier cache
    if topk < 1 or score_page_tokens < b or cache.page_tokens % b or cache.offset % b:
        raise ValueError("topk positive; cache pages/offset must be block aligned")
    if backend == "torch":
        raise ValueError("backend 'torch' is the reference's portable restatement; "
                         "this package only provides the fused HIP kernels")
    if group is not None and torch.distributed.is_initialized() and torch.distributed.get_world_size(group) > 1:
        raise NotImplementedError("sharded sparse inference across GPUs is not implemented")
    if not hip_supported(q, b):
        raise ValueError("unsupported HIP sparse configuration")
    if q.ndim != 4 or positions.shape != q.shape[:2]:
        raise ValueError("expected q[B,Q,H,D], positions[B,Q]")
    if not isinstance(cache, (HostPages, PagedKV)) and _host_resident(cache):
        # a TensorPages / KVCache over host memory (the reference's CPU and
        # disk tiers, st/runtime/inference.py:19-43): streamed like HostPages
        cache = HostPages(cache.k, cache.v, q.device, chunk_tokens=max(b, score_page_tokens // b * b),
                          offset=cache.offset)
    if isinstance(cache, HostPages):
        return _sparse_host(q.contiguous(), cache, positions.to(device=q.device, dtype=torch.int64).contiguous(),
                            b, topk, return_selection)
    lib = _lib.load()
    k, v, table, page_tokens, pages_per_seq, n_tokens, offset = _kv_view(cache, q, b)
    q = q.contiguous()
    positions = positions.to(device=q.device, dtype=torch.int64).contiguous()
    batch, queries, heads, dim = q.shape
    n_blocks = -(-n_tokens // b)
    ws_bytes = lib.st_sparse_workspace_bytes(batch, queries, heads, dim, topk, n_blocks)
    ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8)
    out = torch.empty_like(q)
    ids = torch.empty((*q.shape[:3], topk), device=q.device, dtype=torch.int64)
    scores = torch.empty((*q.shape[:3], topk), device=q.device, dtype=torch.float32)
    log_zr = torch.empty(q.shape[:3], device=q.device, dtype=torch.float32)
    _lib.check(lib.st_sparse_fwd(_lib.DTYPE_CODES[q.dtype], batch, queries, heads, dim, b, topk,
                                 _lib.ptr(q), _lib.ptr(positions), _lib.ptr(k), _lib.ptr(v), _lib.ptr(table),
                                 page_tokens, pages_per_seq, n_tokens, offset,
                                 _lib.ptr(out), _lib.ptr(ids), _lib.ptr(scores), _lib.ptr(log_zr), None,
                                 _lib.ptr(ws), ws_bytes, _lib.stream_of(q)), lib)
    _record("sparse_fwd", q, b, table is not None)
    if return_selection:
        return out, {"indices": ids, "scores": scores, "log_zr": log_zr}
    return out


@torch.inference_mode()
def block_scores(q, k, positions, block_size, offset=0, *, force_streamed=False):
    """Exact block scores ``[B,Q,H,G]`` (float32) of a contiguous KV slab that
    starts at absolute token ``offset`` (reference internal
    ``st/ops/kernels/sparse.py:81-100``). ``force_streamed`` picks the
    reference's small-tile NVIDIA fallback there; one kernel family serves
    both settings here."""
    lib = _lib.load()
    if not hip_supported(q, block_size) or k.dtype != q.dtype:
        raise ValueError("unsupported HIP block-score configuration")
    q, k = q.contiguous(), k.contiguous()
    positions = positions.to(device=q.device, dtype=torch.int64).contiguous()
    batch, queries, heads, dim = q.shape
    n_blocks = -(-k.shape[1] // block_size)
    scores = torch.empty((batch, queries, heads, n_blocks), device=q.device, dtype=torch.float32)
    _lib.check(lib.st_sparse_scores(_lib.DTYPE_CODES[q.dtype], batch, queries, heads, dim, block_size,
                                    _lib.ptr(q), _lib.ptr(positions), _lib.ptr(k), None, block_size, 0,
                                    k.shape[1], offset, _lib.ptr(scores), n_blocks, _lib.stream_of(q)), lib)
    _record("sparse_scores", q, block_size, False)
    return scores


@torch.inference_mode()
def select_blocks(scores, topk, id_base=0):
    """Top-k of ``scores [..., G]``: ``(values, ids, log_zr)`` with values in
    descending order (ties by ascending id), ``ids = -1`` for ``-inf``
    (reference ``st/ops/sparse.py:121-139,154``)."""
    lib = _lib.load()
    scores = scores.contiguous().float()
    rows = scores.numel() // scores.shape[-1]
    values = torch.empty((*scores.shape[:-1], topk), device=scores.device, dtype=torch.float32)
    ids = torch.empty((*scores.shape[:-1], topk), device=scores.device, dtype=torch.int64)
    log_zr = torch.empty(scores.shape[:-1], device=scores.device, dtype=torch.float32)
    _lib.check(lib.st_sparse_select(rows, scores.shape[-1], topk, id_base, _lib.ptr(scores), _lib.ptr(ids),
                                    _lib.ptr(values), _lib.ptr(log_zr), _lib.stream_of(scores)), lib)
    return values, ids, log_zr


@torch.inference_mode()
def sparse_pop(q, k, v, positions, ids, scores, log_zr, block_size, offset=0):
    """Gated softmax read of the local window and the selected blocks from a
    contiguous KV slab starting at absolute token ``offset``; returns
    ``(out float32, lse float32)`` as the reference does
    (``st/ops/kernels/sparse.py:103-113``; its caller merges page partials by
    LSE and casts to ``q.dtype``, ``st/ops/sparse.py:157-174``)."""
    lib = _lib.load()
    if not hip_supported(q, block_size):
        raise ValueError("unsupported HIP sparse configuration")
    q, k, v = q.contiguous(), k.contiguous(), v.contiguous()
    positions = positions.to(device=q.device, dtype=torch.int64).contiguous()
    ids, scores, log_zr = ids.contiguous(), scores.float().contiguous(), log_zr.float().contiguous()
    batch, queries, heads, dim = q.shape
    topk = ids.shape[-1]
    ws_bytes = lib.st_sparse_workspace_bytes(batch, queries, heads, dim, topk, 0)
    ws = torch.empty(max(ws_bytes, 256), device=q.device, dtype=torch.uint8)
    out = torch.empty(q.shape, device=q.device, dtype=torch.float32)
    lse = torch.empty(q.shape[:3], device=q.device, dtype=torch.float32)
    _lib.check(lib.st_sparse_pop(_lib.DTYPE_CODES[q.dtype], batch, queries, heads, dim, block_size,
                                 _lib.ptr(q), _lib.ptr(positions), _lib.ptr(k), _lib.ptr(v), None,
                                 block_size, 0, k.shape[1], offset, _lib.ptr(ids), _lib.ptr(scores),
                                 _lib.ptr(log_zr), topk, _lib.DTYPE_CODES[torch.float32], _lib.ptr(out),
                                 _lib.ptr(lse), _lib.ptr(ws), ws.numel(), _lib.stream_of(q)), lib)
    _record("sparse_pop", q, block_size, False)
    return out, lse
