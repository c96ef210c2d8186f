"""Streaming prefill and paged sparse inference for the Stack model, one GPU.

Restates the reference's ``InferenceSession`` / ``KVCache`` / ``plan_inference``
(``st/runtime/inference.py:19-224``, ``st/runtime/memory.py:28-97``) over this
package's ``sparse_attention``: the prompt is encoded in chunks (hidden states
and raw K/V for one chunk at a time, the local blocks carrying their one-block
halo state across chunks), raw K/V are written once into a cache, hidden
states are kept only at the requested positions, and ``iter_logits`` runs the
global read rounds through the sparse top-k operator with no host
synchronisation.

Cache tiers: ``"cuda"`` keeps K/V in HBM (the cfg5 decode: 131,072 tokens x
16 heads x 64 dims is 512 MiB). ``"cpu"`` keeps them in pinned host memory
and ``"disk"`` in a file-backed mapping under ``cache_dir`` (contexts larger
than host memory); for both the operator streams K through device buffers
and gathers the touched blocks into a device pool (``sparse.HostPages``).
Multi-rank sharding is not built (one GPU).
"""
import os
import shutil
import tempfile
from dataclasses import asdict, dataclass

import torch

from .sparse import HostPages, TensorPages, sparse_attention

GiB = 1 << 30


def available_host_memory():
    """MemAvailable of /proc/meminfo in bytes (None if unreadable)."""
    try:
        with open("/proc/meminfo") as f:
            for line in f:
                if line.startswith("MemAvailable:"):
                    return int(line.split()[1]) * 1024
    except OSError:
        pass
    return None


@dataclass
class InferencePlan:
    """``st/runtime/memory.py:28-40``."""
    cache: str
    cache_bytes: int
    gpu_budget_bytes: int
    page_tokens: int
    encoder_chunk: int
    query_chunk: int
    score_tokens: int
    head_chunk: int
    host_available_bytes: int

    def to_dict(self):
        return asdict(self)


def plan_inference(model, batch, length, *, cache="auto", memory_fraction=.8, page_tokens=65536,
                   encoder_chunk=4096, query_chunk=16, workspace_mb=256, cache_dir=None):
    """Cache tier and chunk sizes (``st/runtime/memory.py:43-97``): K/V bytes
    ``2 B N dim e``; the GPU tier when they fit the budget (a fraction of
    capacity, 2 GiB kept free), else host memory; page, encoder, query, score
    and head chunks bounded by the workspace."""
    if not 0 < memory_fraction < 1 or min(batch, length, page_tokens, encoder_chunk, query_chunk, workspace_mb) < 1:
        raise ValueError("positive sizes and 0 < memory_fraction < 1 required")
    if cache not in ("auto", "cuda", "cpu", "disk"):
        raise ValueError("cache must be auto/cuda/cpu/disk")
    param = next(model.parameters())
    b, dim, heads = model.block_size, model.dim, model.heads
    element = param.element_size()
    total = 2 * batch * length * dim * element
    budget = 0
    if param.is_cuda:
        free, capacity = torch.cuda.mem_get_info(param.device)
        budget = max(0, min(int(capacity * memory_fraction), free - 2 * GiB))
    workspace = workspace_mb << 20
    host = available_host_memory()
    if cache == "auto":
        if param.is_cuda and total + 4 * workspace < budget:
            cache = "cuda"
        elif host is None or total + 4 * workspace < host * .7:
            cache = "cpu"
        elif cache_dir:
            cache = "disk"
        else:
            raise MemoryError(f"KV requires {total / GiB:.2f} GiB; neither HBM nor host memory holds it "
                              "(give cache_dir for the disk tier)")
    if cache == "cuda" and (not param.is_cuda or total + 4 * workspace >= budget):
        raise MemoryError(f"GPU KV requires {total / GiB:.2f} GiB plus workspace; select cache=auto/cpu/disk")
    if cache == "cpu" and host is not None and total + 4 * workspace > host * .7:
        raise MemoryError(f"CPU KV requires {total / GiB:.2f} GiB; available RAM {host / GiB:.2f} GiB; "
                          "select the disk tier")
    if cache == "disk":
        if not cache_dir:
            raise ValueError("the disk KV tier needs cache_dir on a filesystem with room for the cache")
        os.makedirs(cache_dir, exist_ok=True)
        if total + GiB > shutil.disk_usage(cache_dir).free:
            raise MemoryError(f"disk KV requires {total / GiB:.2f} GiB; not free under {cache_dir}")
    page = max(b, min(page_tokens, workspace // max(2 * batch * dim * element, 1)) // b * b)
    enc = max(b, min(encoder_chunk, workspace // max(24 * batch * dim * element, 1)) // b * b)
    qc = max(1, min(query_chunk, workspace // max(batch * heads * model.topk * b * 4, 1)))
    score = max(b, min(page, workspace // max(4 * batch * heads * qc * 4, 1)) // b * b)
    head = max(1, min(qc, workspace // max(batch * model.lm_head.out_features * 4, 1)))
    return InferencePlan(cache, total, budget, page, enc, qc, score, head, host)


class KVCache(TensorPages):
    """Write-once raw K/V ``[B,N,H,hd]`` in HBM (``"cuda"``), pinned host
    memory (``"cpu"``) or a file-backed mapping (``"disk"``), read through the
    page protocol (``st/runtime/inference.py:19-62``). The disk tier's file
    lives in a private temporary directory under ``cache_dir`` with its
    blocks allocated up front (a full filesystem fails here, not half-way
    through a prefill); ``close`` removes it."""

    def __init__(self, batch, length, heads, dim, dtype, device, plan, offset=0, cache_dir=None):
        shape = (batch, length, heads, dim)
        self.directory = None
        if plan.cache == "cuda":
            k, v = (torch.empty(shape, dtype=dtype, device=device) for _ in range(2))
        elif plan.cache == "cpu":
            k, v = (torch.empty(shape, dtype=dtype, pin_memory=True) for _ in range(2))
        elif plan.cache == "disk":
            k, v = self._map_file(shape, dtype, cache_dir)
        else:
            raise ValueError(f"unknown cache tier {plan.cache!r}")
        super().__init__(k, v, plan.page_tokens, offset)
        self.tier = plan.cache
        self.device = torch.device(device)

    def _map_file(self, shape, dtype, cache_dir):
        """K and V as the two halves of one shared file mapping."""
        self.directory = tempfile.mkdtemp(prefix="st-kv-", dir=cache_dir)
        count = shape[0] * shape[1] * shape[2] * shape[3]
        nbytes = 2 * count * torch.empty((), dtype=dtype).element_size()
        path = os.path.join(self.directory, "kv.bin")
        try:
            with open(path, "xb") as f:
                if hasattr(os, "posix_fallocate"):
                    os.posix_fallocate(f.fileno(), 0, nbytes)
                else:
                    f.truncate(nbytes)
            flat = torch.from_file(path, shared=True, size=2 * count, dtype=dtype)
        except BaseException:
            shutil.rmtree(self.directory, ignore_errors=True)
            self.directory = None
            raise
        return flat[:count].view(shape), flat[count:].view(shape)

    def write(self, start, k, v):
        lo = start - self.offset
        if lo < 0 or lo + k.shape[1] > self.length:
            raise ValueError("KV write outside owned shard")
        # pageable file memory: a synchronous copy; HBM and pinned: stream-ordered
        asynchronous = self.tier != "disk"
        self.k[:, lo:lo + k.shape[1]].copy_(k, non_blocking=asynchronous)
        self.v[:, lo:lo + v.shape[1]].copy_(v, non_blocking=asynchronous)

    def reader(self, score_tokens):
        """What the sparse operator reads: the cache itself in HBM, or a
        streaming view of the host or disk tier."""
        if self.tier == "cuda":
            return self
        return HostPages(self.k, self.v, self.device, chunk_tokens=score_tokens, offset=self.offset)

    def close(self):
        self.k, self.v = None, None
        if self.directory is not None:
            shutil.rmtree(self.directory, ignore_errors=True)
            self.directory = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class InferenceSession:
    """A write-once raw-KV cache and bounded query states for one prompt:
    ``prefill(ids_cpu, positions_cpu)`` then ``iter_logits()``
    (``st/runtime/inference.py:65-224``). One GPU; ``group`` must be None."""

    def __init__(self, model, *, group=None, cache="auto", cache_dir=None, memory_fraction=.8,
                 page_tokens=65536, encoder_chunk=4096, query_chunk=16, workspace_mb=256,
                 max_query_states_mb=256):
        if model.training:
            raise ValueError("call model.eval() before creating an inference session")
        if group is not None and torch.distributed.is_initialized() and torch.distributed.get_world_size(group) > 1:
            raise NotImplementedError("sharded inference across GPUs is not built")
        self.model = model
        param = next(model.parameters())
        self.device, self.dtype = param.device, param.dtype
        self.options = dict(cache=cache, cache_dir=cache_dir, memory_fraction=memory_fraction,
                            page_tokens=page_tokens, encoder_chunk=encoder_chunk, query_chunk=query_chunk,
                            workspace_mb=workspace_mb)
        self.max_query_bytes = max_query_states_mb << 20
        self.cache = None
        self.ready = False

    @torch.inference_mode()
    def prefill(self, input_ids, positions):
        if self.cache is not None or self.ready:
            raise RuntimeError("use a new session for each prompt")
        if input_ids.ndim != 2 or min(input_ids.shape) < 1 or input_ids.device.type != "cpu":
            raise ValueError("input_ids must be nonempty CPU [B,N]; pages are transferred automatically")
        batch, n = input_ids.shape
        positions = positions.to("cpu", dtype=torch.long)
        if positions.ndim != 2 or positions.shape[0] != batch or positions.shape[1] < 1:
            raise ValueError("positions must be nonempty [B,Q]")
        if (positions < 0).any() or (positions >= n).any():
            raise ValueError("query positions must lie within the prompt")
        m = self.model
        if positions.numel() * m.dim * self.dtype.itemsize > self.max_query_bytes:
            raise MemoryError("query states exceed max_query_states_mb; evaluate fewer positions")
        self.plan = plan_inference(m, batch, n, **self.options)
        self.cache = KVCache(batch, n, m.heads, m.hd, self.dtype, self.device, self.plan,
                             cache_dir=self.options["cache_dir"])
        self.positions = positions
        self.query_states = torch.zeros(batch, positions.shape[1], m.dim, dtype=self.dtype, device=self.device)
        dev_pos = positions.to(self.device)
        b = m.block_size
        halos = [None] * len(m.local)
        try:
            for lo in range(0, n, self.plan.encoder_chunk):
                hi = min(n, lo + self.plan.encoder_chunk)
                x = m.embed(input_ids[:, lo:hi].to(self.device, non_blocking=True))
                for i, layer in enumerate(m.local):
                    prev = halos[i]
                    halos[i] = x[:, -b:].clone()
                    x = layer(x, previous=prev, start=lo)
                k, v = m.raw_kv(x, None)
                self.cache.write(lo, k, v)
                # hidden states of the requested positions inside this chunk
                inside = (dev_pos >= lo) & (dev_pos < hi)
                rows, cols = inside.nonzero(as_tuple=True)
                self.query_states[rows, cols] = x[rows, dev_pos[rows, cols] - lo]
                del x, k, v
            self.ready = True
        except BaseException:
            self.close()
            raise
        return self

    @torch.inference_mode()
    def iter_logits(self, return_selection=False):
        if not self.ready:
            raise RuntimeError("prefill must complete before inference")
        m = self.model
        cache = self.cache.reader(self.plan.score_tokens)
        for lo in range(0, self.positions.shape[1], self.plan.query_chunk):
            hi = min(lo + self.plan.query_chunk, self.positions.shape[1])
            z = self.query_states[:, lo:hi]
            pos = self.positions[:, lo:hi].to(self.device, non_blocking=True)
            selection = None
            for rd in m.reads:
                q = rd.wq(rd.q_norm(z)).reshape(*z.shape[:2], m.heads, m.hd)
                result = sparse_attention(q, cache, pos, m.block_size, m.topk, backend=m.backend,
                                          score_page_tokens=self.plan.score_tokens,
                                          return_selection=return_selection)
                ctx, selection = result if return_selection else (result, None)
                z = z + rd.read_out(ctx.reshape(*z.shape[:2], m.dim))
                z = z + rd.ffn(rd.ffn_norm(z))
            for j in range(0, hi - lo, self.plan.head_chunk):
                stop = min(j + self.plan.head_chunk, hi - lo)
                yield slice(lo + j, lo + stop), m.lm_head(m.final_norm(z[:, j:stop])), selection

    def close(self):
        if self.cache is not None:
            self.cache.close()
            self.cache = None
        self.query_states = None
        self.ready = False

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
