"""Streaming prefill and paged sparse inference for the Stack model, one GPU.

Restates the reference's ``InferenceSession`` / ``KVCache`` / ``plan_inference``
(``st/runtime/inference.py:19-224``, ``st/runtime/memory.py:28-97``) over this
package's ``sparse_attention``: the prompt is encoded in chunks (hidden states
and raw K/V for one chunk at a time, the local blocks carrying their one-block
halo state across chunks), raw K/V are written once into a cache, hidden
states are kept only at the requested positions, and ``iter_logits`` runs the
global read rounds through the sparse top-k operator with no host
synchronisation.

Cache tiers: ``"cuda"`` keeps K/V in HBM as a ``PagedKV`` of 128-token pages
(the cfg5 decode: 131,072 tokens x 16 heads x 64 dims is 512 MiB), written by
one paged-write kernel per encoder chunk and read by the sparse kernels
through the page table. ``"cpu"`` keeps them in pinned host memory and
``"disk"`` in a file-backed mapping under ``cache_dir`` (contexts larger than
host memory); for both the operator streams K through device buffers and
gathers the touched blocks into a device pool (``sparse.HostPages``).
Multi-rank sharding is not built (one GPU).
"""
import math
import os
import shutil
import tempfile
from dataclasses import asdict, dataclass

import torch

from .sparse import HostPages, PagedKV, TensorPages, sparse_attention, sparse_workspace_bytes

GiB = 1 << 30
HBM_PAGE_TOKENS = 128   # tokens per pool page of the HBM tier
GPU_RESERVE = 2 * GiB   # left free on the GPU for library workspaces and fragmentation


def _read_int(path):
    try:
        with open(path) as f:
            text = f.read().split()
    except OSError:
        return None
    return int(text[0]) if text and text[0].isdigit() else None


def _meminfo_available():
    try:
        with open("/proc/meminfo") as f:
            for line in f:
                if line.startswith("MemAvailable:"):
                    return int(line.split()[1]) * 1024
    except OSError:
        pass
    return None


def _cgroup_room():
    """What a memory-limited control group still allows this process
    (cgroup v2 ``memory.max - memory.current``, or v1
    ``limit_in_bytes - usage_in_bytes``); None when there is no limit."""
    for limit, usage in (("/sys/fs/cgroup/memory.max", "/sys/fs/cgroup/memory.current"),
                         ("/sys/fs/cgroup/memory/memory.limit_in_bytes",
                          "/sys/fs/cgroup/memory/memory.usage_in_bytes")):
        cap, used = _read_int(limit), _read_int(usage)
        if cap is not None and used is not None and cap < 1 << 60:
            return max(0, cap - used)
    return None


def available_host_memory():
    """Host bytes this process can still take: the kernel's MemAvailable,
    lowered to the control group's remaining allowance when the process runs
    under a memory limit (a container); None if neither can be read."""
    known = [x for x in (_meminfo_available(), _cgroup_room()) if x is not None]
    return min(known) if known else None


@dataclass
class InferencePlan:
    """Where a session keeps its K/V and how it cuts the work. The first nine
    fields are the reference's (``st/runtime/memory.py:28-40``);
    ``page_tokens`` is the HBM tier's pool page (128 tokens) or, on the host
    tiers, the chunk streamed to the device for the score scan."""
    cache: str
    cache_bytes: int            # K and V of the prompt
    gpu_budget_bytes: int
    page_tokens: int
    encoder_chunk: int          # prompt tokens encoded per prefill step
    query_chunk: int            # query positions per sparse read
    score_tokens: int           # host tiers: tokens per streamed score chunk
    head_chunk: int             # positions per LM-head call
    host_available_bytes: int
    pool_pages: int = 0         # HBM tier: pages of each of the K and V pools
    read_bytes: int = 0         # device bytes of one sparse read (workspace + outputs)
    device_bytes: int = 0       # device bytes the plan counts on in total

    def to_dict(self):
        return asdict(self)


def _ffn_width(model):
    widths = [layer.ffn[0].out_features for layer in list(model.local) + list(model.reads)]
    return max(widths) if widths else 4 * model.dim


def _largest(limit, unit, budget, per_item):
    """Largest multiple of ``unit`` that is at most ``limit`` and whose
    ``per_item`` cost fits ``budget`` (at least one ``unit``)."""
    fit = budget // max(per_item, 1)
    return max(unit, min(limit, fit) // unit * unit)


def plan_inference(model, batch, length, *, cache="auto", memory_fraction=.8, page_tokens=65536,
                   encoder_chunk=4096, query_chunk=16, workspace_mb=256, cache_dir=None):
    """Tier and chunk sizes of an inference session, from what the HIP path
    allocates (the reference's planner is ``st/runtime/memory.py:43-97``).

    Device memory per tier:

    * ``"cuda"``: the page pools (``2 B ceil(N/128) 128 H hd e`` bytes, the
      last page padded), one encoder chunk's activations and one sparse read;
    * ``"cpu"`` / ``"disk"``: one encoder chunk, one sparse read, two streamed
      score chunks of K and the device pool of the blocks a read touches
      (at most ``rows (topk + 2)`` blocks of all heads, or the whole cache).

    Each chunk size is the largest (a multiple of its unit, at most the
    requested size) whose device bytes fit ``workspace_mb``: the encoder chunk
    (unit ``lcm(b, 128)``; about ``9 dim + 2 ffn`` live elements per token),
    the query chunk (``sparse_workspace_bytes`` plus ids, scores, log Z_R and
    output per row), the score chunk (two K buffers) and the head chunk
    (float32 logits). ``"auto"`` takes the first tier that fits: HBM within
    ``min(memory_fraction * capacity, free - 2 GiB)``, pinned host memory
    within ``memory_fraction`` of ``available_host_memory()``, else the disk
    tier under ``cache_dir``.
    """
    if not 0 < memory_fraction < 1 or min(batch, length, page_tokens, encoder_chunk, query_chunk,
                                          workspace_mb) < 1:
        raise ValueError("positive sizes and 0 < memory_fraction < 1 required")
    if cache not in ("auto", "cuda", "cpu", "disk"):
        raise ValueError("cache must be auto/cuda/cpu/disk")
    param = next(model.parameters())
    b, heads, hd, topk = model.block_size, model.heads, model.hd, model.topk
    e = param.element_size()
    workspace = workspace_mb << 20
    n_blocks = -(-length // b)
    row_kv = heads * hd * e                        # bytes of one token's K (or V)
    kv_bytes = 2 * batch * length * row_kv

    unit = b * HBM_PAGE_TOKENS // math.gcd(b, HBM_PAGE_TOKENS)
    enc = _largest(encoder_chunk, unit, workspace, batch * (9 * model.dim + 2 * _ffn_width(model)) * e)
    enc = min(enc, -(-length // unit) * unit)
    per_row = 12 * topk + 4 + hd * e               # ids, top scores, log Z_R, output
    qc = 1
    while qc < query_chunk and (sparse_workspace_bytes(batch, qc + 1, heads, hd, topk, n_blocks)
                                + batch * (qc + 1) * heads * per_row) <= workspace:
        qc += 1
    read = sparse_workspace_bytes(batch, qc, heads, hd, topk, n_blocks) + batch * qc * heads * per_row
    head = max(1, min(qc, workspace // max(4 * batch * model.lm_head.out_features, 1)))
    score = _largest(page_tokens, b, workspace, 2 * batch * row_kv)
    score = min(score, -(-length // b) * b)
    enc_bytes = batch * enc * (9 * model.dim + 2 * _ffn_width(model)) * e
    pool_pages = batch * -(-length // HBM_PAGE_TOKENS)
    pool_bytes = 2 * pool_pages * HBM_PAGE_TOKENS * row_kv
    touched = min(batch * qc * heads * (topk + 2), batch * n_blocks) * 2 * b * row_kv
    device_need = {"cuda": pool_bytes + enc_bytes + read,
                   "host": enc_bytes + read + 2 * batch * score * row_kv + touched}

    budget = 0
    if param.is_cuda:
        free, capacity = torch.cuda.mem_get_info(param.device)
        budget = max(0, min(int(capacity * memory_fraction), free - GPU_RESERVE))
    host = available_host_memory()
    host_fits = host is None or kv_bytes <= host * memory_fraction
    if cache == "auto":
        if param.is_cuda and device_need["cuda"] <= budget:
            cache = "cuda"
        elif host_fits:
            cache = "cpu"
        elif cache_dir:
            cache = "disk"
        else:
            raise MemoryError(f"KV requires {kv_bytes / GiB:.2f} GiB; neither HBM nor host memory holds it "
                              "(give cache_dir for the disk tier)")
    if cache == "cuda" and (not param.is_cuda or device_need["cuda"] > budget):
        raise MemoryError(f"GPU KV requires {pool_bytes / GiB:.2f} GiB plus "
                          f"{(enc_bytes + read) / GiB:.2f} GiB of working memory; select cache=auto/cpu/disk")
    if cache == "cpu" and not host_fits:
        raise MemoryError(f"CPU KV requires {kv_bytes / GiB:.2f} GiB; available RAM {host / GiB:.2f} GiB; "
                          "select the disk tier")
    if cache == "disk":
        if not cache_dir:
            raise ValueError("the disk KV tier needs cache_dir on a filesystem with room for the cache")
        os.makedirs(cache_dir, exist_ok=True)
        if kv_bytes + GiB > shutil.disk_usage(cache_dir).free:
            raise MemoryError(f"disk KV requires {kv_bytes / GiB:.2f} GiB; not free under {cache_dir}")
    if cache == "cuda":
        return InferencePlan(cache, kv_bytes, budget, HBM_PAGE_TOKENS, enc, qc, score, head, host,
                             pool_pages, read, device_need["cuda"])
    return InferencePlan(cache, kv_bytes, budget, score, enc, qc, score, head, host, 0, read, device_need["host"])


class KVCache:
    """Write-once raw K/V of one prompt (absolute tokens ``[offset, offset +
    length)``), the reference's ``KVCache`` (``st/runtime/inference.py:19-62``)
    on three tiers:

    * ``"cuda"``: a ``PagedKV`` of 128-token pages in HBM (``paged``),
      written by ``st_paged_kv_write`` and read by the sparse kernels through
      its page table;
    * ``"cpu"``: pinned host tensors ``k, v [B, N, H, hd]``;
    * ``"disk"``: the two halves of one file mapping in a private temporary
      directory under ``cache_dir``, its blocks allocated up front (a full
      filesystem fails here, not half-way through a prefill); ``close``
      removes it.

    All tiers keep the page protocol (``pages``, ``touched_pages``)."""

    def __init__(self, batch, length, heads, dim, dtype, device, plan, offset=0, cache_dir=None):
        shape = (batch, length, heads, dim)
        self.directory = None
        self.paged = None
        self.k = self.v = None
        self.tier = plan.cache
        self.device = torch.device(device)
        self.page_tokens, self.offset, self.length = plan.page_tokens, int(offset), int(length)
        if plan.cache == "cuda":
            self.paged = PagedKV.empty(batch, length, heads, dim, dtype, device, plan.page_tokens, offset)
        elif plan.cache == "cpu":
            self.k, self.v = (torch.empty(shape, dtype=dtype, pin_memory=True) for _ in range(2))
        elif plan.cache == "disk":
            self.k, self.v = self._map_file(shape, dtype, cache_dir)
        else:
            raise ValueError(f"unknown cache tier {plan.cache!r}")

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
        if self.paged is not None:
            self.paged.write(start, k, v)
            return
        lo = start - self.offset
        if lo < 0 or lo + k.shape[1] > self.length:
            raise ValueError("KV write outside owned shard")
        # pageable file memory: a synchronous copy; pinned: stream-ordered
        asynchronous = self.tier != "disk"
        self.k[:, lo:lo + k.shape[1]].copy_(k, non_blocking=asynchronous)
        self.v[:, lo:lo + v.shape[1]].copy_(v, non_blocking=asynchronous)

    def _view(self):
        return self.paged if self.paged is not None else TensorPages(self.k, self.v, self.page_tokens, self.offset)

    def pages(self, device, indices=None, keys_only=False):
        return self._view().pages(device, indices, keys_only)

    def touched_pages(self, ids, pos, b):
        return self._view().touched_pages(ids, pos, b)

    def reader(self, score_tokens):
        """What the sparse operator reads: the page pool in HBM, or a
        streaming view of the host or disk tier."""
        if self.paged is not None:
            return self.paged
        return HostPages(self.k, self.v, self.device, chunk_tokens=score_tokens, offset=self.offset)

    def close(self):
        self.k = self.v = self.paged = None
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
        self.device_positions = dev_pos = positions.to(self.device)
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
            pos = self.device_positions[:, lo:hi]
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
