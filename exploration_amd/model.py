"""Stack model over the HIP operators: ``build_model`` / ``StackModel``.

The reference's model (``st/models/stack.py``, ``st/models/blocks.py``,
``st/api.py``, ``st/config.py``) restated for one GPU, with the same module
names, parameter shapes and forward semantics, so that a reference
state_dict loads unchanged. Its global read rounds call this package's
``dense_attention`` (training, ``forward_loss``) and ``sparse_attention``
(inference with ``topk`` below the number of blocks): the operators of the
hot path. Everything else (layer norms, projections, the local halo
attention over two blocks, the loss) is ordinary PyTorch.

Single process: the reference's context-parallel hooks (halo exchange,
Ulysses all-to-all, position gathers; ``st/runtime/parallel.py``) are the
identity here. The reference's differentiable sparse plumbing
(``stack.py:333-383``), which it keeps for mathematical checks only, is not
shipped: a gradient-enabled sparse forward raises ``ValueError``.
"""
import contextlib
import math
import re
from dataclasses import asdict, dataclass, fields
from numbers import Integral

import torch
from torch import nn
from torch.nn import functional as F
from torch.utils.checkpoint import checkpoint

from .attention import dense_attention
from .local import halo_attention, halo_supported
from .sparse import TensorPages, sparse_attention


@dataclass(frozen=True)
class ModelConfig:
    """``st/config.py:5-31`` (the stack model only)."""
    model: str = "stack"
    vocab_size: int = 128
    dim: int = 256
    heads: int = 4
    block_size: int = 16
    topk: int = 64
    arch: str = "Lx2,G"
    ffn_ratio: float = 4.
    layers: int = 3

    @classmethod
    def from_dict(cls, value):
        if isinstance(value, cls):
            return value
        unknown = set(value) - {f.name for f in fields(cls)}
        if unknown:
            raise ValueError(f"unknown model configuration keys: {sorted(unknown)}")
        return cls(**value)

    def to_dict(self):
        if self.model != "stack":
            raise ValueError("only the stack model is built here (the baseline transformer is out of scope)")
        out = asdict(self)
        out.pop("layers")
        return out


@dataclass(frozen=True)
class ExecutionConfig:
    """``st/config.py:34-60``: operator backend and chunk sizes."""
    backend: str = "auto"
    checkpoint_chunks: bool = True
    encoder_chunk: int = 1024
    query_chunk: int = 0
    loss_chunk: int = 128
    flash_attention: str = "auto"
    attention_q_chunk: int = 128
    attention_kv_chunk: int = 4096

    def __post_init__(self):
        if self.backend not in ("auto", "torch", "triton", "hip"):
            raise ValueError("backend must be auto, torch, triton or hip")


_ARCH_ITEM = re.compile(r"\((?P<shared>[^()]*)\)x(?P<repeat>.*)|(?P<kind>[^()x]*)(?:x(?P<count>.*))?", re.S)


def parse_arch(arch):
    """Layer plan of a Stack model, ``'Lx2,(G)x4'`` -> ``[(kind, count,
    shared), ...]`` in application order (the reference's grammar,
    ``st/models/stack.py:75-106``).

    Items are comma separated. ``L`` is a local halo encoder block, ``G`` a
    global read round. ``XxN`` stacks N layers with their own weights,
    ``(X)xN`` applies one shared layer N times, bare ``X`` is one layer. N is
    a positive decimal integer (an empty ``Xx`` is rejected). The model
    encodes, then reads: no ``L`` item may follow a ``G`` item."""
    if not isinstance(arch, str) or not arch.strip():
        raise ValueError("arch must be a nonempty spec like 'Lx2,G'")
    spec, reading = [], False
    for item in (part.strip() for part in arch.split(",")):
        m = _ARCH_ITEM.fullmatch(item)
        if m is None or (m["kind"] is None and m["shared"] is None):
            if item.startswith("("):
                raise ValueError(f"shared layers must look like '(X)xN': {item!r}")
            raise ValueError(f"unknown layer kind in arch item {item!r} (want L or G)")
        shared = m["shared"] is not None
        kind = m["shared"] if shared else m["kind"]
        count = m["repeat"] if shared else ("1" if m["count"] is None else m["count"])
        if kind not in ("L", "G"):
            raise ValueError(f"unknown layer kind in arch item {item!r} (want L or G)")
        if not re.fullmatch(r"[0-9]+", count) or int(count) == 0:
            raise ValueError(f"repeat count must be a positive integer in {item!r}")
        if kind == "L" and reading:
            raise ValueError("all L layers must precede all G layers (encode -> read)")
        reading = reading or kind == "G"
        spec.append((kind, int(count), shared))
    return spec


class RotaryEmbedding(nn.Module):
    """Split-half rotary embedding at given positions (``blocks.py:76-93``):
    frequencies base^(-i/hd) for even i, angles in fp32 outside autocast."""

    def __init__(self, head_dim, base=10_000.0):
        super().__init__()
        self.head_dim, self.base = head_dim, base
        self.register_buffer("frequency_index", torch.arange(0, head_dim, 2), persistent=False)

    def forward(self, x, positions):
        with torch.autocast(device_type=x.device.type, enabled=False):
            freq = self.base ** (-self.frequency_index.float() / self.head_dim)
            angle = positions.float()[..., None] * freq
            cos, sin = angle.cos()[..., None, :].to(x.dtype), angle.sin()[..., None, :].to(x.dtype)
        lo, hi = x.chunk(2, dim=-1)
        return torch.cat([lo * cos - hi * sin, hi * cos + lo * sin], dim=-1)


def _column_sum(t):
    """Sum of a ``[R, C]`` tensor over its rows (accumulated in at least
    fp32), in stages of at most 128 rows: every reduction is short, so the
    library never splits one across workgroups (a split reduction clears its
    semaphore with a memset, and such graph nodes have gone stale on replays
    of a captured step)."""
    dtype = torch.promote_types(t.dtype, torch.float32)
    acc = None
    while t.shape[0] > 128:
        r = t.shape[0] // 128 * 128
        if r < t.shape[0]:
            tail = t[r:].sum(0, dtype=dtype)
            acc = tail if acc is None else acc + tail
        t = t[:r].reshape(-1, 128, t.shape[1]).sum(1, dtype=dtype)
    s = t.sum(0, dtype=dtype)
    return s if acc is None else s + acc


# Weight casts of one training step under autocast without its cast cache
# (the graph-captured step): None, or {id(weight): _StepWeight} while
# weights_cast_once() is active.
_STEP_CASTS = {"cache": None}


class _StepWeight:
    """An fp32 weight's low-precision copy for one step, and the fp32 sum of
    its uses' gradients (``grad`` None until the first one arrives)."""

    def __init__(self, weight):
        self.weight = weight
        self.low = weight.detach().to(torch.get_autocast_dtype(weight.device.type))
        self.grad = None


class _CastUse(torch.autograd.Function):
    """One use of the step's shared low-precision copy of an fp32 weight, in
    place of autocast's cast at that use. The forward returns the copy (the
    same values as the cast). The backward adds this use's gradient, in fp32,
    to the weight's step sum: the first use's converted (``copy_``), each
    later one added (``add_``), in the order the backward produces them. That
    is the sum autograd forms of the casts' fp32 gradients (it keeps the first
    and adds the others as they arrive), with one kernel per use instead of a
    cast kernel plus an add; ``weights_cast_once`` hands the sum to the weight
    as its gradient."""

    @staticmethod
    def forward(ctx, low, weight, step):
        ctx.step = step
        return low.view_as(low)

    @staticmethod
    def backward(ctx, grad):
        step = ctx.step
        if step.grad is None:
            step.grad = torch.empty_like(step.weight).copy_(grad)
        else:
            step.grad.add_(grad)
        return None, None, None


def _w(weight):
    """A linear layer's weight at its use: inside ``weights_cast_once()``,
    under autocast with gradients, the step's shared low-precision copy
    (cast at the first use); otherwise the weight itself (autocast casts it)."""
    cache = _STEP_CASTS["cache"]
    if (cache is None or weight.dtype != torch.float32 or not torch.is_grad_enabled()
            or not torch.is_autocast_enabled(weight.device.type)):
        return weight
    step = cache.get(id(weight))
    if step is None or step.weight is not weight:
        step = cache[id(weight)] = _StepWeight(weight)
    return _CastUse.apply(step.low, weight, step)


@contextlib.contextmanager
def weights_cast_once():
    """Scope of one training step (forward and backward, whose checkpointed
    chunks recompute their forward): each fp32 weight is cast to the autocast
    dtype once and every linear use reads that copy; on leaving the scope the
    uses' fp32 gradient sum becomes the weight's gradient (added before any
    gradient autograd gave the weight directly: the embedding's, whose
    backward runs after every use of the tied output weight). For steps whose
    autocast runs without its own cast cache (graph capture), which otherwise
    casts the weight again at every use."""
    previous = _STEP_CASTS["cache"]
    cache = _STEP_CASTS["cache"] = {}
    try:
        yield
        for step in cache.values():
            if step.grad is not None:
                w = step.weight
                w.grad = step.grad if w.grad is None else step.grad.add_(w.grad)
    finally:
        _STEP_CASTS["cache"] = previous


class _BiasAdd(torch.autograd.Function):
    """``y + b`` (b cast to y's dtype, as a fused linear bias under autocast);
    the bias gradient through ``_column_sum``."""

    @staticmethod
    def forward(ctx, y, b):
        ctx.b_dtype = b.dtype
        return y + b.to(y.dtype)

    @staticmethod
    def backward(ctx, grad):
        return grad, _column_sum(grad.reshape(-1, grad.shape[-1])).to(ctx.b_dtype)


class FeedForward(nn.Sequential):
    """Linear -> GELU -> Linear, hidden width round(dim * ratio) (``blocks.py:96-99``).
    The biases are added outside the matrix products, so their gradients are
    the staged column sums of ``_BiasAdd`` (same parameters and state_dict
    as the reference's ``nn.Sequential``)."""

    def __init__(self, dim, ratio):
        hidden = max(1, round(dim * ratio))
        super().__init__(nn.Linear(dim, hidden), nn.GELU(), nn.Linear(hidden, dim))

    def forward(self, x):
        fc1, act, fc2 = self
        h = act(_BiasAdd.apply(F.linear(x, _w(fc1.weight)), fc1.bias))
        return _BiasAdd.apply(F.linear(h, _w(fc2.weight)), fc2.bias)


def _window_attention(q, k, v, mask):
    """q ``[B,G,T,H,hd]`` against k/v ``[B,G,K,H,hd]`` under a boolean
    ``[B|1,G,T,K]`` mask (every row sees at least one key)."""
    batch, groups, length, heads, hd = q.shape
    flat = lambda t: t.permute(0, 1, 3, 2, 4).reshape(batch * groups, heads, t.shape[2], hd)
    m = mask.expand(batch, groups, length, k.shape[2]).reshape(batch * groups, 1, length, k.shape[2])
    out = F.scaled_dot_product_attention(flat(q), flat(k), flat(v), attn_mask=m)
    return out.reshape(batch, groups, heads, length, hd).permute(0, 1, 3, 2, 4)


class HaloMemoryBlock(nn.Module):
    """Pre-norm causal attention of each block over [previous block ++ own
    block], then an FFN, streamed over query chunks of whole blocks
    (``blocks.py:102-179``). RoPE is applied at offsets relative to the query
    block (q at 0..b-1, keys at -b..b-1)."""

    def __init__(self, dim, heads, block_size, rope, ffn_ratio, query_chunk_size, checkpoint_chunks=False):
        super().__init__()
        self.heads, self.hd = heads, dim // heads
        self.block_size, self.query_chunk_size = block_size, query_chunk_size
        self.rope = rope
        self.checkpoint_chunks = checkpoint_chunks
        self.attn_norm = nn.LayerNorm(dim)
        self.qkv = nn.Linear(dim, 3 * dim, bias=False)
        self.out = nn.Linear(dim, dim, bias=False)
        self.ffn_norm = nn.LayerNorm(dim)
        self.ffn = FeedForward(dim, ffn_ratio)
        # the fused window-attention kernels for supported GPU shapes (False:
        # always the PyTorch attention below)
        self.fused = True

    def forward_chunk(self, x, previous=None, start=0):
        batch, n, dim = x.shape
        b = self.block_size
        if start % b:
            raise ValueError("halo chunk start must be block aligned")
        groups = -(-n // b)
        if previous is None:
            previous, first_key = x.new_zeros(batch, b, dim), start
        else:
            if previous.shape != (batch, b, dim):
                raise ValueError("previous halo must contain exactly one block")
            first_key = max(0, start - b)
        seq = torch.cat((previous, F.pad(x, (0, 0, 0, groups * b - n))), 1)
        qkv = F.linear(self.attn_norm(seq), _w(self.qkv.weight))
        if self.fused and halo_supported(qkv, b, self.hd):
            # rotary, window and attention in one kernel per direction
            ctx = halo_attention(qkv, self.rope, b, self.heads, n, start, first_key)
            y = x + F.linear(ctx, _w(self.out.weight))
            return y + self.ffn(self.ffn_norm(y))
        qkv = qkv.reshape(batch, groups + 1, b, 3, self.heads, self.hd)
        q, k, v = qkv.unbind(3)
        q = self.rope(q[:, 1:], torch.arange(b, device=x.device))
        kw = self.rope(torch.cat((k[:, :-1], k[:, 1:]), 2), torch.arange(-b, b, device=x.device))
        vw = torch.cat((v[:, :-1], v[:, 1:]), 2)
        qo = torch.arange(b, device=x.device)[:, None]
        ko = torch.arange(2 * b, device=x.device)[None, :]
        key_pos = start + (torch.arange(groups, device=x.device)[:, None, None] - 1) * b + ko
        mask = (ko <= qo + b)[None] & (key_pos >= first_key) & (key_pos < start + n)
        ctx = _window_attention(q, kw, vw, mask[None]).reshape(batch, groups * b, dim)[:, :n]
        y = x + F.linear(ctx, _w(self.out.weight))
        return y + self.ffn(self.ffn_norm(y))

    def forward(self, x, positions=None, previous=None, start=0):
        if positions is not None:
            start = int(positions[0])
        step = self.query_chunk_size * self.block_size
        b = self.block_size
        outs = []
        # the chunks as one split of x (its backward is one concatenation; a
        # basic slice per chunk would make every chunk's backward a
        # zero-filled x-sized gradient, added up over the chunks), and the
        # halo blocks (the last block of every chunk but the last) as one
        # copy of a strided view of x, so that all of them cost one x-sized
        # gradient in backward. Both keep the gradient's sums exactly those of
        # slicing every chunk and halo (a slice of the previous piece would
        # sum them in another order).
        pieces = x.split(step, 1) if x.shape[1] > step else (x,)
        if len(pieces) > 1:
            halos = x[:, :(len(pieces) - 1) * step].unflatten(1, (len(pieces) - 1, step))[:, :, step - b:]
            halos = halos.contiguous()
        for i, piece in enumerate(pieces):
            lo = i * step
            prev = previous if i == 0 else halos[:, i - 1]
            if self.checkpoint_chunks and torch.is_grad_enabled():
                outs.append(checkpoint(self.forward_chunk, piece, prev, start + lo, use_reentrant=False,
                                       preserve_rng_state=False))
            else:
                outs.append(self.forward_chunk(piece, prev, start + lo))
        return torch.cat(outs, 1)


class KVProjection(nn.Module):
    """LayerNorm + linear to (k, v) per head, in token chunks (``blocks.py:182-207``)."""

    def __init__(self, dim, heads, rope, use_rope=True, chunk_tokens=1 << 16):
        super().__init__()
        self.heads, self.hd = heads, dim // heads
        self.norm = nn.LayerNorm(dim)
        self.proj = nn.Linear(dim, 2 * dim, bias=False)
        self.rope, self.use_rope, self.chunk_tokens = rope, use_rope, chunk_tokens

    def forward(self, x, positions):
        ks, vs = [], []
        for lo in range(0, x.shape[1], self.chunk_tokens):
            sl = slice(lo, lo + self.chunk_tokens)
            k, v = F.linear(self.norm(x[:, sl]), _w(self.proj.weight)).reshape(
                x.shape[0], -1, 2, self.heads, self.hd).unbind(2)
            if self.use_rope:
                k = self.rope(k, positions[sl])
            ks.append(k)
            vs.append(v)
        return torch.cat(ks, 1), torch.cat(vs, 1)


class GlobalReadBlock(nn.Module):
    """Query-side weights of one global read round (``stack.py:109-124``)."""

    def __init__(self, dim, ffn_ratio):
        super().__init__()
        self.q_norm = nn.LayerNorm(dim)
        self.wq = nn.Linear(dim, dim, bias=False)
        self.read_out = nn.Linear(dim, dim, bias=False)
        self.ffn_norm = nn.LayerNorm(dim)
        self.ffn = FeedForward(dim, ffn_ratio)


def _positive_int(value):
    return isinstance(value, Integral) and not isinstance(value, bool) and value >= 1


class StackModel(nn.Module):
    """``forward([B,N], sup=None) -> [B,N,vocab]`` and ``forward_loss``
    (``stack.py:127-462``). Raw K/V are written once after the last local
    block; every global round reads them through the gated attention
    operator with its own query projection."""

    def __init__(self, vocab_size, dim=256, heads=4, block_size=16, topk=64, arch="Lx2,G", ffn_ratio=4,
                 pos_chunk=0, backend="auto", checkpoint_chunks=False, encoder_chunk=1024, loss_chunk=128,
                 attention_q_chunk=128, attention_kv_chunk=4096):
        super().__init__()
        for name, value in (("vocab_size", vocab_size), ("dim", dim), ("heads", heads),
                            ("block_size", block_size), ("topk", topk)):
            if not _positive_int(value):
                raise ValueError(f"{name} must be a positive integer")
        if isinstance(pos_chunk, bool) or not isinstance(pos_chunk, Integral) or pos_chunk < 0:
            raise ValueError("pos_chunk must be a non-negative integer (0 = auto)")
        if block_size < 2:
            raise ValueError("block_size must be at least 2")
        if dim % heads or (dim // heads) % 2:
            raise ValueError("dim / heads must be an even integer for RoPE")
        if not math.isfinite(ffn_ratio) or ffn_ratio <= 0:
            raise ValueError("ffn_ratio must be finite and positive")
        if backend not in ("auto", "torch", "triton", "hip"):
            raise ValueError("backend must be auto, torch, triton or hip")
        chunks = (encoder_chunk, loss_chunk, attention_q_chunk, attention_kv_chunk)
        if not all(_positive_int(c) for c in chunks) or encoder_chunk < block_size:
            raise ValueError("encoder_chunk >= block_size and attention/loss chunks > 0 required")
        self.dim, self.heads, self.hd = dim, heads, dim // heads
        self.block_size, self.topk, self.pos_chunk, self.arch = block_size, topk, pos_chunk, arch
        self.backend, self.checkpoint_chunks, self.loss_chunk = backend, checkpoint_chunks, loss_chunk
        self.attention_q_chunk, self.attention_kv_chunk = attention_q_chunk, attention_kv_chunk
        self.embedding = nn.Embedding(vocab_size, dim)
        nn.init.normal_(self.embedding.weight, std=0.02)
        self.rope = RotaryEmbedding(self.hd)
        shared, local, reads = {}, [], []
        for kind, count, is_shared in parse_arch(arch):
            for _ in range(count):
                if is_shared and kind in shared:
                    layer = shared[kind]
                elif kind == "L":
                    layer = HaloMemoryBlock(dim, heads, block_size, self.rope, ffn_ratio,
                                            max(1, encoder_chunk // block_size), checkpoint_chunks)
                else:
                    layer = GlobalReadBlock(dim, ffn_ratio)
                if is_shared:
                    shared[kind] = layer
                (local if kind == "L" else reads).append(layer)
        self.local = nn.ModuleList(local)
        self.reads = nn.ModuleList(reads)
        self.raw_kv = KVProjection(dim, heads, self.rope, use_rope=False)
        self.final_norm = nn.LayerNorm(dim)
        self.lm_head = nn.Linear(dim, vocab_size, bias=False)
        self.lm_head.weight = self.embedding.weight

    # ----------------------------------------------------------------- encode
    def encode(self, input_ids, offset=0):
        """Tokens -> (x, raw_k, raw_v), raw K/V contiguous ``[B,N,H,hd]``."""
        if input_ids.ndim != 2 or min(input_ids.shape) < 1:
            raise ValueError("input_ids must have nonempty shape [batch, sequence]")
        x = self.embed(input_ids)
        for layer in self.local:
            x = layer(x, start=offset)
        raw_k, raw_v = self.raw_kv(x, None)
        # one copy here instead of one per operator call
        return x, raw_k.contiguous(), raw_v.contiguous()

    def embed(self, input_ids):
        """``self.embedding(ids)`` without the embedding's sort-based backward
        (a device sort and a look-back segment pass). Vocabularies up to 4096
        (the byte-level configurations) with at most 2^28 one-hot elements: a
        one-hot fp32 product, exactly the weight rows forward and a
        fixed-order, deterministic product backward. Otherwise: a row gather,
        whose backward adds rows with atomics."""
        w = self.embedding.weight
        flat = input_ids.reshape(-1)
        if w.shape[0] <= 4096 and flat.numel() * w.shape[0] <= 1 << 28:
            with torch.autocast(w.device.type, enabled=False):
                onehot = F.one_hot(flat, w.shape[0]).to(w.dtype)
                x = onehot @ w
        else:
            x = w.index_select(0, flat)
        return x.view(*input_ids.shape, w.shape[1])

    def _chunk_size(self, n):
        """Supervised positions per read chunk (``stack.py:315-331``): bounds
        the largest per-chunk temporary by an element budget."""
        if self.pos_chunk > 0:
            return self.pos_chunk
        groups = -(-n // self.block_size)
        m = min(self.topk, groups)
        per_pos = self.heads * (n + 2 * m * self.block_size * self.hd)
        cap, budget = (2048, 1 << 31) if self.dim <= 512 else (512, 1 << 29)
        return min(cap, max(16, budget // max(per_pos, 1)))

    # ------------------------------------------------------------ dense reads
    def _dense_round(self, rd, z, k, v, positions):
        """``stack.py:198-213``: q from z, the gated dense operator, readout and FFN."""
        def project(hidden):
            return F.linear(rd.q_norm(hidden), _w(rd.wq.weight))

        def finish(hidden, context):
            hidden = hidden + F.linear(context, _w(rd.read_out.weight))
            return hidden + rd.ffn(rd.ffn_norm(hidden))

        ckpt = self.checkpoint_chunks and torch.is_grad_enabled()
        q = checkpoint(project, z, use_reentrant=False, preserve_rng_state=False) if ckpt else project(z)
        q = q.reshape(*z.shape[:2], self.heads, self.hd)
        ctx = dense_attention(q, k, v, positions, self.block_size, self.backend,
                              q_chunk=self.attention_q_chunk, kv_chunk=self.attention_kv_chunk)
        ctx = ctx.reshape(*z.shape[:2], self.dim)
        return checkpoint(finish, z, ctx, use_reentrant=False, preserve_rng_state=False) if ckpt else finish(z, ctx)

    def forward_loss(self, input_ids, targets, sup=None, offset=0, width=None):
        """Dense training loss (``stack.py:215-279``): SUM of token losses and
        counts at the supervised positions, never ``[B,N,V]``.

        ``width`` (optional) is the number of query slots per row; it must be
        at least the largest supervised count of a row (``N`` always is).
        Given, it spares the one host synchronisation that reads that count,
        so the step can be captured into a graph."""
        if input_ids.ndim != 2 or input_ids.shape != targets.shape or min(input_ids.shape) < 1:
            raise ValueError("ids and targets must have identical nonempty [B,N] shape")
        if sup is None:
            sup = targets != -100
        if sup.shape != targets.shape or sup.dtype != torch.bool:
            raise ValueError("sup must be bool [B,N]")
        sup = sup & (targets != -100)
        batch, n = input_ids.shape
        if width is None:
            width = int(sup.sum(1).max())
        elif not 1 <= width <= n:
            raise ValueError("width must lie in [1, sequence length]")
        width = max(int(width), 1)
        # supervised positions of each row in increasing order, padded with n:
        # a row prefix sum gives each one its slot, a scatter places it (the
        # unsupervised ones all land in a discarded extra column). No sort and
        # no boolean selection: those run rocprim look-back scans that clear
        # their counters with a memset, and a captured memset node has not
        # re-run reliably on replays here (a replayed partition kernel then
        # wrote out of bounds: a memory aperture fault).
        idx = torch.arange(n, device=input_ids.device)[None].expand(batch, -1)
        # (a zero row keeps the prefix sum a per-row scan: one row alone goes
        # to the library's device-wide scan, which is a look-back scan)
        count = torch.cat((sup.long(), sup.new_zeros((1, n), dtype=torch.long))).cumsum(1)[:batch]
        slot = torch.where(sup, count - 1, n)
        order = torch.full((batch, n + 1), n, device=input_ids.device, dtype=torch.long)
        order = order.scatter_(1, slot, idx)[:, :width]
        valid = order < n
        safe = order.clamp_max(n - 1)
        pos = torch.where(valid, order + offset, -1)
        labels = targets.gather(1, safe).masked_fill(~valid, -100)
        x, k, v = self.encode(input_ids, offset)
        losses, hits = [], []
        step = self._chunk_size(n)
        # the supervised rows in slot order, gathered once and split into
        # the read chunks (backward: one scatter-add into a zero-filled x
        # gradient and one concatenation, instead of both per chunk; advanced
        # indexing's backward sorts and runs a look-back unique pass)
        rows = torch.gather(x, 1, safe[:, :, None].expand(-1, -1, x.shape[-1]))
        rows = rows.split(step, 1) if width > step else (rows,)

        def head_loss(hidden, lab):
            logits = F.linear(self.final_norm(hidden), _w(self.lm_head.weight)).float()
            loss = F.cross_entropy(logits.flatten(0, 1), lab.flatten(), ignore_index=-100, reduction="sum")
            return loss, (logits.argmax(-1) == lab) | (lab == -100)

        for lo in range(0, width, step):
            hi = min(lo + step, width)
            z = rows[lo // step]
            for rd in self.reads:
                z = self._dense_round(rd, z, k, v, pos[:, lo:hi])
            for j in range(0, hi - lo, self.loss_chunk):
                lab = labels[:, lo + j:min(lo + j + self.loss_chunk, hi)]
                h = z[:, j:j + self.loss_chunk]
                if self.checkpoint_chunks and torch.is_grad_enabled():
                    loss, hit = checkpoint(head_loss, h, lab, use_reentrant=False, preserve_rng_state=False)
                else:
                    loss, hit = head_loss(h, lab)
                losses.append(loss)
                hits.append(hit.detach())
        hit = torch.cat(hits, 1)
        return {"loss_sum": torch.stack(losses).sum(), "count": valid.sum(), "correct": (hit & valid).sum(),
                "row_errors": ((~hit) & valid).sum(1), "positions": pos, "hits": hit}

    @staticmethod
    def supervised_positions(sup, n):
        """``[B,S]`` supervised positions (equal count per row), or None for all."""
        if sup is None:
            return None, n
        counts = sup.sum(1)
        s = int(counts[0])
        if s < 1 or not bool((counts == s).all()):
            raise ValueError("sup must mark the same positive count per row")
        return sup.nonzero()[:, 1].reshape(sup.shape[0], s), s

    def read_rounds(self, z, raw_k, raw_v, positions, cache=None):
        """All global rounds for query states z at ``positions``: the dense
        operator when ``topk`` covers every block, else (no gradient) the
        sparse operator over ``cache`` (default: raw K/V as pages,
        ``stack.py:437-446``)."""
        b = self.block_size
        n = raw_k.shape[1] if raw_k is not None else cache.length
        groups = -(-n // b)
        if self.topk >= groups:
            for rd in self.reads:
                z = self._dense_round(rd, z, raw_k, raw_v, positions)
            return z
        if torch.is_grad_enabled():
            raise ValueError("the sparse read is inference-only: call under torch.no_grad() or use forward_loss")
        if cache is None:
            cache = TensorPages(raw_k, raw_v, page_tokens=max(b, 65536 // b * b))
        batch, count = z.shape[:2]
        for rd in self.reads:
            q = rd.wq(rd.q_norm(z)).reshape(batch, count, self.heads, self.hd)
            ctx = sparse_attention(q, cache, positions, b, min(self.topk, groups), self.backend)
            z = z + rd.read_out(ctx.reshape(batch, count, self.dim).to(z.dtype))
            z = z + rd.ffn(rd.ffn_norm(z))
        return z

    def forward(self, input_ids, sup=None, *, targets=None, offset=0, compact=False):
        if targets is not None:
            return self.forward_loss(input_ids, targets, sup, offset)
        if input_ids.ndim != 2 or min(input_ids.shape) < 1:
            raise ValueError("input_ids must have nonempty shape [batch, sequence]")
        batch, n = input_ids.shape
        x, raw_k, raw_v = self.encode(input_ids)
        pos, count = self.supervised_positions(sup, n)
        if pos is None:
            pos = torch.arange(n, device=x.device)[None].expand(batch, n)
        rows = torch.arange(batch, device=x.device)[:, None]
        outs = []
        step = self._chunk_size(n)
        for lo in range(0, count, step):
            pc = pos[:, lo:min(count, lo + step)]
            outs.append(self.read_rounds(x[rows, pc], raw_k, raw_v, pc))
        logits = self.lm_head(self.final_norm(torch.cat(outs, 1)))
        if compact:
            return logits
        full = logits.new_zeros(batch, n, logits.shape[-1])
        full[rows, pos] = logits
        return full


def build_model(config=ModelConfig(), *, execution=ExecutionConfig(), device="cpu", dtype=None):
    """``st/api.py:10-32`` for the stack model."""
    config = ModelConfig.from_dict(config)
    if isinstance(execution, dict):
        execution = ExecutionConfig(**execution)
    options = config.to_dict()
    options.pop("model")
    with torch.device(device):
        model = StackModel(**options, backend=execution.backend, checkpoint_chunks=execution.checkpoint_chunks,
                           encoder_chunk=execution.encoder_chunk, pos_chunk=execution.query_chunk,
                           loss_chunk=execution.loss_chunk, attention_q_chunk=execution.attention_q_chunk,
                           attention_kv_chunk=execution.attention_kv_chunk)
    model.model_config = config
    if dtype is not None:
        model.to(dtype=dtype)
    return model


STACK_100M = {"vocab_size": 256, "dim": 1024, "heads": 16, "block_size": 16, "topk": 64, "arch": "Lx7,G",
              "ffn_ratio": 4.0}
"""``configs/stack_100m.json`` (model section)."""
