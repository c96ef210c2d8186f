"""The local blocks' two-block window attention on the HIP kernels.

``HaloMemoryBlock`` (reference ``st/models/blocks.py:102-179``) rotates the
queries and the [previous block ++ own block] keys of every block
(``blocks.py:76-93``) and attends with torch's scaled dot-product attention
under a causal window mask. ``halo_attention`` does the same from the
projection output ``qkv [B, (G+1)*b, 3*H*hd]`` in one kernel per direction:
no rotated copies, no window concatenation, no head permutes, and a
deterministic backward that writes ``d qkv`` directly.
"""
import torch
from torch.autograd.function import once_differentiable

from . import _lib

_tables = {}


def rope_tables(rope, b, dtype, device):
    """cos/sin of positions -b..b-1 as ``RotaryEmbedding.forward`` computes
    them (fp32 angles, rounded to ``dtype``), as fp32 ``[2b, hd/2]``."""
    key = (b, dtype, str(device), float(rope.base), rope.head_dim)
    found = _tables.get(key)
    if found is None:
        # ordinary tensors even when first built under inference_mode: the
        # cache serves later training steps too
        with torch.inference_mode(False), torch.autocast(torch.device(device).type, enabled=False):
            freq = rope.base ** (-rope.frequency_index.to(device).float() / rope.head_dim)
            angle = torch.arange(-b, b, device=device).float()[:, None] * freq
            found = (angle.cos().to(dtype).float().contiguous(), angle.sin().to(dtype).float().contiguous())
        _tables[key] = found
    return found


def halo_supported(qkv, block_size, head_dim):
    """Whether the fused kernels take this projection output and shape."""
    if not (isinstance(qkv, torch.Tensor) and qkv.is_cuda and qkv.dtype in _lib.DTYPE_CODES):
        return False
    return bool(_lib.load().st_halo_supported(_lib.DTYPE_CODES[qkv.dtype], block_size, head_dim))


class _HaloAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, qkv, cos_t, sin_t, b, heads, n, start, first_key):
        lib = _lib.load()
        batch, rows, width = qkv.shape
        hd = width // (3 * heads)
        groups = rows // b - 1
        out = torch.empty((batch, n, heads * hd), device=qkv.device, dtype=qkv.dtype)
        code = _lib.DTYPE_CODES[qkv.dtype]
        _lib.check(lib.st_halo_attn_fwd(code, batch, groups, b, heads, hd, n, start, first_key, _lib.ptr(qkv),
                                        _lib.ptr(cos_t), _lib.ptr(sin_t), _lib.ptr(out), _lib.stream_of(qkv)),
                   lib)
        ctx.save_for_backward(qkv, out)
        ctx.tables = (cos_t, sin_t)  # constants: not saved as autograd inputs
        ctx.args = (code, batch, groups, b, heads, hd, n, start, first_key)
        return out

    @staticmethod
    @once_differentiable
    def backward(ctx, dout):
        lib = _lib.load()
        qkv, out = ctx.saved_tensors
        cos_t, sin_t = ctx.tables
        dout = dout.to(qkv.dtype).contiguous()
        dqkv = torch.empty_like(qkv)
        _lib.check(lib.st_halo_attn_bwd(*ctx.args, _lib.ptr(qkv), _lib.ptr(cos_t), _lib.ptr(sin_t), _lib.ptr(out),
                                        _lib.ptr(dout), _lib.ptr(dqkv), _lib.stream_of(qkv)), lib)
        return dqkv, None, None, None, None, None, None, None


def halo_attention(qkv, rope, block_size, heads, n, start, first_key):
    """Window attention context ``[B, n, H*hd]`` of the first ``n`` query rows
    from ``qkv [B, (G+1)*b, 3*H*hd]`` (raw block 0 = the previous block),
    keys visible within ``[first_key, start + n)``."""
    cos_t, sin_t = rope_tables(rope, block_size, qkv.dtype, qkv.device)
    return _HaloAttention.apply(qkv.contiguous(), cos_t, sin_t, int(block_size), int(heads), int(n), int(start),
                                int(first_key))
