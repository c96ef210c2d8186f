"""Exact gated dense block attention on gfx950: the drop-in for ``st.ops``.

``dense_attention`` keeps the reference signature
(``st/ops/attention.py:148``); the forward and backward run the HIP kernels
of ``libst_attn.so`` through ``torch.autograd.Function`` (reference
``st/ops/kernels/dense.py:195-239``). The remote gate is
``log M_j - log Z_R`` with ``M_j = sum_{i in j} exp(q.k_i)``; both gate terms
enter the backward. No Q x N tensor is allocated.

Backends: ``"auto"`` and ``"triton"`` (kept as the reference's name for "the
fused kernel is required") and ``"hip"`` run the HIP kernels and raise
``ValueError`` for configurations outside their envelope. ``"torch"`` is the
reference's portable restatement and is not part of this package.
"""
import torch

from . import _lib

BACKENDS = ("auto", "torch", "triton", "hip")

_records = {}


def _record(kernel, q, block_size, extra=None):
    key = (kernel, q.device.index, str(q.dtype), q.shape[-1], block_size)
    if key not in _records:
        rec = {"kernel": kernel, "path": "hip", "device": q.device.index, "dtype": str(q.dtype),
               "head_dim": q.shape[-1], "block_size": block_size}
        rec.update(extra or {})
        _records[key] = rec


def launch_report():
    """Kernels launched so far with their configuration (reference
    ``st/ops/kernels/launch.py:96-98``)."""
    return list(_records.values())


def hip_supported(q, block_size):
    """Whether the fused HIP kernels handle this query tensor and block size
    (the reference's ``triton_supported``, ``st/ops/attention.py:142-145``):
    a ROCm device tensor in fp32/fp16/bf16, ``block_size`` a power of two in
    [2, 128] and ``head_dim <= 256`` (head dimensions that are not a
    multiple of 8 run on zero-padded rows, as the reference pads D to a power
    of two inside its kernel, ``st/ops/kernels/dense.py:210``)."""
    if not (isinstance(q, torch.Tensor) and q.is_cuda and q.dtype in _lib.DTYPE_CODES):
        return False
    b = int(block_size)
    return 2 <= b <= 128 and b & (b - 1) == 0 and 1 <= q.shape[-1] <= 256


# The reference's name for the capability predicate.
triton_supported = hip_supported


def _check_inputs(q, k, v, positions, block_size, q_chunk=1, kv_chunk=1):
    """Shape checks of ``st/ops/attention.py:157-162``."""
    if q.ndim != 4 or k.ndim != 4 or k.shape != v.shape or positions.shape != q.shape[:2]:
        raise ValueError("expected q[B,Q,H,D], k/v[B,N,H,D], positions[B,Q]")
    if k.shape[0] != q.shape[0] or k.shape[2:] != q.shape[2:]:
        raise ValueError("query and KV batch/head dimensions differ")
    if min(q.shape) < 1 or k.shape[1] < 1 or min(block_size, q_chunk, kv_chunk) < 1:
        raise ValueError("attention dimensions and tile sizes must be positive")


class _DenseHip(torch.autograd.Function):
    @staticmethod
    def forward(ctx, q, k, v, positions, block_size):
        lib = _lib.load()
        q, k, v = (t.contiguous() for t in (q, k, v))
        positions = positions.to(device=q.device, dtype=torch.int64).contiguous()
        batch, queries, heads, dim = q.shape
        keys = k.shape[1]
        out = torch.empty_like(q)
        rc = torch.empty(q.shape, device=q.device, dtype=torch.float32)
        pr = torch.empty(q.shape[:3], device=q.device, dtype=torch.float32)
        zr, z = torch.empty_like(pr), torch.empty_like(pr)
        code = _lib.DTYPE_CODES[q.dtype]
        ws_bytes = lib.st_dense_fwd_workspace_bytes(code, batch, queries, keys, heads, dim, block_size)
        ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8) if ws_bytes else None
        _lib.check(lib.st_dense_fwd(code, batch, queries, keys, heads, dim, block_size,
                                    _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(positions),
                                    _lib.ptr(out), _lib.ptr(rc), _lib.ptr(pr), _lib.ptr(zr), _lib.ptr(z),
                                    _lib.ptr(ws), ws_bytes, _lib.stream_of(q)), lib)
        _record("dense_fwd", q, block_size)
        ctx.save_for_backward(q, k, v, positions, out, rc, pr, zr, z)
        ctx.block_size = block_size
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad):
        lib = _lib.load()
        q, k, v, positions, out, rc, pr, zr, z = ctx.saved_tensors
        grad = grad.to(q.dtype).contiguous()
        batch, queries, heads, dim = q.shape
        keys = k.shape[1]
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        code = _lib.DTYPE_CODES[q.dtype]
        ws_bytes = lib.st_dense_bwd_workspace_bytes(code, batch, queries, keys, heads, dim, ctx.block_size)
        ws = torch.empty(ws_bytes, device=q.device, dtype=torch.uint8)
        _lib.check(lib.st_dense_bwd(code, batch, queries, keys, heads, dim, ctx.block_size,
                                    _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(positions),
                                    _lib.ptr(out), _lib.ptr(rc), _lib.ptr(pr), _lib.ptr(zr), _lib.ptr(z),
                                    _lib.ptr(grad), _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv),
                                    _lib.ptr(ws), ws_bytes, _lib.stream_of(q)), lib)
        _record("dense_bwd", q, ctx.block_size)
        return dq, dk, dv, None, None


def dense_forward_stats(q, k, v, positions, block_size):
    """Forward without autograd, returning ``(out, rc, pr, zr, z)``: the output
    and the statistics saved for backward (reference
    ``st/ops/kernels/dense.py:200-215``)."""
    with torch.no_grad():
        ctx = type("Ctx", (), {"save_for_backward": lambda self, *t: setattr(self, "saved", t)})()
        _DenseHip.forward(ctx, q, k, v, positions, int(block_size))
        return ctx.saved[4:]


def dense_hip(q, k, v, positions, block_size, *, force_streamed=False):
    """Fused forward (autograd-aware) with the reference's internal signature
    ``dense_triton(q, k, v, positions, block_size, *, force_streamed=False)``
    (``st/ops/kernels/dense.py:236-239``). ``force_streamed`` selects the
    reference's small-tile fallback for NVIDIA shared-memory limits
    (``st/ops/kernels/streamed.py``); every supported configuration fits the
    LDS of one compute unit here, so both settings run the same kernels."""
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError("q/k/v must use the same dtype")
    if not (k.device == q.device and v.device == q.device and positions.device == q.device):
        raise ValueError("q, k, v and positions must be on the same device")
    return _DenseHip.apply(q, k, v, positions, int(block_size))


def dense_attention(q, k, v, positions, block_size, backend="auto", q_chunk=32, kv_chunk=1024):
    """[B,Q,H,D] x [B,N,H,D], positions [B,Q]; -1 denotes padding.

    Same signature and checks as the reference (``st/ops/attention.py:148-176``).
    ``q_chunk``/``kv_chunk`` tile the reference's torch path only and are
    validated but otherwise unused. First derivatives only.
    """
    if backend not in BACKENDS:
        raise ValueError(f"unknown attention backend {backend!r}")
    _check_inputs(q, k, v, positions, block_size, q_chunk, kv_chunk)
    if backend == "torch":
        raise ValueError("backend 'torch' is the reference's portable restatement; "
                         "this package only provides the fused HIP kernels")
    if not hip_supported(q, block_size):
        raise ValueError("the HIP kernels require ROCm fp16/bf16/fp32 tensors, head_dim <= 256 "
                         "and a power-of-two block_size in 2..128")
    # Kernel arithmetic is fp32-accumulated regardless of autocast.
    with torch.autocast(q.device.type, enabled=False):
        return dense_hip(q, k, v, positions, block_size)
