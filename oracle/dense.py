"""Gated dense block attention: CPU restatement (test infrastructure only).

Semantics (reference ``st/ops/attention.py:1-4,17-30``,
``st/ops/kernels/dense.py:32-86``, ``docs/ARCHITECTURE.md:20-26``), for one
(batch, query row, head) with absolute key position ``p`` and block size ``b``:

* ``a_i = q.k_i / sqrt(D)``;
* remote keys ``R = {i : i//b < p//b - 1}``, local keys
  ``L = {i : i//b >= p//b - 1 and i <= p}``;
* block score ``s_j = logsumexp_{i in block j} a_i``, ``log Z_R =
  logsumexp_{i in R} a_i``;
* logits ``a_i`` on L and ``a_i + s_{i//b} - log Z_R`` on R, softmax over
  L u R, output ``sum softmax * v``; a padding row (``p < 0``) gives 0.

Four forms are given: a per-row loop (``loop_attention``), the vectorised
Q x N algebra with autograd (``eager_attention``), the statistics the fused
forward saves plus the explicit backward formulas (``forward_stats`` /
``backward_explicit``), and the reference's bounded-memory chunked form
(``chunked_forward`` / ``chunked_backward`` / ``chunked_attention``).
"""
import math

import torch
import torch.nn.functional as F


def work_dtype(t):
    """float64 stays float64, everything else computes in float32
    (reference ``st/ops/attention.py:13-14``)."""
    return torch.float64 if t.dtype == torch.float64 else torch.float32


def _heads(t, dtype):
    return t.transpose(1, 2).to(dtype)


def _scores(q, k, dtype):
    """``a = q k^T / sqrt(D)`` as ``[B,H,Q,N]`` (``st/ops/attention.py:19``)."""
    return _heads(q, dtype) @ _heads(k, dtype).transpose(-1, -2) / math.sqrt(q.shape[-1])


def _block_lse(a, b):
    """Per-block logsumexp broadcast back to keys, tail padded with -inf
    (``st/ops/attention.py:28-29``, ``st/ops/kernels/dense.py:12-19``)."""
    n = a.shape[-1]
    groups = -(-n // b)
    padded = F.pad(a, (0, groups * b - n), value=-math.inf)
    s = padded.reshape(*a.shape[:-1], groups, b).logsumexp(-1)
    return s, s.repeat_interleave(b, -1)[..., :n]


def masks(positions, n, b):
    """Remote / local key masks ``[B,1,Q,N]`` (``st/ops/attention.py:21-27``,
    ``st/ops/kernels/dense.py:58-60``)."""
    pos = positions[:, None, :, None]
    t = torch.arange(n, device=positions.device)
    group = (t // b)[None, None, None, :]
    valid = pos >= 0
    remote = (group < torch.div(pos, b, rounding_mode="floor") - 1) & valid
    local = ((group >= torch.div(pos, b, rounding_mode="floor") - 1)
             & (t[None, None, None, :] <= pos) & valid)
    return remote, local


def loop_attention(q, k, v, positions, block_size, topk=None):
    """Brute force, one row at a time (shape of the reference's loop oracle
    ``tests/test_attention.py:11-44``). With ``topk`` only the ``topk``
    highest-scoring remote blocks are read, still gated by the full ``Z_R``
    (``st/ops/sparse.py:132-134``). Differentiable; intended for tiny inputs."""
    batch, nq, heads, dim = q.shape
    b = block_size
    rows = []
    for bi in range(batch):
        per_query = []
        for t in range(nq):
            p = int(positions[bi, t])
            per_head = []
            for h in range(heads):
                if p < 0:
                    per_head.append(torch.zeros(dim, dtype=q.dtype, device=q.device)
                                    + 0 * q[bi, t, h])
                    continue
                a = k[bi, :p + 1, h] @ q[bi, t, h] / math.sqrt(dim)
                n_remote = max(0, p // b - 1)
                lo = n_remote * b
                logits = [a[lo:p + 1]]
                values = [v[bi, lo:p + 1, h]]
                if n_remote:
                    s = a[:lo].reshape(n_remote, b).logsumexp(-1)
                    log_zr = s.logsumexp(0)
                    chosen = range(n_remote)
                    if topk is not None and topk < n_remote:
                        chosen = s.topk(topk).indices.tolist()
                    for j in chosen:
                        logits.append(a[j * b:(j + 1) * b] + s[j] - log_zr)
                        values.append(v[bi, j * b:(j + 1) * b, h])
                weights = torch.cat(logits).softmax(0)
                per_head.append(weights @ torch.cat(values))
            per_query.append(torch.stack(per_head))
        rows.append(torch.stack(per_query))
    return torch.stack(rows)


def eager_attention(q, k, v, positions, block_size):
    """Vectorised Q x N algebra with autograd (``st/tools/benchmark.py:27-43``).

    The reference's eager form leaves a padding row as 0/0; here such a row
    is 0, matching the fused operator (``st/ops/kernels/dense.py:43,58-60``).
    Returns ``[B,Q,H,D]`` in ``q.dtype``.
    """
    dtype = work_dtype(q)
    n, b = k.shape[1], block_size
    a = _scores(q, k, dtype)
    s, _ = _block_lse(a, b)
    pos = positions[:, None, :, None]
    blocks = torch.arange(s.shape[-1], device=q.device)[None, None, None, :]
    visible = (blocks < torch.div(pos, b, rounding_mode="floor") - 1) & (pos >= 0)
    s = s.masked_fill(~visible, -math.inf)
    has_remote = visible.any(-1, keepdim=True)
    safe_s = torch.where(has_remote, s, torch.zeros_like(s))
    gate = (safe_s - safe_s.logsumexp(-1, keepdim=True)).masked_fill(~visible, 0.)
    bias = gate.repeat_interleave(b, -1)[..., :n]
    causal = torch.arange(n, device=q.device)[None, None, None, :] <= pos
    row_valid = pos >= 0
    logits = torch.where(causal, a + bias, torch.full_like(a, -math.inf))
    logits = torch.where(row_valid, logits, torch.zeros_like(logits))
    out = logits.softmax(-1) @ _heads(v, dtype)
    out = torch.where(row_valid, out, torch.zeros_like(out))
    return out.transpose(1, 2).to(q.dtype)


def forward_stats(q, k, v, positions, block_size):
    """Output plus the statistics the fused forward saves for backward
    (``st/ops/attention.py:52-93``, ``st/ops/kernels/dense.py:61-86``):

    ``out`` (q.dtype), ``rc`` remote part of the output, ``pr`` remote
    probability mass, ``zr = log Z_R`` and ``z = logsumexp`` of all logits,
    with ``-inf`` for ``zr`` when no remote block exists and for both when the
    row is padding. All but ``out`` are in the work dtype.
    """
    dtype = work_dtype(q)
    n, b = k.shape[1], block_size
    a = _scores(q, k, dtype)
    _, sb = _block_lse(a, b)
    remote, local = masks(positions, n, b)
    ninf = torch.full_like(a, -math.inf)
    zr = torch.where(remote, a, ninf).logsumexp(-1)
    zr_safe = torch.where(torch.isfinite(zr), zr, torch.zeros_like(zr))
    remote_logit = torch.where(remote, a + sb - zr_safe[..., None], ninf)
    local_logit = torch.where(local, a, ninf)
    lr, ll = remote_logit.logsumexp(-1), local_logit.logsumexp(-1)
    total = torch.logaddexp(lr, ll)
    safe_total = torch.where(torch.isfinite(total), total, torch.zeros_like(total))
    vh = _heads(v, dtype)
    rc = torch.exp(remote_logit - safe_total[..., None]) @ vh
    lc = torch.exp(local_logit - safe_total[..., None]) @ vh
    pr = torch.exp(lr - safe_total)
    out = (rc + lc).transpose(1, 2).to(q.dtype)
    flip = lambda t: t.transpose(1, 2).contiguous()
    return out, flip(rc), flip(pr), flip(zr), flip(total)


def backward_explicit(q, k, v, positions, block_size, grad_out, saved=None):
    """Input gradients from the closed-form derivative, including both gate
    terms (``st/ops/attention.py:105-139``, ``st/ops/kernels/dense.py:89-120``):

    ``delta = dO.O``, ``rho = dO.RC - delta*PR``, ``P = exp(logit - Z)``,
    ``direct = P (dO.v - delta)``, ``g_j = sum_{i in j} direct_i``,
    ``gate_i = exp(a_i - s_j) g_j - exp(a_i - log Z_R) rho`` on R,
    ``dA = (direct + [R] gate) / sqrt(D)``; ``dQ = dA K``, ``dK = dA^T Q``,
    ``dV = P^T dO``. Returns ``(dq, dk, dv)`` in the input dtypes.
    """
    dtype = work_dtype(q)
    n, b = k.shape[1], block_size
    if saved is None:
        saved = forward_stats(q, k, v, positions, block_size)
    out, rc, pr, zr, z = saved
    go = _heads(grad_out, dtype)
    delta = (go * _heads(out, dtype)).sum(-1)
    rho = (go * _heads(rc, dtype)).sum(-1) - delta * pr.transpose(1, 2)
    zr = zr.transpose(1, 2)
    z = z.transpose(1, 2)
    zr = torch.where(torch.isfinite(zr), zr, torch.zeros_like(zr))
    z = torch.where(torch.isfinite(z), z, torch.zeros_like(z))
    a = _scores(q, k, dtype)
    _, sb = _block_lse(a, b)
    remote, local = masks(positions, n, b)
    probs = torch.exp(torch.where(remote, a + sb - zr[..., None], a) - z[..., None])
    probs = torch.where(remote | local, probs, torch.zeros_like(probs))
    kh, vh, qh = _heads(k, dtype), _heads(v, dtype), _heads(q, dtype)
    direct = probs * (go @ vh.transpose(-1, -2) - delta[..., None])
    groups = -(-n // b)
    padded = F.pad(direct, (0, groups * b - n))
    block_grad = padded.reshape(*direct.shape[:-1], groups, b).sum(-1)
    block_grad = block_grad.repeat_interleave(b, -1)[..., :n]
    gate = torch.exp(a - sb) * block_grad - torch.exp(a - zr[..., None]) * rho[..., None]
    da = (direct + torch.where(remote, gate, torch.zeros_like(gate))) / math.sqrt(q.shape[-1])
    dq = (da @ kh).transpose(1, 2).to(q.dtype)
    dk = (da.transpose(-1, -2) @ qh).transpose(1, 2).to(k.dtype)
    dv = (probs.transpose(-1, -2) @ go).transpose(1, 2).to(v.dtype)
    return dq, dk, dv


class _Running:
    """Softmax over key tiles seen one at a time: running maximum ``m``,
    denominator ``den`` and weighted value sum ``num`` (the online merge of
    ``st/ops/attention.py:43-48``). All-masked rows keep ``m = -inf``."""

    def __init__(self, rows, dim, dtype):
        self.m = torch.full(rows, -math.inf, dtype=dtype)
        self.den = torch.zeros(rows, dtype=dtype)
        self.num = torch.zeros(*rows, dim, dtype=dtype)

    def add(self, logits, values):
        m = torch.maximum(self.m, logits.amax(-1))
        ref = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
        carry = torch.exp(self.m - ref)
        w = torch.exp(logits - ref[..., None])
        self.den = self.den * carry + w.sum(-1)
        self.num = self.num * carry[..., None] + w @ values
        self.m = m

    def log_mass(self):
        """log of the softmax mass, log(den) + m (-inf when nothing was seen)."""
        return self.m + self.den.log()

    def mean(self, dtype):
        return self.num / self.den.clamp_min(torch.finfo(dtype).tiny)[..., None]


def _kv_step(kv_chunk, b):
    """Key tile length: a positive multiple of the block size, so every
    block's logsumexp stays inside one tile (``st/ops/attention.py:60``)."""
    return max(b, kv_chunk // b * b)


def _tile_terms(qh, kh, pos, start, n, b):
    """Scores of one (query chunk, key tile) pair and its masks.

    ``qh`` ``[B,H,q,D]`` and ``kh`` ``[B,H,t,D]`` hold keys ``[start,
    start + t)``, ``start`` a multiple of ``b``. Returns ``a``, the per-key
    block logsumexp ``sb`` (a partial last block sums its real keys only),
    and the remote / local masks of ``st/ops/attention.py:17-30``."""
    a = qh @ kh.transpose(-1, -2) / math.sqrt(qh.shape[-1])
    _, sb = _block_lse(a, b)
    t = torch.arange(start, start + kh.shape[-2])
    grp = (t // b)[None, None, None, :]
    p = pos[:, None, :, None]
    own = torch.div(p, b, rounding_mode="floor")
    live = p >= 0
    remote = (grp < own - 1) & live
    local = (grp >= own - 1) & (t[None, None, None, :] <= p) & live & (t[None, None, None, :] < n)
    return a, sb, remote, local


def chunked_forward(q, k, v, positions, block_size, q_chunk=32, kv_chunk=1024):
    """The reference's bounded-memory forward (``st/ops/attention.py:51-93``):
    query chunks of ``q_chunk`` rows against key tiles of ``kv_chunk`` keys
    (rounded down to a multiple of the block size), never holding more than
    one ``q_chunk x kv_chunk`` score tile.

    Per chunk, three running states are kept across key tiles: ``log Z_R``
    (logaddexp of each tile's remote logsumexp), the remote softmax over
    ``a + s_j`` and the local softmax over ``a``; ``log Z_R`` is subtracted
    from the remote log-mass only at the end, where the two parts are
    combined. Returns the five tensors of ``forward_stats``."""
    dtype = work_dtype(q)
    batch, nq, heads, dim = q.shape
    n, b = k.shape[1], block_size
    step = _kv_step(kv_chunk, b)
    out = torch.empty_like(q)
    rc = torch.empty(q.shape, dtype=dtype)
    pr, zr_all, z_all = (torch.empty(batch, nq, heads, dtype=dtype) for _ in range(3))
    for lo in range(0, nq, q_chunk):
        hi = min(lo + q_chunk, nq)
        qh = _heads(q[:, lo:hi], dtype)
        pos = positions[:, lo:hi]
        rows = qh.shape[:-1]
        zr = torch.full(rows, -math.inf, dtype=dtype)
        far, near = _Running(rows, dim, dtype), _Running(rows, dim, dtype)
        for start in range(0, n, step):
            end = min(start + step, n)
            kh, vh = _heads(k[:, start:end], dtype), _heads(v[:, start:end], dtype)
            a, sb, remote, local = _tile_terms(qh, kh, pos, start, n, b)
            ninf = torch.full_like(a, -math.inf)
            zr = torch.logaddexp(zr, torch.where(remote, a, ninf).logsumexp(-1))
            far.add(torch.where(remote, a + sb, ninf), vh)
            near.add(torch.where(local, a, ninf), vh)
        zr_safe = torch.where(torch.isfinite(zr), zr, torch.zeros_like(zr))
        lr = far.log_mass() - zr_safe
        ll = near.log_mass()
        total = torch.logaddexp(lr, ll)
        safe_total = torch.where(torch.isfinite(total), total, torch.zeros_like(total))
        p_far = torch.exp(lr - safe_total)
        rc_c = far.mean(dtype) * p_far[..., None]
        lc_c = near.mean(dtype) * torch.exp(ll - safe_total)[..., None]
        out[:, lo:hi] = (rc_c + lc_c).transpose(1, 2).to(q.dtype)
        rc[:, lo:hi] = rc_c.transpose(1, 2)
        pr[:, lo:hi] = p_far.transpose(1, 2)
        zr_all[:, lo:hi] = zr.transpose(1, 2)
        z_all[:, lo:hi] = total.transpose(1, 2)
    return out, rc, pr, zr_all, z_all


def chunked_backward(q, k, v, positions, block_size, grad_out, saved, q_chunk=32, kv_chunk=1024):
    """The reference's bounded-memory backward (``st/ops/attention.py:104-139``):
    the closed form of ``backward_explicit`` evaluated one (query chunk, key
    tile) pair at a time from the saved statistics, accumulating ``dq`` over
    tiles and ``dk``/``dv`` over chunks. Block sums of ``direct`` stay inside
    a tile because tiles are block aligned. Returns ``(dq, dk, dv)``."""
    dtype = work_dtype(q)
    n, b = k.shape[1], block_size
    step = _kv_step(kv_chunk, b)
    out, rc, pr, zr_all, z_all = saved
    scale = math.sqrt(q.shape[-1])
    dq = torch.zeros(q.shape, dtype=dtype)
    dk = torch.zeros(k.shape, dtype=dtype)
    dv = torch.zeros(v.shape, dtype=dtype)
    finite = lambda t: torch.where(torch.isfinite(t), t, torch.zeros_like(t))
    for lo in range(0, q.shape[1], q_chunk):
        hi = min(lo + q_chunk, q.shape[1])
        qh = _heads(q[:, lo:hi], dtype)
        go = _heads(grad_out[:, lo:hi], dtype)
        delta = (go * _heads(out[:, lo:hi], dtype)).sum(-1)
        rho = (go * _heads(rc[:, lo:hi], dtype)).sum(-1) - delta * pr[:, lo:hi].transpose(1, 2)
        zr = finite(zr_all[:, lo:hi].transpose(1, 2))[..., None]
        z = finite(z_all[:, lo:hi].transpose(1, 2))[..., None]
        pos = positions[:, lo:hi]
        for start in range(0, n, step):
            end = min(start + step, n)
            kh, vh = _heads(k[:, start:end], dtype), _heads(v[:, start:end], dtype)
            a, sb, remote, local = _tile_terms(qh, kh, pos, start, n, b)
            probs = torch.exp(torch.where(remote, a + sb - zr, a) - z)
            probs = torch.where(remote | local, probs, torch.zeros_like(probs))
            direct = probs * (go @ vh.transpose(-1, -2) - delta[..., None])
            t = direct.shape[-1]
            sums = F.pad(direct, (0, -t % b)).reshape(*direct.shape[:-1], -1, b).sum(-1)
            block_grad = sums.repeat_interleave(b, -1)[..., :t]
            gate = torch.exp(a - sb) * block_grad - torch.exp(a - zr) * rho[..., None]
            da = (direct + torch.where(remote, gate, torch.zeros_like(gate))) / scale
            dq[:, lo:hi] += (da @ kh).transpose(1, 2)
            dk[:, start:end] += (da.transpose(-1, -2) @ qh).transpose(1, 2)
            dv[:, start:end] += (probs.transpose(-1, -2) @ go).transpose(1, 2)
    return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype)


class ChunkedDense(torch.autograd.Function):
    """``chunked_forward`` / ``chunked_backward`` as one autograd node, the
    reference's ``_TorchDense`` (``st/ops/attention.py:96-139``): only the
    per-row statistics are saved, never a Q x N tensor."""

    @staticmethod
    def forward(ctx, q, k, v, positions, block_size, q_chunk, kv_chunk):
        saved = chunked_forward(q, k, v, positions, block_size, q_chunk, kv_chunk)
        ctx.save_for_backward(q, k, v, positions, *saved)
        ctx.tiles = (block_size, q_chunk, kv_chunk)
        return saved[0]

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad):
        q, k, v, positions, *saved = ctx.saved_tensors
        b, q_chunk, kv_chunk = ctx.tiles
        dq, dk, dv = chunked_backward(q, k, v, positions, b, grad, saved, q_chunk, kv_chunk)
        return dq, dk, dv, None, None, None, None


def chunked_attention(q, k, v, positions, block_size, q_chunk=32, kv_chunk=1024):
    """``dense_attention(backend="torch")`` (``st/ops/attention.py:148,174-176``):
    the chunked form, outside autocast, on CPU tensors."""
    with torch.autocast("cpu", enabled=False):
        return ChunkedDense.apply(q, k, v, positions, block_size, q_chunk, kv_chunk)


def dense_flops(batch, heads, dim, positions, n_keys):
    """Algorithmic FLOP of one forward+backward: 2 matmuls forward and 5
    backward over the causal prefix of every row, ``14 B H D sum(p+1)``
    (recompute excluded). ``positions`` is ``[B,Q]``."""
    lengths = (positions.clamp(max=n_keys - 1) + 1).clamp(min=0)
    return 14 * heads * dim * int(lengths.sum())
