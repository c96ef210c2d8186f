"""st_sparse_fwd_noalloc (workspace in a file-scope device array) against
st_sparse_fwd (caller workspace), called through the C ABI: two calls in a
row on one GPU, the second smaller, each compared bit-exactly with the
workspace entry point. (Its host-side size check runs in tests/test_abi.py.)"""
import pytest
import torch

from exploration_amd import _lib

pytestmark = pytest.mark.gpu


def _inputs(device, seed, batch, queries, heads, dim, n, dtype=torch.bfloat16):
    g = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(batch, queries, heads, dim, generator=g, device=device).to(dtype)
    k = torch.randn(batch, n, heads, dim, generator=g, device=device).to(dtype)
    v = torch.randn(batch, n, heads, dim, generator=g, device=device).to(dtype)
    pos = torch.randint(0, n, (batch, queries), generator=g, device=device)
    pos[:, 0] = n - 1
    return q, k, v, pos


def _run(lib, noalloc, q, k, v, pos, b, topk):
    batch, queries, heads, dim = q.shape
    n = k.shape[1]
    out = torch.empty_like(q)
    ids = torch.empty((batch, queries, heads, topk), device=q.device, dtype=torch.int64)
    top = torch.empty((batch, queries, heads, topk), device=q.device, dtype=torch.float32)
    zr = torch.empty((batch, queries, heads), device=q.device, dtype=torch.float32)
    lse = torch.empty_like(zr)
    common = [_lib.DTYPE_CODES[q.dtype], batch, queries, heads, dim, b, topk, _lib.ptr(q), _lib.ptr(pos),
              _lib.ptr(k), _lib.ptr(v), None, b, 0, n, 0, _lib.ptr(out), _lib.ptr(ids), _lib.ptr(top),
              _lib.ptr(zr), _lib.ptr(lse)]
    if noalloc:
        status = lib.st_sparse_fwd_noalloc(*common, _lib.stream_of(q))
    else:
        need = lib.st_sparse_workspace_bytes(batch, queries, heads, dim, topk, -(-n // b))
        ws = torch.empty(need, device=q.device, dtype=torch.uint8)
        status = lib.st_sparse_fwd(*common, _lib.ptr(ws), need, _lib.stream_of(q))
    _lib.check(status, lib)
    torch.cuda.synchronize()
    return out, ids, top, zr, lse


def test_noalloc_matches_workspace_entry_point(device):
    lib = _lib.load()
    assert lib.st_sparse_noalloc_scratch_bytes() == 16 << 20
    # first call: the cfg5 decode shape (16 tail-ish queries, H16 D64 b16,
    # 131,072 tokens, top-64: 9.2 MiB of scratch); second call smaller
    for label, (seed, batch, queries, heads, dim, n, b, topk) in (
            ("cfg5-decode", (1, 1, 16, 16, 64, 131072, 16, 64)),
            ("small", (2, 2, 6, 8, 128, 20000, 128, 8))):
        print(f"noalloc {label}", flush=True)
        q, k, v, pos = _inputs(device, seed, batch, queries, heads, dim, n)
        want = _run(lib, False, q, k, v, pos, b, topk)
        got = _run(lib, True, q, k, v, pos, b, topk)
        for name, a, e in zip(("out", "ids", "scores", "log_zr", "lse"), got, want):
            assert torch.equal(a, e), f"{label}: {name} differs"
