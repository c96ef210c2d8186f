"""Paged sparse top-k forward: HIP kernels against the oracle.

Cases: the reference's CPU sparse test (tests/test_attention.py:75-86: seed
124, b=4, keep in {1, 2, 64}, several page sizes), its GPU sparse/score
cases (st/tools/validate.py:119-136: keep=2, pages of 4b, score offset 2b),
exact-tie selection, and cfg4 at full size (1M tokens in 128-token pages
behind a random page table, 64 planted blocks per query). Selected ids are
compared bit-exactly wherever the oracle's score margin rules out float
reordering; the margin is asserted first.
"""
import math

import pytest
import torch

from exploration_amd import PagedKV, TensorPages, block_scores, select_blocks, sparse_attention, sparse_pop
from exploration_amd.workloads import CFG4, plant_blocks, planted_sparse
from oracle import dense as od
from oracle import sparse as osp
from tests.helpers import assert_close, error_metrics

pytestmark = pytest.mark.gpu


def _row_margins(scores, topk):
    """Per row: the smallest gap between consecutive sorted finite scores
    among the top topk+1 (inf when fewer are finite)."""
    top = torch.sort(scores, -1, descending=True).values[..., :topk + 1]
    gaps = top[..., :-1] - top[..., 1:]
    gaps = torch.where(torch.isfinite(gaps), gaps, torch.full_like(gaps, math.inf))
    return gaps.min(-1).values if gaps.shape[-1] else torch.full(scores.shape[:-1], math.inf)


def _margin(scores, topk):
    """Smallest row margin of the whole tensor."""
    return float(_row_margins(scores, topk).min())


def _assert_decided_ids(got, ref_scores, topk, min_rows, label):
    """Selected ids equal the oracle's on every row whose top-(k+1) order is
    decided by more than float reordering noise (margin > 1e-3); at least
    min_rows rows must be decided, so the comparison is never empty."""
    _, ids, _ = osp.select_topk(ref_scores, topk)
    ok = _row_margins(ref_scores, topk) > 1e-3
    print(f"  {label}: {int(ok.sum())}/{ok.numel()} rows with a decided top-{topk}", flush=True)
    assert int(ok.sum()) >= min_rows, f"{label}: only {int(ok.sum())} decided rows"
    assert torch.equal(got.cpu()[ok], ids[ok])


@pytest.mark.parametrize("keep", [1, 2, 64])
@pytest.mark.parametrize("kind", ["tensor_pages", "paged"])
def test_reference_sparse_case(device, keep, kind):
    print(f"sparse reference case keep={keep} {kind}", flush=True)
    g = torch.Generator().manual_seed(124)
    q = torch.randn(2, 4, 3, 8, generator=g, dtype=torch.float64)
    k = torch.randn(2, 45, 3, 8, generator=g, dtype=torch.float64)
    v = torch.randn(2, 45, 3, 8, generator=g, dtype=torch.float64)
    pos = torch.tensor([[0, 7, 44, 22], [13, 44, 1, 43]])
    expected = od.loop_attention(q, k, v, pos, 4, keep)
    qf, kf, vf = (t.float().to(device) for t in (q, k, v))
    for page in (4, 12, 64):
        if kind == "tensor_pages":
            cache = TensorPages(kf, vf, page)
        else:
            table = torch.randperm(2 * (-(-45 // page)), generator=g).reshape(2, -1)
            cache = PagedKV.from_dense(kf, vf, page, table.to(device))
        out, sel = sparse_attention(qf, cache, pos.to(device), 4, keep, return_selection=True)
        assert_close(out, expected, torch.float32, f"keep={keep} page={page}")
        _, ids, zr = osp.select_topk(osp.block_scores(q, k, pos, 4), keep)
        assert torch.equal(sel["indices"].cpu(), ids)
        assert_close(sel["log_zr"], zr, torch.float32, "log_zr")


VALIDATE_CASES = [(17, 2, 16), (129, 16, 32), (257, 32, 64), (193, 64, 96), (385, 128, 128),
                  (131, 16, 256), (385, 128, 256)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
@pytest.mark.parametrize("n,b,d", VALIDATE_CASES)
def test_validation_matrix(device, n, b, d, dtype):
    """st/tools/validate.py:119-136: block scores of a slab at offset 2b, and
    sparse keep=2 over pages of 4b against the loop oracle."""
    print(f"sparse case n={n} b={b} d={d} {dtype}", flush=True)
    g = torch.Generator().manual_seed(772)
    q = torch.randn(2, 5, 2, d, generator=g).to(dtype)
    k = torch.randn(2, n, 2, d, generator=g).to(dtype)
    v = torch.randn(2, n, 2, d, generator=g).to(dtype)
    pos = torch.tensor([[0, b - 1, min(2 * b + 1, n - 1), n - 1, -1], [n - 1, 0, n // 2, -1, n - 2]])
    qd, kd, vd = (t.double() for t in (q, k, v))
    offset = 2 * b
    shifted = torch.where(pos >= 0, pos + offset, pos)
    s = block_scores(q.to(device), k.to(device), shifted.to(device), b, offset)
    assert_close(s, osp.block_scores(qd, kd, shifted, b, offset), torch.float32, "scores")
    keep = 2
    expected = od.loop_attention(qd, kd, vd, pos, b, keep)
    out, sel = sparse_attention(q.to(device), TensorPages(k.to(device), v.to(device), 4 * b), pos.to(device),
                                b, keep, score_page_tokens=2 * b, return_selection=True)
    print(f"  errors {error_metrics(out, expected)}", flush=True)
    assert_close(out, expected, dtype, "sparse out")
    ref_scores = osp.block_scores(qd, kd, pos, b)
    _assert_decided_ids(sel["indices"], ref_scores, keep, 8, f"n={n} b={b} d={d}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
@pytest.mark.parametrize("d", [20, 33, 130])
def test_head_dim_not_multiple_of_8(device, d, dtype):
    """Head dimensions that are not a multiple of 8 (the reference accepts
    any D <= 256, st/ops/attention.py:142-145): block scores and the sparse
    read with element loads, against the oracle."""
    print(f"sparse head_dim {d} {dtype}", flush=True)
    g = torch.Generator().manual_seed(90 + d)
    n, b = 200, 16
    q = torch.randn(2, 5, 2, d, generator=g).to(dtype)
    k = torch.randn(2, n, 2, d, generator=g).to(dtype)
    v = torch.randn(2, n, 2, d, generator=g).to(dtype)
    pos = torch.tensor([[199, 150, 40, 17, -1], [120, 199, 3, 64, 190]])
    qd, kd, vd = (t.double() for t in (q, k, v))
    s = block_scores(q.to(device), k.to(device), pos.to(device), b)
    assert_close(s, osp.block_scores(qd, kd, pos, b), torch.float32, "scores")
    expected = od.loop_attention(qd, kd, vd, pos, b, 3)
    for cache in (TensorPages(k.to(device), v.to(device), 4 * b),
                  PagedKV.from_dense(k.to(device), v.to(device), 2 * b)):
        out, sel = sparse_attention(q.to(device), cache, pos.to(device), b, 3, return_selection=True)
        assert_close(out, expected, dtype, "sparse out")
        _assert_decided_ids(sel["indices"], osp.block_scores(qd, kd, pos, b), 3, 8, f"d={d}")


@pytest.mark.parametrize("tier", ["pinned", "pageable"])
def test_host_resident_tensor_pages(device, tier):
    """A TensorPages (or the reference's KVCache) whose k/v live in host
    memory goes straight to sparse_attention, as the reference's CPU and
    disk tiers do (st/ops/sparse.py:81-96,126): the same selection and output
    as the device-resident cache."""
    print(f"sparse host-resident TensorPages ({tier})", flush=True)
    g = torch.Generator().manual_seed(31)
    n, h, d, b = 5000, 4, 64, 16
    q = torch.randn(1, 6, h, d, generator=g).to(torch.bfloat16)
    k = torch.randn(1, n, h, d, generator=g).to(torch.bfloat16)
    v = torch.randn(1, n, h, d, generator=g).to(torch.bfloat16)
    if tier == "pinned":
        k, v = k.pin_memory(), v.pin_memory()
    pos = torch.tensor([[4999, 4000, 2500, 1234, 300, 40]])
    want, wsel = sparse_attention(q.to(device), TensorPages(k.to(device), v.to(device), 1024), pos.to(device), b,
                                  8, score_page_tokens=1024, return_selection=True)
    got, sel = sparse_attention(q.to(device), TensorPages(k, v, 1024), pos.to(device), b, 8,
                                score_page_tokens=1024, return_selection=True)
    assert torch.equal(sel["indices"], wsel["indices"])
    assert torch.equal(sel["scores"], wsel["scores"])
    assert_close(got, want, torch.bfloat16, "host tier out")
    expected = od.loop_attention(q.double(), k.double(), v.double(), pos, b, 8)
    assert_close(got, expected, torch.bfloat16, "host tier vs oracle")


def test_select_exact_ties_and_short_rows(device):
    """Ties are broken by ascending block id; rows with fewer finite scores
    than topk pad with -1/-inf; log Z_R is the row logsumexp."""
    print("sparse select ties", flush=True)
    g = torch.Generator().manual_seed(3)
    rows, n = 37, 3000
    s = torch.randint(0, 20, (rows, n), generator=g).float() / 4  # many exact ties
    s[5, 100:] = -math.inf
    s[6] = -math.inf
    s[7, :10] = torch.tensor([3.0, 1, 3, 3, 2, 3, 0, 3, 3, 3])
    s[7, 10:] = -math.inf
    for topk in (1, 8, 64, 200):
        values, ids, zr = select_blocks(s.to(device), topk, id_base=0)
        ev, ei, ez = osp.select_topk(s, topk)
        assert torch.equal(ids.cpu(), ei), topk
        assert torch.equal(values.cpu(), ev), topk
        assert_close(zr, ez, torch.float32, "log_zr")
    _, ids, _ = select_blocks(s[7:8].to(device), 8, id_base=1000)
    assert ids.tolist() == [[1000, 1002, 1003, 1005, 1007, 1008, 1009, 1004]]


@pytest.mark.parametrize("n", [1, 40, 64, 65, 4097, 8192, 8193, 16384, 16385])
def test_select_row_lengths(device, n):
    """Every selection kernel size class (up to 8192 and 16384 blocks per
    row in registers, longer rows streamed), rows shorter than topk, exact
    ties at the cut, all -inf rows, and continuous scores."""
    print(f"sparse select n={n}", flush=True)
    g = torch.Generator().manual_seed(n)
    rows = 6
    s = torch.randn(rows, n, generator=g) * 3
    s[1] = torch.randint(0, 6, (n,), generator=g).float()  # ties straddle every cut
    s[2] = 2.5
    s[3] = -math.inf
    s[4, ::3] = -math.inf
    s[5] = torch.randint(-3, 3, (n,), generator=g).float() * 1e30
    for topk in (1, 17, 64):
        values, ids, zr = select_blocks(s.to(device), topk, id_base=7)
        ev, ei, ez = osp.select_topk(s, topk)
        ei = torch.where(ei >= 0, ei + 7, ei)
        assert torch.equal(ids.cpu(), ei), (n, topk)
        assert torch.equal(values.cpu(), ev), (n, topk)
        assert_close(zr, ez, torch.float32, "log_zr")


def test_pop_with_given_selection(device):
    """sparse_pop on a caller-supplied selection (including -1 slots)."""
    print("sparse pop", flush=True)
    g = torch.Generator().manual_seed(9)
    q = torch.randn(1, 6, 2, 64, generator=g)
    k = torch.randn(1, 300, 2, 64, generator=g)
    v = torch.randn(1, 300, 2, 64, generator=g)
    pos = torch.tensor([[299, 250, 130, 17, 64, -1]])
    s = osp.block_scores(q.double(), k.double(), pos, 16)
    values, ids, zr = osp.select_topk(s, 5)
    ids[0, 1, 0, 4] = -1
    values[0, 1, 0, 4] = -math.inf
    out_e, lse_e = osp.pop(q.double(), k.double(), v.double(), pos, ids, values, zr, 16)
    out, lse = sparse_pop(q.to(device), k.to(device), v.to(device), pos.to(device), ids.to(device),
                          values.float().to(device), zr.float().to(device), 16)
    assert_close(out, out_e, torch.float32, "pop out")
    assert_close(lse, lse_e, torch.float32, "pop lse")


def test_cfg5_decode_shape(device):
    """cfg5 tail shape: 16 tail queries over 131,072 tokens, H16 D64 b16,
    top-64, bf16, contiguous cache (oracle in float32 on the GPU)."""
    print("sparse cfg5 decode", flush=True)
    gen = torch.Generator(device=device).manual_seed(11)
    n, h, d, b = 131072, 16, 64, 16
    q = torch.randn(1, 16, h, d, generator=gen, device=device).to(torch.bfloat16)
    k = torch.randn(1, n, h, d, generator=gen, device=device).to(torch.bfloat16)
    v = torch.randn(1, n, h, d, generator=gen, device=device).to(torch.bfloat16)
    pos = torch.arange(n - 16, n, device=device)[None]
    # random scores leave almost no row with a top-64 order decided beyond
    # float noise: plant 64 well-separated blocks for four of the queries
    # (every head), so that 64 rows pin the selection bit-exactly
    planted = (0, 5, 10, 15)
    expected = plant_blocks(q, k, pos, b, 64, planted, gen)
    out, sel = sparse_attention(q, TensorPages(k, v), pos, b, 64, return_selection=True)
    ref_s = osp.block_scores(q.float(), k.float(), pos, b)
    ev, ei, ez = osp.select_topk(ref_s, 64)
    assert_close(sel["log_zr"], ez, torch.float32, "log_zr")
    assert torch.equal(ei[:, list(planted)], expected)
    assert torch.equal(sel["indices"][:, list(planted)], expected)
    _assert_decided_ids(sel["indices"], ref_s.cpu(), 64, 64, "cfg5 decode")
    assert_close(sel["scores"], ev, torch.float32, "top scores")
    out_e, _ = osp.pop(q.float(), k.float(), v.float(), pos, sel["indices"], sel["scores"], sel["log_zr"], b)
    assert_close(out, out_e, torch.bfloat16, "out")


def test_cfg4_full_size(device):
    """cfg4: bf16 B1 H8, 1,048,576 tokens in 128-token pages behind a seeded
    random page table, 16 tail queries, D128, b128, top-64 with 64 planted
    blocks per query: ids bit-exact against the planted order and the
    oracle, scores/log Z_R/output within tolerance."""
    print("sparse cfg4", flush=True)
    c = dict(CFG4)
    q, (k, v), pos, expected = planted_sparse(**c, device=device, paged=False)
    gen = torch.Generator(device=device).manual_seed(1)
    pages = c["length"] // c["page_tokens"]
    table = torch.randperm(pages, generator=gen, device=device).reshape(1, pages)
    cache = PagedKV.from_dense(k, v, c["page_tokens"], table)
    out, sel = sparse_attention(q, cache, pos, c["block"], c["topk"], return_selection=True)
    torch.cuda.synchronize()
    ref_s = osp.block_scores(q.float(), k.float(), pos, c["block"])
    margin = _margin(ref_s, c["topk"])
    print(f"  oracle score margin {margin:.4f}", flush=True)
    assert margin > 1e-2
    ev, ei, ez = osp.select_topk(ref_s, c["topk"])
    assert torch.equal(ei, expected)
    assert torch.equal(sel["indices"], expected)
    assert_close(sel["scores"], ev, torch.float32, "top scores")
    assert_close(sel["log_zr"], ez, torch.float32, "log_zr")
    out_e, _ = osp.pop(q.float(), k.float(), v.float(), pos, ei, ev, ez, c["block"])
    print(f"  out errors {error_metrics(out, out_e)}", flush=True)
    assert_close(out, out_e, torch.bfloat16, "out")
    # the same cache read contiguously gives identical results
    out2, sel2 = sparse_attention(q, TensorPages(k, v), pos, c["block"], c["topk"], return_selection=True)
    assert torch.equal(sel2["indices"], sel["indices"])
    assert torch.equal(out2, out)
