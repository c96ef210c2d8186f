"""Pins the CPU oracle (oracle/) before anything is compared against it.

Each check is independent of the formula it checks: three separate
restatements must agree; autograd must pass finite differences; special
cases must reduce to textbook routines (SDPA, logsumexp, closed-form block
masses); and a planted mistake in a copy of the oracle must be caught.
Cases (shapes, seeds, positions) follow the reference's tests
(tests/test_attention.py:48-86, st/tools/validate.py:75-136).
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import dense as od
from oracle import sparse as osp

F64 = torch.float64


def _gen(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _rand(shape, g, dtype=F64, requires_grad=False):
    t = torch.randn(shape, generator=g, dtype=dtype)
    return t.requires_grad_(requires_grad)


@pytest.mark.parametrize("n,b", [(1, 2), (7, 3), (17, 4), (33, 8)])
def test_three_forms_agree_and_gradients_match(n, b):
    """tests/test_attention.py:48-63 cases: loop, eager and flash-statistics
    forms agree; explicit backward equals autograd of both."""
    g = _gen(981)
    q = _rand((2, 5, 2, 6), g, requires_grad=True)
    k = _rand((2, n, 2, 6), g, requires_grad=True)
    v = _rand((2, n, 2, 6), g, requires_grad=True)
    pos = torch.tensor([[0, min(3, n - 1), n - 1, -1, n // 2], [n - 1, -1, 0, n // 2, n - 1]])
    loop = od.loop_attention(q, k, v, pos, b)
    eager = od.eager_attention(q, k, v, pos, b)
    stats = od.forward_stats(q.detach(), k.detach(), v.detach(), pos, b)
    torch.testing.assert_close(eager, loop, atol=1e-11, rtol=1e-10)
    torch.testing.assert_close(stats[0], loop.detach(), atol=1e-11, rtol=1e-10)
    probe = _rand(loop.shape, g)
    gl = torch.autograd.grad((loop * probe).sum(), (q, k, v))
    ge = torch.autograd.grad((eager * probe).sum(), (q, k, v))
    gx = od.backward_explicit(q.detach(), k.detach(), v.detach(), pos, b, probe, stats)
    for a, e, x in zip(ge, gl, gx):
        torch.testing.assert_close(a, e, atol=1e-10, rtol=1e-9)
        torch.testing.assert_close(x, e, atol=1e-10, rtol=1e-9)


@pytest.mark.parametrize("n,b,q_chunk,kv_chunk", [
    (1, 2, 1, 1), (17, 4, 3, 8), (33, 8, 5, 13), (33, 8, 32, 1024), (70, 16, 2, 16), (70, 16, 7, 48)])
def test_chunked_form_matches_stats_and_explicit_backward(n, b, q_chunk, kv_chunk):
    """The bounded-memory form (st/ops/attention.py:51-139) at several tile
    sizes, including tiles smaller than a block (rounded up to one block),
    tiles that cut the ragged last block and padding rows: its five saved
    statistics equal forward_stats, its gradients equal backward_explicit and
    autograd through the loop form."""
    g = _gen(77 + n)
    q = _rand((2, 6, 3, 8), g, requires_grad=True)
    k = _rand((2, n, 3, 8), g, requires_grad=True)
    v = _rand((2, n, 3, 8), g, requires_grad=True)
    pos = torch.tensor([[n - 1, 0, -1, n // 2, min(2 * b, n - 1), n - 1],
                        [-1, n // 3, n - 1, 0, n - 1, max(0, n - b)]])
    ref = od.forward_stats(q.detach(), k.detach(), v.detach(), pos, b)
    got = od.chunked_forward(q.detach(), k.detach(), v.detach(), pos, b, q_chunk, kv_chunk)
    for name, x, e in zip(("out", "rc", "pr", "zr", "z"), got, ref):
        torch.testing.assert_close(x, e, atol=1e-12, rtol=1e-11, msg=name)
    probe = _rand(q.shape, g)
    out = od.chunked_attention(q, k, v, pos, b, q_chunk, kv_chunk)
    gc = torch.autograd.grad((out * probe).sum(), (q, k, v))
    gx = od.backward_explicit(q.detach(), k.detach(), v.detach(), pos, b, probe, ref)
    gl = torch.autograd.grad((od.loop_attention(q, k, v, pos, b) * probe).sum(), (q, k, v))
    for c, x, l in zip(gc, gx, gl):
        torch.testing.assert_close(c, x, atol=1e-11, rtol=1e-10)
        torch.testing.assert_close(c, l, atol=1e-10, rtol=1e-9)


def test_chunked_form_fp32_cfg1_tiles():
    """cfg1 shape (B2 H4 N=Q=512 D64 b64, fp32, arange positions) at the
    reference's default tiles q_chunk=32, kv_chunk=1024 and at kv_chunk=128
    (four key tiles per row): within fp32 rounding of the float64 eager form."""
    g = _gen(0)
    q, k, v, do = (torch.randn(2, 512, 4, 64, generator=g) for _ in range(4))
    pos = torch.arange(512).expand(2, 512)
    want = od.eager_attention(q.double(), k.double(), v.double(), pos, 64)
    qd, kd, vd = (t.double() for t in (q, k, v))
    saved = od.forward_stats(qd, kd, vd, pos, 64)
    dwant = od.backward_explicit(qd, kd, vd, pos, 64, do.double(), saved)
    for kv_chunk in (1024, 128):
        qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
        out = od.chunked_attention(qg, kg, vg, pos, 64, 32, kv_chunk)
        assert out.dtype == torch.float32
        torch.testing.assert_close(out.double(), want, atol=1e-5, rtol=1e-5)
        out.backward(do)
        for got, e in zip((qg.grad, kg.grad, vg.grad), dwant):
            torch.testing.assert_close(got.double(), e, atol=2e-5, rtol=1e-5)


def test_gate_gradient_finite_difference():
    """tests/test_attention.py:65-73 case, through both gate terms."""
    g = _gen(4)
    q = _rand((1, 2, 1, 4), g, requires_grad=True)
    k = _rand((1, 13, 1, 4), g, requires_grad=True)
    v = _rand((1, 13, 1, 4), g, requires_grad=True)
    pos = torch.tensor([[9, 12]])
    assert torch.autograd.gradcheck(lambda q, k, v: od.eager_attention(q, k, v, pos, 2), (q, k, v),
                                    eps=1e-6, atol=1e-5, rtol=1e-4)


def _sdpa_window(q, k, v, pos, b):
    """Plain softmax attention over keys [max(0, (p//b-1) b), p] via SDPA."""
    n = k.shape[1]
    t = torch.arange(n)
    lo = (torch.div(pos, b, rounding_mode="floor") - 1).clamp(min=0) * b
    mask = (t[None, None, :] <= pos[:, :, None]) & (t[None, None, :] >= lo[:, :, None])
    out = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                         attn_mask=mask[:, None])
    return out.transpose(1, 2)


@pytest.mark.parametrize("n,b", [(40, 32), (9, 16), (64, 64)])
def test_no_remote_block_is_causal_softmax(n, b):
    """With every p < 2b (or b >= N) no block is remote: plain causal
    softmax attention, as computed by torch SDPA."""
    g = _gen(11)
    q, k, v = _rand((2, 6, 3, 8), g), _rand((2, n, 3, 8), g), _rand((2, n, 3, 8), g)
    pos = torch.randint(0, min(n, 2 * b), (2, 6), generator=g)
    expected = _sdpa_window(q, k, v, pos, b)
    for fn in (od.eager_attention, od.loop_attention, lambda *a: od.forward_stats(*a)[0]):
        torch.testing.assert_close(fn(q, k, v, pos, b), expected, atol=1e-12, rtol=1e-10)


def test_window_only_equals_sdpa_with_remote_present():
    """Local-window special case: when every remote score is -inf-like
    (keys of remote blocks are huge negatives) the output is SDPA over the
    window."""
    g = _gen(12)
    n, b = 50, 8
    q = _rand((1, 4, 2, 8), g).abs() + 0.5
    k, v = _rand((1, n, 2, 8), g), _rand((1, n, 2, 8), g)
    pos = torch.tensor([[49, 40, 33, 47]])
    k[:, :24] = -80.0  # blocks 0..2: remote for every row, mass ~ exp(-hundreds)
    out = od.eager_attention(q, k, v, pos, b)
    lo = torch.div(pos, b, rounding_mode="floor") - 1
    assert (lo * b >= 24).all()
    # rows see remote blocks 0..lo-1; blocks >= 3 carry finite mass, so only
    # compare rows whose remote set is exactly the suppressed blocks
    rows = (lo == 3)[0]
    exp = _sdpa_window(q, k, v, pos, b)
    torch.testing.assert_close(out[:, rows], exp[:, rows], atol=1e-12, rtol=1e-10)


def test_padding_rows_are_zero():
    g = _gen(13)
    q, k, v = _rand((2, 3, 2, 8), g), _rand((2, 20, 2, 8), g), _rand((2, 20, 2, 8), g)
    pos = torch.tensor([[-1, 19, 5], [7, -1, -1]])
    for fn in (od.eager_attention, od.loop_attention):
        out = fn(q, k, v, pos, 4)
        assert torch.all(out[0, 0] == 0) and torch.all(out[1, 1:] == 0)
    out, rc, pr, zr, z = od.forward_stats(q, k, v, pos, 4)
    assert torch.all(out[0, 0] == 0) and torch.isinf(z[0, 0]).all() and torch.isinf(zr[0, 0]).all()


def _constant_block_case(seed=21):
    """Keys constant inside every block, so a_i = A_j for i in block j."""
    g = _gen(seed)
    b, nblk, dim = 4, 9, 8
    q = _rand((1, 1, 1, dim), g)
    kb = _rand((nblk, dim), g)
    k = kb.repeat_interleave(b, 0)[None, :, None, :]
    v = _rand((1, nblk * b, 1, dim), g)
    return q, k, v, b, nblk


def _closed_form_output(q, k, v, p, b):
    """O = (sum_{j remote} b e^{2A_j}/S * mean_j(v) + sum_{i local} e^{a_i} v_i)
           / (sum_{j remote} b e^{2A_j}/S + sum_{i local} e^{a_i}),
    S = sum_{j remote} e^{A_j}: each remote block carries mass M_j^2 / Z_R with
    M_j = b e^{A_j}, Z_R = b S (docs/ARCHITECTURE.md:22-24 of the reference)."""
    dim = q.shape[-1]
    a = [float(k[0, i, 0] @ q[0, 0, 0]) / math.sqrt(dim) for i in range(p + 1)]
    c = p // b
    remote = list(range(max(0, c - 1)))
    S = sum(math.exp(a[j * b]) for j in remote)
    num = torch.zeros(dim, dtype=F64)
    den = 0.0
    for j in remote:
        w = b * math.exp(2 * a[j * b]) / S
        num += w * v[0, j * b:(j + 1) * b, 0].mean(0)
        den += w
    for i in range(max(0, c - 1) * b, p + 1):
        num += math.exp(a[i]) * v[0, i, 0]
        den += math.exp(a[i])
    return num / den


@pytest.mark.parametrize("p", [35, 30, 9, 3])
def test_gate_closed_form_on_constant_blocks(p):
    q, k, v, b, _ = _constant_block_case()
    pos = torch.tensor([[p]])
    expected = _closed_form_output(q, k, v, p, b)
    for fn in (od.eager_attention, od.loop_attention, lambda *a: od.forward_stats(*a)[0]):
        torch.testing.assert_close(fn(q, k, v, pos, b)[0, 0, 0], expected, atol=1e-12, rtol=1e-10)


def test_planted_mistake_is_caught():
    """A copy of the oracle that drops the block-mass term (logit a_i -
    log Z_R instead of a_i + s_j - log Z_R) must fail the closed form."""
    q, k, v, b, _ = _constant_block_case()
    p = 35
    pos = torch.tensor([[p]])

    def mutated(q, k, v, positions, block_size):
        n = k.shape[1]
        a = od._scores(q, k, F64)
        remote, local = od.masks(positions, n, block_size)
        zr = torch.where(remote, a, torch.full_like(a, -math.inf)).logsumexp(-1, keepdim=True)
        logits = torch.where(remote, a - zr, torch.where(local, a, torch.full_like(a, -math.inf)))
        return (logits.softmax(-1) @ od._heads(v, F64)).transpose(1, 2)

    expected = _closed_form_output(q, k, v, p, b)
    assert not torch.allclose(mutated(q, k, v, pos, b)[0, 0, 0], expected, atol=1e-6, rtol=1e-4)


def test_remote_block_permutation_invariance():
    """The gate depends on blocks only through their masses, so permuting
    whole remote blocks (keys and values together) leaves the output fixed."""
    g = _gen(31)
    b, n = 4, 48
    q, k, v = _rand((1, 3, 2, 8), g), _rand((1, n, 2, 8), g), _rand((1, n, 2, 8), g)
    pos = torch.tensor([[47, 45, 44]])  # c = 11: remote blocks 0..9 for all rows
    perm = torch.randperm(10, generator=g)
    order = torch.cat([(perm[:, None] * b + torch.arange(b)).reshape(-1), torch.arange(40, n)])
    out = od.eager_attention(q, k, v, pos, b)
    out_p = od.eager_attention(q, k[:, order], v[:, order], pos, b)
    torch.testing.assert_close(out_p, out, atol=1e-12, rtol=1e-10)


@pytest.mark.parametrize("keep", [1, 2, 64])
def test_sparse_matches_loop_oracle_with_topk(keep):
    """tests/test_attention.py:75-86 case: sparse forward equals the loop
    oracle restricted to the top-k blocks (the degenerate keep=64 equals the
    dense operator)."""
    g = _gen(124)
    q, k, v = _rand((2, 4, 3, 8), g), _rand((2, 45, 3, 8), g), _rand((2, 45, 3, 8), g)
    pos = torch.tensor([[0, 7, 44, 22], [13, 44, 1, 43]])
    expected = od.loop_attention(q, k, v, pos, 4, keep)
    actual, sel = osp.sparse_attention(q, k, v, pos, 4, keep)
    torch.testing.assert_close(actual, expected, rtol=1e-10, atol=1e-11)
    if keep == 64:
        torch.testing.assert_close(actual, od.eager_attention(q, k, v, pos, 4), rtol=1e-10, atol=1e-11)


def test_block_scores_brute_force_and_offset():
    g = _gen(5)
    b, n = 4, 23
    q, k = _rand((1, 3, 2, 8), g), _rand((1, n, 2, 8), g)
    pos = torch.tensor([[22, 13, -1]])
    s = osp.block_scores(q, k, pos, b)
    for t in range(3):
        p = int(pos[0, t])
        for h in range(2):
            for j in range(s.shape[-1]):
                if p < 0 or j >= p // b - 1 or (j + 1) * b > n:
                    assert s[0, t, h, j] == -math.inf
                    continue
                a = [float(k[0, i, h] @ q[0, t, h]) / math.sqrt(8) for i in range(j * b, (j + 1) * b)]
                assert abs(float(s[0, t, h, j]) - math.log(sum(math.exp(x) for x in a))) < 1e-12
    # a slab starting at absolute token 2b scores the same blocks
    # (st/tools/validate.py:120-125)
    shifted = torch.where(pos >= 0, pos + 2 * b, pos)
    full = osp.block_scores(q, torch.cat([k[:, :2 * b], k], 1), shifted, b)
    part = osp.block_scores(q, k, shifted, b, offset=2 * b)
    torch.testing.assert_close(part, full[..., 2:], rtol=0, atol=0)
    _, _, log_zr = osp.select_topk(s, 3)
    fin = torch.isfinite(s)
    for t in range(3):
        for h in range(2):
            vals = s[0, t, h][fin[0, t, h]].tolist()
            exp = math.log(sum(math.exp(x) for x in vals)) if vals else -math.inf
            assert (math.isinf(exp) and math.isinf(float(log_zr[0, t, h]))) or \
                abs(float(log_zr[0, t, h]) - exp) < 1e-12


def test_select_tie_order_and_padding():
    s = torch.tensor([[1.0, 3.0, 3.0, -math.inf, 2.0, 3.0]], dtype=torch.float32)
    values, ids, _ = osp.select_topk(s, 4)
    assert ids.tolist() == [[1, 2, 5, 4]]
    assert values.tolist() == [[3.0, 3.0, 3.0, 2.0]]
    values, ids, _ = osp.select_topk(s, 8)
    assert ids.tolist() == [[1, 2, 5, 4, 0, -1, -1, -1]]
    assert values[0, 5:].isinf().all()


def test_planted_selection_is_recovered():
    """Planted blocks (exploration_amd.workloads.planted_sparse, the cfg4
    generator) are the oracle's top-k, in plant order."""
    from exploration_amd.workloads import planted_sparse
    q, (k, v), pos, expected = planted_sparse(batch=1, heads=2, length=4096, queries=4, dim=32, block=16,
                                              topk=8, page_tokens=16, dtype=torch.float32, seed=3,
                                              device="cpu", paged=False)
    s = osp.block_scores(q, k, pos, 16)
    values, ids, _ = osp.select_topk(s, 8)
    assert torch.equal(ids, expected)
    # margin between consecutive selected blocks and to the first unselected
    top9 = torch.sort(s, -1, descending=True).values[..., :9]
    assert float((top9[..., :-1] - top9[..., 1:]).min()) > 0.01
