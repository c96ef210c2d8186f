"""Streaming prefill + paged sparse decode (InferenceSession) on the GPU.

* topk >= every visible block: the session's sparse read selects every
  remote block, which is the dense operator (the reference's degenerate
  case, st/models/stack.py:20-25), so its logits must equal model.forward's
  dense path; a multi-chunk prefill also checks the halo hand-over between
  encoder chunks;
* topk below the block count, single-chunk prefill (bitwise the same
  hidden states and K/V as model.encode): logits equal model.forward's
  sparse path;
* the host tier (K/V in pinned host memory, streamed scan and paged read)
  and the disk tier (a file mapping, staged through pinned buffers) equal
  the HBM tier, and the disk tier leaves its directory empty.
fp32 models; tolerance 1e-4 relative to the largest logit.
"""
import pytest
import torch

import exploration_amd.model as M
from exploration_amd.inference import InferenceSession
from exploration_amd.train import synthetic_lm_batch

pytestmark = pytest.mark.gpu


def model(device, topk):
    torch.manual_seed(0)
    cfg = {"vocab_size": 64, "dim": 128, "heads": 2, "block_size": 16, "topk": topk, "arch": "Lx2,G",
           "ffn_ratio": 4.0}
    return M.build_model(cfg, execution={"checkpoint_chunks": False}, device=device).eval()


def session_logits(m, ids, positions, **options):
    with InferenceSession(m, **options) as s:
        s.prefill(ids, positions)
        parts = [logits for _, logits, _ in s.iter_logits()]
    return torch.cat(parts, 1).float()


def close(a, b):
    torch.testing.assert_close(a, b, rtol=1e-4, atol=1e-4 * float(b.abs().max()))


@pytest.mark.parametrize("encoder_chunk", [256, 4096])
def test_all_blocks_selected_equals_dense(device, encoder_chunk):
    print(f"session dense-equivalent encoder_chunk={encoder_chunk}", flush=True)
    n = 1024
    m = model(device, topk=n // 16)
    ids, _ = synthetic_lm_batch(64, n, batch=1, seed=3)
    positions = torch.tensor([[0, 5, 31, 32, 100, 511, 777, n - 1]])
    got = session_logits(m, ids, positions, encoder_chunk=encoder_chunk, query_chunk=4)
    sup = torch.zeros(1, n, dtype=torch.bool)
    sup[0, positions[0]] = True
    with torch.no_grad():
        want = m(ids.to(device), sup=sup.to(device), compact=True).float()
    close(got, want)


def test_sparse_session_equals_model_forward(device):
    print("session sparse", flush=True)
    n = 1024
    m = model(device, topk=4)
    ids, _ = synthetic_lm_batch(64, n, batch=1, seed=4)
    positions = torch.arange(n - 16, n)[None]
    got = session_logits(m, ids, positions, encoder_chunk=4096)
    sup = torch.zeros(1, n, dtype=torch.bool)
    sup[0, n - 16:] = True
    with torch.no_grad():
        want = m(ids.to(device), sup=sup.to(device), compact=True).float()
    close(got, want)


@pytest.mark.parametrize("tier", ["cpu", "disk"])
@pytest.mark.parametrize("topk", [4, 64])
def test_host_tier_equals_hbm_tier(device, topk, tier, tmp_path):
    print(f"session {tier} tier topk={topk}", flush=True)
    n = 1024
    m = model(device, topk=topk)
    ids, _ = synthetic_lm_batch(64, n, batch=2, seed=5)
    positions = torch.tensor([[n - 1, 600, 17, n - 300], [n - 2, 33, 511, 512]])
    # same encoder chunking in both sessions: identical hidden states and K/V
    hbm = session_logits(m, ids, positions, cache="cuda", encoder_chunk=256)
    host = session_logits(m, ids, positions, cache=tier, cache_dir=str(tmp_path), encoder_chunk=256,
                          page_tokens=240)
    close(host, hbm)
    assert list(tmp_path.iterdir()) == []


@pytest.mark.parametrize("dtype,dim", [(torch.bfloat16, 64), (torch.float32, 40), (torch.float16, 3)], ids=str)
def test_paged_write_round_trip(device, dtype, dim):
    """st_paged_kv_write through a random page table, in chunks that start
    and end inside pages: reading the pages back gives the rows written,
    bit for bit (16-, 16- and 2-byte pieces for these row lengths)."""
    print(f"paged write {dtype} D={dim}", flush=True)
    from exploration_amd import PagedKV
    gen = torch.Generator(device=device).manual_seed(3)
    batch, n, heads, page = 2, 1000, 3, 128
    k = torch.randn(batch, n, heads, dim, generator=gen, device=device).to(dtype)
    v = torch.randn(batch, n, heads, dim, generator=gen, device=device).to(dtype)
    pages = -(-n // page)
    pool = torch.zeros(batch * pages + 3, heads, page, dim, dtype=dtype, device=device)
    table = torch.randperm(batch * pages + 3, generator=gen, device=device)[:batch * pages].reshape(batch, pages)
    cache = PagedKV(pool, torch.zeros_like(pool), table, n, offset=256)
    for lo, hi in [(0, 1), (1, 200), (200, 640), (640, 999), (999, 1000)]:
        cache.write(256 + lo, k[:, lo:hi], v[:, lo:hi])
    gk, gv = cache.gather()
    assert torch.equal(gk, k) and torch.equal(gv, v)
    with pytest.raises(ValueError, match="outside owned shard"):
        cache.write(256 + 990, k[:, :20], v[:, :20])


def test_paged_write_skips_entries_outside_the_pool(device):
    """A table entry outside [0, pool_pages) writes nothing; the other pages
    are written."""
    from exploration_amd import _lib
    lib = _lib.load()
    k = torch.arange(2 * 8 * 4, device=device, dtype=torch.float32).reshape(1, 16, 1, 4)
    v = -k
    kp, vp = (torch.zeros(2, 1, 8, 4, device=device) for _ in range(2))
    table = torch.tensor([[1, 7]], dtype=torch.int32, device=device)   # page 1 of the sequence is bad
    _lib.check(lib.st_paged_kv_write(0, 1, 16, 1, 4, _lib.ptr(k), _lib.ptr(v), _lib.ptr(table), 8, 2, 0,
                                     _lib.ptr(kp), _lib.ptr(vp), 2, _lib.stream_of(k)), lib)
    torch.cuda.synchronize()
    assert torch.equal(kp[1, 0], k[0, :8, 0]) and torch.equal(vp[1, 0], v[0, :8, 0])
    assert not kp[0].any() and not vp[0].any()


def test_session_131072_tokens_paged_hbm_tier(device, monkeypatch):
    """stack_100m shape (dim 1024, H16 hd64, b16, top-64, Lx7,G), bf16, random
    init, one 131,072-token prompt, 16 tail queries, HBM tier. The K/V sit
    in 128-token pages written by the paged-write kernel; the session's
    sparse read (recorded at the call) is checked against the oracle's block
    scores, selection and pop on the K/V read back from those pages. With
    random weights the top-64 order is rarely decided beyond float noise, so
    every row's selection must be a top-64 of the oracle's scores within
    1e-3, ids must match bit-exactly on every decided row, and the output
    uses the kernel's own selection."""
    print("session 131072 tokens, HBM pages", flush=True)
    import exploration_amd.inference as inf
    from exploration_amd import PagedKV
    from oracle import sparse as osp
    from tests.helpers import assert_close
    calls = []
    real = inf.sparse_attention

    def recording(q, cache, positions, b, topk, **kw):
        want = kw.pop("return_selection", False)
        out, sel = real(q, cache, positions, b, topk, return_selection=True, **kw)
        calls.append((q.clone(), cache, positions.clone(), out.clone(), sel))
        return (out, sel) if want else out

    monkeypatch.setattr(inf, "sparse_attention", recording)
    torch.manual_seed(0)
    m = M.build_model(M.STACK_100M, device=device, dtype=torch.bfloat16).eval()
    n, b, topk = 131072, 16, 64
    ids, _ = synthetic_lm_batch(256, n, batch=1, seed=6)
    positions = torch.arange(n - 16, n)[None]
    with InferenceSession(m) as s:
        s.prefill(ids, positions)
        assert s.plan.cache == "cuda" and s.plan.page_tokens == 128 and s.plan.query_chunk == 16
        logits = [x for _, x, _ in s.iter_logits()]
        torch.cuda.synchronize()
        assert len(calls) == 1 and torch.isfinite(logits[0].float()).all()
        q, cache, pos, out, sel = calls[0]
        assert isinstance(cache, PagedKV) and cache.page_tokens == 128 and cache.length == n
        k, v = cache.gather()
    ref_s = osp.block_scores(q.float(), k.float(), pos, b)
    ev, ei, ez = osp.select_topk(ref_s, topk)
    assert_close(sel["log_zr"], ez, torch.float32, "log_zr")
    assert_close(sel["scores"], ev, torch.float32, "top scores")
    got = sel["indices"]
    assert (got >= 0).all()
    picked = ref_s.gather(-1, got)
    assert float((ev[..., -1:] - picked).max()) < 1e-3, "a selected block is not in the oracle's top-64"
    assert (got.sort(-1).values.diff(dim=-1) > 0).all(), "repeated block in a selection"
    margins = torch.sort(ref_s, -1, descending=True).values[..., :topk + 1]
    decided = (margins[..., :-1] - margins[..., 1:]).min(-1).values > 1e-3
    print(f"  {int(decided.sum())}/{decided.numel()} rows with a decided top-{topk}", flush=True)
    assert torch.equal(got[decided], ei[decided])
    out_e, _ = osp.pop(q.float(), k.float(), v.float(), pos, got, sel["scores"], sel["log_zr"], b)
    assert_close(out, out_e, torch.bfloat16, "out")
