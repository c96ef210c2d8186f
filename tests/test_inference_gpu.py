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
