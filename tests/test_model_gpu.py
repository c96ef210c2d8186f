"""Stack model on the GPU: its read rounds through the HIP operators against
the same model with the oracle operators (same weights, same inputs).

* dense training path (forward_loss + backward), fp32 end to end and bf16
  autocast (the cfg5 setting), at head_dim 64 / block 16 (the stack_100m
  operator shape);
* no-grad sparse read (topk below the block count) against the per-position
  loop with the same top-k.
Tolerances: fp32 rtol 1e-4 on the loss and 1e-3 on gradients (the operator
is fp32-exact to ~1e-5; the model adds ~1e3 summations); bf16 autocast 2e-2
on the loss and a gradient cosine above 0.999.
"""
import pytest
import torch

import exploration_amd.model as M
from exploration_amd.train import synthetic_lm_batch
from oracle import model as om

pytestmark = pytest.mark.gpu


def small_model(device, topk=64):
    torch.manual_seed(0)
    cfg = {"vocab_size": 64, "dim": 128, "heads": 2, "block_size": 16, "topk": topk, "arch": "Lx2,G",
           "ffn_ratio": 4.0}
    return M.build_model(cfg, execution={"checkpoint_chunks": False, "query_chunk": 96}, device=device)


def loss_and_grads(model, ids, targets, autocast):
    model.zero_grad(set_to_none=True)
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        out = model.forward_loss(ids, targets)
        loss = out["loss_sum"] / out["count"]
    loss.backward()
    return loss.detach(), [p.grad.detach().clone() for p in model.parameters()]


@pytest.mark.parametrize("autocast", [False, True], ids=["fp32", "bf16"])
def test_forward_loss_and_grads_match_oracle(device, monkeypatch, autocast):
    print(f"model dense autocast={autocast}", flush=True)
    m = small_model(device)
    ids, targets = synthetic_lm_batch(64, 512, batch=2, seed=1, device=device)
    loss, grads = loss_and_grads(m, ids, targets, autocast)
    monkeypatch.setattr(M, "dense_attention", om.dense_op)
    ref_loss, ref_grads = loss_and_grads(m, ids, targets, False)
    torch.cuda.synchronize()
    assert torch.isfinite(loss)
    if not autocast:
        torch.testing.assert_close(loss, ref_loss, rtol=1e-4, atol=1e-5)
        for g, r in zip(grads, ref_grads):
            torch.testing.assert_close(g, r, rtol=1e-3, atol=1e-5 * float(r.abs().max()) + 1e-7)
    else:
        torch.testing.assert_close(loss, ref_loss, rtol=2e-2, atol=0.0)
        cos = torch.nn.functional.cosine_similarity(torch.cat([g.flatten().float() for g in grads]),
                                                    torch.cat([r.flatten().float() for r in ref_grads]), dim=0)
        assert float(cos) > 0.999, float(cos)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
def test_sparse_read_matches_oracle(device, monkeypatch, dtype):
    """topk 4 of 64 blocks: the no-grad read through st_sparse_fwd. Random
    weights leave near-ties among block scores, so the oracle side pops the
    blocks the kernel selected and checks separately that each of them
    scores within rounding of the oracle's own top-k threshold."""
    print(f"model sparse {dtype}", flush=True)
    import exploration_amd.sparse as S
    from oracle import sparse as osp

    m = small_model(device, topk=4).to(dtype).eval()
    ids, _ = synthetic_lm_batch(64, 1024, batch=1, seed=2, device=device)
    sup = torch.zeros(1, 1024, dtype=torch.bool, device=device)
    sup[:, -16:] = True
    selections = []

    def hip_recording(q, cache, positions, b, topk, backend="auto", **kw):
        out, sel = S.sparse_attention(q, cache, positions, b, topk, backend, return_selection=True)
        selections.append(sel["indices"].clone())
        return out

    work = torch.float64 if dtype == torch.float32 else torch.float32
    tol = 1e-4 if dtype == torch.float32 else 5e-2

    def oracle_with_selection(q, cache, positions, b, topk, backend="auto", **kw):
        chosen = selections.pop(0)
        qw, kw_, vw = q.to(work), cache.k.to(work), cache.v.to(work)
        scores = osp.block_scores(qw, kw_, positions, b)
        values, _, log_zr = osp.select_topk(scores, topk)
        ok = chosen >= 0
        picked = scores.gather(-1, chosen.clamp(min=0)).masked_fill(~ok, float("-inf"))
        kth = values[..., -1:].expand_as(picked)
        assert bool(((picked >= kth - tol * kth.abs().clamp(min=1)) | ~ok).all()), "selection beyond a near-tie"
        assert torch.equal(ok, torch.isfinite(values)), "selected block count differs"
        out, _ = osp.pop(qw, kw_, vw, positions, chosen, picked, log_zr, b)
        return out.to(q.dtype)

    with torch.no_grad():
        monkeypatch.setattr(M, "sparse_attention", hip_recording)
        got = m(ids, sup=sup, compact=True).float()
        assert len(selections) == 1
        monkeypatch.setattr(M, "sparse_attention", oracle_with_selection)
        want = m(ids, sup=sup, compact=True).float()
    torch.cuda.synchronize()
    torch.testing.assert_close(got, want, rtol=tol, atol=tol * float(want.abs().max()))
