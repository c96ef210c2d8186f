"""The graphed training step (one HIP graph per step) against eager steps.

Two copies of one model train on the same batches: one with ``train_step``,
one with ``GraphedStep`` (capture once, replay). Every replay's loss and
gradient norm must match the eager step's, and the parameters after the last
step must agree: a graph node that goes stale after its first replay
(memsets, host-side values baked in at capture) shows up as a drift here.
Between replays the test does its own eager work and synchronises.
checkpoint_chunks on, several encoder and read chunks per step, bf16
autocast: the cfg5 step's structure at a small size; and the cfg5 widths
(dim 1024, FFN 4096) over 8192 tokens in one chunk, where the reductions
over all rows are long (two layers to keep it quick).
"""
import copy

import pytest
import torch

import exploration_amd.model as M
from exploration_amd.train import GraphedStep, make_optimizer, synthetic_lm_batch, train_step

pytestmark = pytest.mark.gpu


def test_graphed_step_matches_eager(device):
    print("graphed training step vs eager", flush=True)
    torch.manual_seed(0)
    cfg = {"vocab_size": 64, "dim": 128, "heads": 2, "block_size": 16, "topk": 64, "arch": "Lx2,G",
           "ffn_ratio": 4.0}
    execution = {"checkpoint_chunks": True, "encoder_chunk": 128}
    eager = M.build_model(cfg, execution=execution, device=device)
    eager.pos_chunk = 200  # three read chunks of a 512-token sequence
    graphed = copy.deepcopy(eager)
    n, warmup, steps = 512, 2, 4
    batches = [synthetic_lm_batch(64, n, batch=2, seed=s, device=device) for s in range(steps + 1)]
    batches[2][1][0, 100:] = -100  # a step with fewer supervised positions in one row

    opt_e = make_optimizer(eager, capturable=True)
    for _ in range(warmup):
        train_step(eager, opt_e, *batches[0], width=n, autocast_cache=False)
    want = []
    for ids, targets in batches[1:]:
        loss, norm, count = train_step(eager, opt_e, ids, targets, width=n, autocast_cache=False)
        want.append((loss.item(), norm.item(), count.item()))

    opt_g = make_optimizer(graphed, capturable=True)
    step = GraphedStep(graphed, opt_g, *batches[0], warmup=warmup)
    got = []
    for i, (ids, targets) in enumerate(batches[1:]):
        loss, norm, count = step(ids, targets)
        got.append((loss.item(), norm.item(), count.item()))
        torch.ones(1000, device=device).cumsum(0)  # eager work between replays
        torch.cuda.synchronize()
        print(f"  step {i}: eager {want[i]} graphed {got[i]}", flush=True)
    for (le, ne, ce), (lg, ng, cg) in zip(want, got):
        assert ce == cg
        assert lg == pytest.approx(le, rel=1e-4)
        assert ng == pytest.approx(ne, rel=1e-3)
    for (name, pe), pg in zip(eager.named_parameters(), graphed.parameters()):
        torch.testing.assert_close(pg, pe, rtol=1e-4, atol=1e-5, msg=name)


def test_graphed_step_matches_eager_full_width(device):
    """Every replay bitwise equal to the eager step at cfg5 widths with whole
    8192-token chunks: long reductions (the FFN bias gradients over 8192
    rows) once recorded memset nodes that went stale from the third replay."""
    print("graphed training step vs eager, cfg5 widths, whole chunks", flush=True)
    cfg = dict(M.STACK_100M, arch="Lx1,G")
    execution = {"checkpoint_chunks": True, "encoder_chunk": 8192, "query_chunk": 8192, "loss_chunk": 8192}
    ids, targets = synthetic_lm_batch(cfg["vocab_size"], 8192, batch=1, seed=0, device=device)
    runs = {}
    for mode in ("eager", "graph"):
        torch.manual_seed(0)
        m = M.build_model(cfg, execution=execution, device=device)
        opt = make_optimizer(m, capturable=True)
        if mode == "eager":
            losses = [train_step(m, opt, ids, targets, width=8192, autocast_cache=False)[0].item() for _ in range(7)]
        else:
            step = GraphedStep(m, opt, ids, targets, warmup=1)
            print(f"  captured nodes {step.node_types}", flush=True)
            assert set(step.node_types) <= {"kernel", "memcpy", "empty", "event_record", "wait_event"}
            # six replays queued back to back, read afterwards
            out = [step(ids, targets)[0].clone() for _ in range(6)]
            losses = [None] + [x.item() for x in out]
        runs[mode] = (losses, [p.detach().clone() for p in m.parameters()])
        print(f"  {mode}: {losses}", flush=True)
    assert runs["graph"][0][1:] == runs["eager"][0][1:]
    for pe, pg in zip(runs["eager"][1], runs["graph"][1]):
        assert torch.equal(pe, pg)


def test_graphed_step_skips_empty_and_nonfinite_batches(device):
    """A replay whose batch has no supervised token (0/0 loss) leaves every
    parameter and optimizer moment unchanged on the device (fused AdamW's
    found_inf), and the next replay trains normally; the eager path raises
    before backward, as the reference does (st/runtime/engine.py:170-177)."""
    print("graphed step skip on empty batch", flush=True)
    torch.manual_seed(0)
    cfg = {"vocab_size": 64, "dim": 64, "heads": 2, "block_size": 16, "topk": 64, "arch": "Lx1,G",
           "ffn_ratio": 2.0}
    m = M.build_model(cfg, execution={"checkpoint_chunks": True, "encoder_chunk": 128}, device=device)
    opt = make_optimizer(m, capturable=True)
    ids, targets = synthetic_lm_batch(64, 256, batch=1, seed=1, device=device)
    step = GraphedStep(m, opt, ids, targets, warmup=1)
    before = [p.detach().clone() for p in m.parameters()]
    moments = [opt.state[p]["exp_avg"].clone() for p in m.parameters()]
    steps = [opt.state[p]["step"].clone() for p in m.parameters()]
    empty = torch.full_like(targets, -100)
    loss, norm, count = step(ids, empty)
    torch.cuda.synchronize()
    assert int(count) == 0 and not bool(torch.isfinite(loss))
    for p, b, mo, st in zip(m.parameters(), before, moments, steps):
        assert torch.equal(p, b)
        assert torch.equal(opt.state[p]["exp_avg"], mo)
        assert torch.equal(opt.state[p]["step"], st)
    loss, _, count = step(ids, targets)
    torch.cuda.synchronize()
    assert int(count) == 255 and bool(torch.isfinite(loss))
    assert any(not torch.equal(p, b) for p, b in zip(m.parameters(), before))
    with pytest.raises(ValueError, match="no supervised tokens"):
        train_step(m, opt, ids, empty)
