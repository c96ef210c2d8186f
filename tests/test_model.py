"""Stack model restatement on the CPU: architecture, parameter inventory and
the read plumbing, with the package's attention operators replaced by the
oracle (the product path has no CPU operator). Cases follow the reference's
tests/test_stack_model.py (model(): vocab 31, dim 16, heads 2, b 2, topk 3,
pos_chunk 3; arch parser cases; future perturbation and prefix invariance;
the dense read at topk >= blocks against the per-position loop)."""
import re

import pytest
import torch

import exploration_amd.model as M
from oracle import model as om

pytestmark = pytest.mark.filterwarnings("ignore::UserWarning")


@pytest.fixture(autouse=True)
def oracle_ops(monkeypatch):
    monkeypatch.setattr(M, "dense_attention", om.dense_op)
    monkeypatch.setattr(M, "sparse_attention", om.sparse_op)


def small(**overrides):
    args = dict(vocab_size=31, dim=16, heads=2, block_size=2, topk=3, arch="Lx2,G", pos_chunk=3)
    args.update(overrides)
    return M.StackModel(**args)


@pytest.mark.parametrize("bad", ["", "G,L", "Lx0", "X", "(L)x0", "(G)", "L,", "Lx2,(G)x", "L,Gx2,Lx1",
                                 "Lx", "Lx2x3", "(L)x+1", "((L))x2", "L x2"])
def test_arch_parser_rejects(bad):
    with pytest.raises(ValueError):
        small(arch=bad)


def test_arch_parser_results_and_messages():
    assert M.parse_arch(" Lx2 , (G)x3,G ") == [("L", 2, False), ("G", 3, True), ("G", 1, False)]
    assert M.parse_arch("(L)x1") == [("L", 1, True)]
    for bad, message in [("", "nonempty spec"), ("(G)", "'(X)xN'"), ("Q", "unknown layer kind"),
                         ("Lx0", "positive integer"), ("G,L", "precede")]:
        with pytest.raises(ValueError, match=re.escape(message)):
            M.parse_arch(bad)


@pytest.mark.parametrize("good,passes", [("L", 1), ("Lx2,G", 3), ("(L)x3,(G)x2", 5), ("Gx2", 2)])
def test_arch_parser_accepts(good, passes):
    m = small(arch=good)
    assert len(m.local) + len(m.reads) == passes


def test_shared_weight_cycling():
    shared = small(arch="L,(G)x2")
    assert shared.reads[0] is shared.reads[1]
    indep = small(arch="L,Gx2")
    assert indep.reads[0] is not indep.reads[1]


def test_stack_100m_parameter_count():
    """configs/stack_100m.json is ~101M parameters (docs/VALIDATION.md:63).
    Counted from the reference's modules: embedding tied with lm_head
    256*1024; seven local blocks of 2 LayerNorms (4096), qkv 3*1024^2, out
    1024^2, FFN 2*4*1024^2 + 4096 + 1024; one read block of 2 LayerNorms, wq,
    read_out and the FFN; raw K/V LayerNorm + 2*1024^2; final LayerNorm."""
    m = M.build_model(M.STACK_100M, device="meta")
    d = 1024
    ffn = 2 * 4 * d * d + 4 * d + d
    local = 4 * d + 4 * d * d + ffn
    read = 4 * d + 2 * d * d + ffn
    expected = 256 * d + 7 * local + read + (2 * d + 2 * d * d) + 2 * d
    assert expected == 101_003_264
    assert sum(p.numel() for p in m.parameters()) == expected


def test_state_dict_names_and_shapes():
    """The reference's module names (st/models/stack.py:170-188,
    st/models/blocks.py:102-207), so its checkpoints load unchanged."""
    m = small(arch="L,G")
    shapes = {k: tuple(v.shape) for k, v in m.state_dict().items()}
    d, h = 16, 64
    expected = {
        "embedding.weight": (31, d),
        "local.0.attn_norm.weight": (d,), "local.0.attn_norm.bias": (d,),
        "local.0.qkv.weight": (3 * d, d), "local.0.out.weight": (d, d),
        "local.0.ffn_norm.weight": (d,), "local.0.ffn_norm.bias": (d,),
        "local.0.ffn.0.weight": (h, d), "local.0.ffn.0.bias": (h,),
        "local.0.ffn.2.weight": (d, h), "local.0.ffn.2.bias": (d,),
        "reads.0.q_norm.weight": (d,), "reads.0.q_norm.bias": (d,),
        "reads.0.wq.weight": (d, d), "reads.0.read_out.weight": (d, d),
        "reads.0.ffn_norm.weight": (d,), "reads.0.ffn_norm.bias": (d,),
        "reads.0.ffn.0.weight": (h, d), "reads.0.ffn.0.bias": (h,),
        "reads.0.ffn.2.weight": (d, h), "reads.0.ffn.2.bias": (d,),
        "raw_kv.norm.weight": (d,), "raw_kv.norm.bias": (d,), "raw_kv.proj.weight": (2 * d, d),
        "final_norm.weight": (d,), "final_norm.bias": (d,),
        "lm_head.weight": (31, d),
    }
    assert shapes == expected
    assert m.lm_head.weight is m.embedding.weight


def test_dense_read_matches_loop_oracle():
    """topk >= blocks: the chunked dense read equals the per-position loop."""
    torch.manual_seed(123)
    m = small(topk=64).double().eval()
    ids = torch.randint(31, (2, 21))
    sup = torch.zeros(2, 21, dtype=torch.bool)
    sup[:, -4:] = True
    with torch.no_grad():
        got = m(ids, sup=sup)
        want = om.oracle_logits(m, ids, [17, 18, 19, 20])
        torch.testing.assert_close(got[:, -4:], want, rtol=1e-9, atol=1e-10)
        assert got[:, :-4].abs().max() == 0
        full = m(ids)
        torch.testing.assert_close(full, om.oracle_logits(m, ids, list(range(21))), rtol=1e-9, atol=1e-10)


def test_sparse_read_matches_loop_oracle():
    """topk below the block count: the no-grad sparse read (top-k blocks per
    head) equals the per-position loop with the same top-k."""
    torch.manual_seed(7)
    m = small(topk=2).double().eval()
    ids = torch.randint(31, (2, 19))
    with torch.no_grad():
        torch.testing.assert_close(m(ids), om.oracle_logits(m, ids, list(range(19))), rtol=1e-9, atol=1e-10)
    with pytest.raises(ValueError):
        m(ids)  # gradient-enabled sparse read is not shipped


@pytest.mark.parametrize("arch", ["Lx2,G", "Lx2,(G)x2", "Lx2,Gx2"])
def test_future_perturbation_and_prefix_invariance(arch):
    torch.manual_seed(1)
    m = small(arch=arch, topk=64).double().eval()
    ids = torch.randint(31, (2, 33))
    with torch.no_grad():
        full = m(ids)
        for cut in [1, 3, 4, 5, 8, 15, 16, 17, 31, 32]:
            changed = ids.clone()
            changed[:, cut:] = (changed[:, cut:] + 7) % 31
            torch.testing.assert_close(m(changed)[:, :cut], full[:, :cut], rtol=1e-9, atol=1e-10)
            torch.testing.assert_close(m(ids[:, :cut])[:, :cut], full[:, :cut], rtol=1e-9, atol=1e-10)


def test_encoder_chunk_invariance():
    """Streaming the local blocks in query chunks never changes values
    (st/models/blocks.py:1-9)."""
    torch.manual_seed(3)
    a = small(encoder_chunk=2).double()
    b = small(encoder_chunk=16).double()
    b.load_state_dict(a.state_dict())
    ids = torch.randint(31, (2, 27))
    with torch.no_grad():
        for x, y in zip(a.encode(ids), b.encode(ids)):
            torch.testing.assert_close(x, y, rtol=1e-12, atol=1e-12)


def test_forward_loss_matches_logits():
    """forward_loss's SUM cross entropy and hit counts equal those of the
    logits forward() gives at the same supervised positions."""
    torch.manual_seed(5)
    m = small(topk=64).double()
    ids = torch.randint(31, (2, 23))
    targets = torch.randint(31, (2, 23))
    targets[0, 4] = -100
    sup = torch.rand(2, 23) < 0.5
    out = m.forward_loss(ids, targets, sup)
    mask = sup & (targets != -100)
    logits = m(ids)
    # the loss head works in fp32 (st/models/stack.py:263)
    want = torch.nn.functional.cross_entropy(logits[mask].float(), targets[mask], reduction="sum")
    torch.testing.assert_close(out["loss_sum"], want, rtol=1e-6, atol=1e-6)
    assert int(out["count"]) == int(mask.sum())
    assert int(out["correct"]) == int((logits[mask].argmax(-1) == targets[mask]).sum())
    out["loss_sum"].backward()
    assert all(torch.isfinite(p.grad).all() for p in m.parameters() if p.grad is not None)


def test_configuration_errors():
    with pytest.raises(ValueError):
        small(block_size=1)
    with pytest.raises(ValueError):
        small(dim=18, heads=4)
    with pytest.raises(ValueError):
        M.ModelConfig.from_dict({"dim": 8, "nonsense": 1})
    with pytest.raises(ValueError):
        small()(torch.zeros(0, 3, dtype=torch.long))


def test_training_step_has_no_lookback_ops(monkeypatch):
    """The training step (forward_loss with a given width, then backward)
    runs no aten op whose GPU kernel is a decoupled look-back scan (device
    sort, unique, selection, advanced-index scatter, the sort-based embedding
    backward): such kernels spin on flags set by other workgroups and have
    hung in replays of the captured step. The dense operator is replaced by a
    differentiable stand-in so the trace runs on the CPU."""
    from torch.utils._python_dispatch import TorchDispatchMode

    class Ops(TorchDispatchMode):
        def __init__(self):
            super().__init__()
            self.seen = set()

        def __torch_dispatch__(self, func, types, args=(), kwargs=None):
            self.seen.add(str(func))
            return func(*args, **(kwargs or {}))

    torch.manual_seed(0)
    cfg = {"vocab_size": 64, "dim": 64, "heads": 2, "block_size": 16, "topk": 64, "arch": "Lx1,G", "ffn_ratio": 2.0}
    m = M.build_model(cfg, execution={"checkpoint_chunks": True, "encoder_chunk": 128, "query_chunk": 100,
                                      "loss_chunk": 64})
    monkeypatch.setattr(M, "dense_attention", lambda q, k, v, pos, b, backend, **kw: q * 1.0)
    ids = torch.randint(64, (2, 256))
    targets = torch.roll(ids, -1, 1)
    targets[:, -1] = -100
    targets[1, 30:90] = -100
    with Ops() as ops:
        r = m.forward_loss(ids, targets, width=256)
        (r["loss_sum"] / r["count"]).backward()
    banned = ("aten.sort", "aten.index.", "aten.index_put", "aten.nonzero", "aten._unique", "aten.unique",
              "aten.masked_select", "aten.embedding_dense_backward")
    assert not [op for op in ops.seen if op.startswith(banned)], sorted(ops.seen)
    # and the loss is the one the oracle-checked path computes
    ref = m.forward_loss(ids, targets)
    torch.testing.assert_close(r["loss_sum"], ref["loss_sum"], rtol=1e-6, atol=1e-6)
    assert int(r["count"]) == int(ref["count"]) == 2 * 255 - 60


@pytest.mark.parametrize("rows", [1, 5, 128, 129, 240, 8192, 40000])
def test_column_sum_stages(rows):
    """The staged bias-gradient reduction equals a plain row sum (float64
    stays float64; 16-bit inputs accumulate in fp32)."""
    t = torch.randn(rows, 33, generator=torch.Generator().manual_seed(rows), dtype=torch.float64)
    torch.testing.assert_close(M._column_sum(t), t.sum(0), rtol=1e-12, atol=1e-10)
    tb = t.bfloat16()
    got = M._column_sum(tb)
    assert got.dtype == torch.float32
    torch.testing.assert_close(got.double(), tb.double().sum(0), rtol=1e-5, atol=1e-3)


def test_feedforward_matches_sequential():
    """FeedForward's split bias add is the reference's Linear/GELU/Linear,
    values and gradients (gradcheck in float64)."""
    torch.manual_seed(0)
    f = M.FeedForward(16, 2.0).double()
    x = torch.randn(3, 7, 16, dtype=torch.float64, requires_grad=True)
    ref = torch.nn.Sequential.forward(f, x)
    y = f(x)
    torch.testing.assert_close(y, ref, rtol=1e-12, atol=1e-12)
    assert torch.autograd.gradcheck(lambda t: f(t), (x,))
    params = [f[0].weight, f[0].bias, f[2].weight, f[2].bias, x]
    for a, b in zip(torch.autograd.grad(y.sum(), params), torch.autograd.grad(ref.sum(), params)):
        torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)


def test_eager_step_guards_run_before_backward(monkeypatch):
    """Without ``width`` the step applies the reference's host guards before
    backward (st/runtime/engine.py:170-177): an empty batch raises
    ValueError, a non-finite loss FloatingPointError, and in both cases no
    gradient is written and the optimizer never steps."""
    from exploration_amd.train import make_optimizer, train_step

    torch.manual_seed(0)
    cfg = {"vocab_size": 64, "dim": 64, "heads": 2, "block_size": 16, "topk": 64, "arch": "Lx1,G", "ffn_ratio": 2.0}
    m = M.build_model(cfg, execution={"checkpoint_chunks": False, "encoder_chunk": 128})
    monkeypatch.setattr(M, "dense_attention", lambda q, k, v, pos, b, backend, **kw: q * 1.0)
    opt = make_optimizer(m)
    ids = torch.randint(64, (1, 64))
    targets = torch.roll(ids, -1, 1)
    before = [p.detach().clone() for p in m.parameters()]
    with pytest.raises(ValueError, match="no supervised tokens"):
        train_step(m, opt, ids, torch.full_like(targets, -100), precision="fp32")
    with torch.no_grad():
        m.lm_head.weight[0, 0] = float("nan")
    before = [p.detach().clone() for p in m.parameters()]
    with pytest.raises(FloatingPointError, match="not applied"):
        train_step(m, opt, ids, targets, precision="fp32")
    assert all(p.grad is None for p in m.parameters())
    assert not opt.state
    for p, b in zip(m.parameters(), before):
        assert torch.equal(p.nan_to_num(), b.nan_to_num())


def test_weights_cast_once_leaves_gradients_bitwise_unchanged():
    """Under autocast without its cast cache (the graph-captured step), each
    linear use casts its fp32 weight; weights_cast_once() casts each weight
    once per step and sums the uses' gradients in fp32 itself. The loss and
    every parameter gradient (the tied embedding / output weight included)
    must be bitwise those of casting at every use (checkpointed encoder
    chunks, read rounds and loss chunks included), and each weight must be
    cast once."""
    torch.manual_seed(0)
    cfg = {"vocab_size": 64, "dim": 32, "heads": 2, "block_size": 4, "topk": 64, "arch": "Lx2,G", "ffn_ratio": 2.0}
    m = M.build_model(cfg, execution={"checkpoint_chunks": True, "encoder_chunk": 16, "loss_chunk": 8})
    ids = torch.randint(64, (2, 48))
    targets = torch.roll(ids, -1, 1)

    def grads(scope):
        m.zero_grad(set_to_none=True)
        with scope:
            with torch.autocast("cpu", dtype=torch.bfloat16, cache_enabled=False):
                loss = m.forward_loss(ids, targets)["loss_sum"]
            loss.backward()
        return loss.detach(), [p.grad.clone() for p in m.parameters()]

    import contextlib

    uses, copies = [], {}
    real_apply = M._CastUse.apply

    def counting_apply(low, weight, step):
        uses.append(id(weight))
        copies.setdefault(id(weight), low)
        assert copies[id(weight)] is low  # every use of a weight reads the same copy
        return real_apply(low, weight, step)

    loss_ref, g_ref = grads(contextlib.nullcontext())
    M._CastUse.apply = counting_apply
    try:
        loss_once, g_once = grads(M.weights_cast_once())
    finally:
        M._CastUse.apply = real_apply
    assert torch.equal(loss_ref, loss_once)
    for a, b in zip(g_ref, g_once):
        assert a.dtype == torch.float32 and torch.equal(a, b)
    weights = {id(p) for p in m.parameters() if p.ndim == 2 and p is not m.embedding.weight}
    assert weights <= set(copies)              # every linear weight went through the copy
    assert len(uses) > 2 * len(copies)         # and was used many times (chunks, recomputes)
    assert M._STEP_CASTS["cache"] is None     # the scope is closed
