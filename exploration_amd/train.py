"""One training step of the Stack model (the reference engine's inner loop,
``st/runtime/engine.py:150-180``), single GPU: bf16 autocast, SUM loss over
the supervised tokens divided by their count, gradient clipping, AdamW with
the reference's betas (0.9, 0.95) and defaults (lr 3e-4, weight decay 0.01,
clip 1.0; ``engine.py:88-119``, ``cli.py:71-73``).

Unlike the reference, a step makes no host synchronisation: the reference's
checks that the batch has supervised tokens and that the loss is finite
(``engine.py:170-175``) read device values back every step; here they are
left to the caller (``check_step``).
"""
import torch


def make_optimizer(model, lr=3e-4, weight_decay=0.01):
    fused = next(model.parameters()).is_cuda
    return torch.optim.AdamW(model.parameters(), lr=lr, betas=(0.9, 0.95), weight_decay=weight_decay, fused=fused)


def train_step(model, optimizer, ids, targets, sup=None, clip_grad=1.0, precision="bf16"):
    """Forward loss, backward, clip, optimizer step. Returns device tensors
    (mean loss, gradient norm, supervised count)."""
    optimizer.zero_grad(set_to_none=True)
    with torch.autocast(ids.device.type, dtype=torch.bfloat16, enabled=precision == "bf16"):
        result = model.forward_loss(ids, targets, sup)
        loss = result["loss_sum"] / result["count"]
    loss.backward()
    norm = torch.nn.utils.clip_grad_norm_(model.parameters(), clip_grad)
    optimizer.step()
    return loss.detach(), norm.detach(), result["count"]


def check_step(loss, count):
    """The reference's per-step guards (``engine.py:170-175``), on the host."""
    if int(count) == 0:
        raise ValueError("batch has no supervised tokens")
    if not bool(torch.isfinite(loss)):
        raise FloatingPointError("non-finite loss; optimizer step was applied before the check")


def synthetic_lm_batch(vocab, length, batch=1, seed=0, device="cpu"):
    """Uniform token ids over the vocabulary, next-token targets (last -100)."""
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(vocab, (batch, length), generator=g)
    targets = torch.roll(ids, -1, 1)
    targets[:, -1] = -100
    return ids.to(device), targets.to(device)
