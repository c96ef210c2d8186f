"""One training step of the Stack model (the reference engine's inner loop,
``st/runtime/engine.py:150-180``), single GPU: bf16 autocast, SUM loss over
the supervised tokens divided by their count, gradient clipping, AdamW with
the reference's betas (0.9, 0.95) and defaults (lr 3e-4, weight decay 0.01,
clip 1.0; ``engine.py:88-119``, ``cli.py:71-73``).

The reference's checks that the batch has supervised tokens and that the
loss is finite (``engine.py:170-175``) read device values back every step;
here they are left to the caller (``check_step``). With ``width`` given, a
step makes no host synchronisation at all, and ``GraphedStep`` captures the
whole step (forward, backward, clipping, optimizer) into one HIP graph: the
model's ~20,000 small kernels per step then cost one graph launch instead
of as many launches from Python.
"""
import torch


def make_optimizer(model, lr=3e-4, weight_decay=0.01, capturable=False):
    fused = next(model.parameters()).is_cuda
    return torch.optim.AdamW(model.parameters(), lr=lr, betas=(0.9, 0.95), weight_decay=weight_decay, fused=fused,
                             capturable=capturable and fused)


def train_step(model, optimizer, ids, targets, sup=None, clip_grad=1.0, precision="bf16", width=None,
               autocast_cache=True):
    """Forward loss, backward, clip, optimizer step. Returns device tensors
    (mean loss, gradient norm, supervised count)."""
    optimizer.zero_grad(set_to_none=True)
    with torch.autocast(ids.device.type, dtype=torch.bfloat16, enabled=precision == "bf16",
                        cache_enabled=autocast_cache):
        result = model.forward_loss(ids, targets, sup, width=width)
        loss = result["loss_sum"] / result["count"]
    loss.backward()
    norm = torch.nn.utils.clip_grad_norm_(model.parameters(), clip_grad)
    optimizer.step()
    return loss.detach(), norm.detach(), result["count"]


class GraphedStep:
    """``train_step`` captured once into a HIP graph and replayed.

    ``ids``/``targets`` fix the batch shape; each call copies the new batch
    into the captured input buffers and replays the graph. Every position
    may be supervised (the captured width is the sequence length), so any
    targets of that shape are valid. The optimizer must be capturable
    (``make_optimizer(model, capturable=True)``). Construction runs
    ``warmup`` eager steps on a side stream first (they update the model
    like any step), then captures one step without running it. Returns the
    same device tensors as ``train_step``; they are overwritten by the next
    call, which returns after the replay has finished.

    The model's step is written so that the graph holds no library kernel
    with a decoupled look-back (device-wide sort, unique, select or a
    one-row scan): such kernels spin on flags other workgroups set and have
    hung in replays here."""

    def __init__(self, model, optimizer, ids, targets, clip_grad=1.0, precision="bf16", warmup=3):
        if not ids.is_cuda:
            raise ValueError("graph capture needs the model and batch on the GPU")
        if not all(g.get("capturable", False) for g in optimizer.param_groups):
            raise ValueError("the optimizer must be built with capturable=True")
        self.ids, self.targets = ids.clone(), targets.clone()
        options = dict(clip_grad=clip_grad, precision=precision, width=ids.shape[1], autocast_cache=False)

        def step():
            return train_step(model, optimizer, self.ids, self.targets, **options)

        main = torch.cuda.current_stream(ids.device)
        side = torch.cuda.Stream(ids.device)
        side.wait_stream(main)
        with torch.cuda.stream(side):
            for _ in range(max(1, warmup)):
                step()
        main.wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.outputs = step()

    def __call__(self, ids, targets):
        self.ids.copy_(ids)
        self.targets.copy_(targets)
        self.graph.replay()
        # one replay at a time: replays queued back to back have hung here in
        # a library kernel whose workgroups spin on each other's flags (a
        # look-back scan); waiting costs a fraction of a percent of a step
        torch.cuda.current_stream(self.ids.device).synchronize()
        return self.outputs


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


def main(argv=None):
    """``python -m exploration_amd.train``: the cfg5 training step (a
    stack_100m-shaped model, random init, batch 1, length 8192, every position
    supervised) as one HIP graph, replayed ``--steps`` times; prints tokens/s.
    ``--whole-chunks`` uses whole-sequence encoder, read and loss chunks
    instead of the config's (1024, auto, 128)."""
    import argparse
    import time

    from .model import STACK_100M, build_model

    p = argparse.ArgumentParser(description=main.__doc__)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--length", type=int, default=8192)
    p.add_argument("--whole-chunks", action="store_true")
    args = p.parse_args(argv)
    n = args.length
    runtime = ({"checkpoint_chunks": True, "encoder_chunk": n, "query_chunk": n, "loss_chunk": n}
               if args.whole_chunks else
               {"checkpoint_chunks": True, "encoder_chunk": 1024, "query_chunk": 0, "loss_chunk": 128})
    torch.manual_seed(0)
    model = build_model(STACK_100M, execution=runtime, device="cuda")
    opt = make_optimizer(model, capturable=True)
    ids, targets = synthetic_lm_batch(STACK_100M["vocab_size"], n, batch=1, seed=0, device="cuda")
    step = GraphedStep(model, opt, ids, targets, warmup=1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        loss = step(ids, targets)[0]
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    print(f"runtime {runtime}: {dt * 1e3:.2f} ms per step, {n / dt:.0f} tokens/s, loss {float(loss):.4f}",
          flush=True)


if __name__ == "__main__":
    main()
