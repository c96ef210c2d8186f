"""One training step of the Stack model (the reference engine's inner loop,
``st/runtime/engine.py:150-180``), single GPU: bf16 autocast, SUM loss over
the supervised tokens divided by their count, gradient clipping, AdamW with
the reference's betas (0.9, 0.95) and defaults (lr 3e-4, weight decay 0.01,
clip 1.0; ``engine.py:88-119``, ``cli.py:71-73``).

Guards (``engine.py:170-177``). Without ``width`` the step reads the
supervised count and the loss on the host before backward, as the reference
does: an empty batch raises ``ValueError``, a non-finite loss
``FloatingPointError``, and clipping raises on a non-finite gradient norm;
the optimizer step is never applied. With ``width`` given, a step makes no
host synchronisation at all: the same two conditions are evaluated on the
device and passed to the fused AdamW as its ``found_inf`` flag, which skips
the update of every parameter and moment (and the step count) on the device.
``GraphedStep`` captures that whole step (forward, backward, clipping,
optimizer) into one HIP graph: the model's thousands of small kernels per
step then cost one graph launch instead of as many launches from Python.
"""
import contextlib

import torch

from .model import weights_cast_once


def make_optimizer(model, lr=3e-4, weight_decay=0.01, capturable=False):
    fused = next(model.parameters()).is_cuda
    return torch.optim.AdamW(model.parameters(), lr=lr, betas=(0.9, 0.95), weight_decay=weight_decay, fused=fused,
                             capturable=capturable and fused)


def train_step(model, optimizer, ids, targets, sup=None, clip_grad=1.0, precision="bf16", width=None,
               autocast_cache=True):
    """Forward loss, backward, clip, optimizer step. Returns device tensors
    (mean loss, gradient norm, supervised count). With ``width`` the step
    is skipped on the device (no host check) when the count is zero or the
    loss is not finite."""
    optimizer.zero_grad(set_to_none=True)
    # without autocast's cast cache (graph capture), one cast per weight and
    # step for forward and backward (the checkpointed chunks' recomputes)
    with weights_cast_once() if not autocast_cache else contextlib.nullcontext():
        with torch.autocast(ids.device.type, dtype=torch.bfloat16, enabled=precision == "bf16",
                            cache_enabled=autocast_cache):
            result = model.forward_loss(ids, targets, sup, width=width)
            count = result["count"]
            if width is None and int(count) == 0:
                raise ValueError("global batch has no supervised tokens")
            loss = result["loss_sum"] / count
        if width is None:
            if not bool(torch.isfinite(loss.detach())):
                raise FloatingPointError("non-finite loss; optimizer step was not applied")
            loss.backward()
        else:
            ok = (count > 0) & torch.isfinite(loss.detach())
            loss.backward()
    if width is None:
        norm = torch.nn.utils.clip_grad_norm_(model.parameters(), clip_grad, error_if_nonfinite=True)
        optimizer.step()
        return loss.detach(), norm.detach(), count
    norm = torch.nn.utils.clip_grad_norm_(model.parameters(), clip_grad)
    if not _fused(optimizer):
        raise ValueError("a step without host checks needs the fused AdamW (make_optimizer on the GPU)")
    optimizer.found_inf = (~(ok & torch.isfinite(norm))).float()
    try:
        optimizer.step()
    finally:
        del optimizer.found_inf
    return loss.detach(), norm.detach(), count


def _fused(optimizer):
    return all(g.get("fused", False) for g in optimizer.param_groups)


class GraphedStep:
    """``train_step`` captured once into a HIP graph and replayed.

    ``ids``/``targets`` fix the batch shape; each call copies the new batch
    into the captured input buffers and replays the graph (stream-ordered,
    no host synchronisation). Every position may be supervised (the captured
    width is the sequence length), so any targets of that shape are valid; a
    batch with no supervised token or a non-finite loss leaves the model and
    the optimizer state unchanged (see ``train_step``). The optimizer must be
    capturable (``make_optimizer(model, capturable=True)``). Construction
    runs ``warmup`` eager steps on a side stream first (they update the model
    like any step), then captures one step without running it. Returns the
    same device tensors as ``train_step``; the next call overwrites them.

    The captured graph must hold kernel nodes only: construction raises
    ``RuntimeError`` if capture recorded a memset node. A memset node that
    a library records during capture (rocprim's partition/unique clears its
    selected-item counters with ``hipMemsetAsync``; the split reduction of a
    long row sum clears its semaphores) has not re-run reliably on replays
    on this platform, and the kernels behind it then read stale counters:
    an out-of-bounds write in the first case (a memory aperture fault), a
    drifting sum in the second. The model's step avoids every such op
    (``tests/test_model.py`` traces its aten ops); this check keeps it so."""

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
        self.graph = torch.cuda.CUDAGraph(keep_graph=True)
        with torch.cuda.graph(self.graph):
            self.outputs = step()
        self.node_types = graph_node_types(self.graph)
        memsets = self.node_types.get("memset", 0)
        if memsets:
            raise RuntimeError(f"the captured step holds {memsets} memset node(s); they do not replay "
                               f"reliably here ({self.node_types})")
        self.graph.instantiate()

    def __call__(self, ids, targets):
        self.ids.copy_(ids)
        self.targets.copy_(targets)
        self.graph.replay()
        return self.outputs


_NODE_TYPES = {0: "kernel", 1: "memcpy", 2: "memset", 3: "host", 4: "graph", 5: "empty", 6: "wait_event",
               7: "event_record", 8: "ext_semaphore_signal", 9: "ext_semaphore_wait", 10: "mem_alloc",
               11: "mem_free", 12: "memcpy_from_symbol", 13: "memcpy_to_symbol", 14: "batch_mem_op"}


def graph_node_types(graph):
    """Counts of the node types of a captured ``torch.cuda.CUDAGraph(keep_graph=True)``
    (``hipGraphGetNodes`` / ``hipGraphNodeGetType`` of the HIP runtime torch
    loaded; host calls only)."""
    import ctypes

    from ._lib import hip_runtimes_mapped

    runtimes = hip_runtimes_mapped()
    if len(runtimes) != 1:
        raise RuntimeError(f"expected one HIP runtime in the process, found {runtimes}")
    hip = ctypes.CDLL(runtimes[0])
    handle = ctypes.c_void_p(graph.raw_cuda_graph())
    n = ctypes.c_size_t(0)
    if hip.hipGraphGetNodes(handle, None, ctypes.byref(n)) != 0:
        raise RuntimeError("hipGraphGetNodes failed")
    nodes = (ctypes.c_void_p * max(1, n.value))()
    if hip.hipGraphGetNodes(handle, nodes, ctypes.byref(n)) != 0:
        raise RuntimeError("hipGraphGetNodes failed")
    counts = {}
    kind = ctypes.c_int(0)
    for i in range(n.value):
        if hip.hipGraphNodeGetType(ctypes.c_void_p(nodes[i]), ctypes.byref(kind)) != 0:
            raise RuntimeError("hipGraphNodeGetType failed")
        name = _NODE_TYPES.get(kind.value, str(kind.value))
        counts[name] = counts.get(name, 0) + 1
    return counts


def check_step(loss, count):
    """The reference's per-step guards (``engine.py:170-175``) for a step that
    ran without host checks (it was skipped on the device; this reports why)."""
    if int(count) == 0:
        raise ValueError("batch has no supervised tokens; the optimizer step was skipped")
    if not bool(torch.isfinite(loss)):
        raise FloatingPointError("non-finite loss; the optimizer step was skipped")


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
