"""Benchmark of the Stack attention operators on one MI355X.

Headline (BASELINE.json metric): dense gated forward+backward TFLOP/s at
cfg2 (bf16, B1 H8 N=Q=4096 D128 b128, causal), plus the paged sparse top-k
forward at cfg4 (bf16, B1 H8, 1,048,576 tokens in 128-token pages behind a
random page table, 16 tail queries, D128 b128, top-64) in GB/s and ms.

A step is one forward+backward (dense) or one forward (sparse) over inputs
already resident in HBM. Timing: W untimed warmup steps, then K steps
bracketed by torch.cuda.synchronize(); per-step HIP events (on the stream
the kernels run on) give the per-step durations. Prints ONE JSON line.
"""
import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "dense fwd+bwd TFLOP/s @N=4096 bf16; sparse fwd GB/s+ms @1M ctx topk=64"
MFMA_BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA (AMD published)
HBM_PEAK_GBS = 8000.0            # MI355X HBM3E


def parse():
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU oracle timing")
    p.add_argument("--no-sparse", action="store_true", help="skip the cfg4 sparse measurement")
    p.add_argument("--cpu-seconds", type=float, default=20.0, help="budget of the CPU baseline sample")
    p.add_argument("--no-model", action="store_true", help="skip the cfg5 Stack model training step")
    p.add_argument("--model-steps", type=int, default=20, help="timed cfg5 training steps")
    p.add_argument("--dense-rows", choices=("causal", "last"), default="causal",
                   help="diagnostic: 'last' puts every cfg2 query at the last position (all keys visible, "
                        "no causal structure, twice the work); the headline uses 'causal'")
    return p.parse_args()


def profiled_traffic():
    """HBM bytes per step of the dense and sparse paths, from the calibrated
    FETCH_SIZE/WRITE_SIZE summary committed under profiles/ (None if absent)."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic_cfg2_dense_cfg4_sparse.md")
    found = {}
    try:
        for line in open(path):
            parts = line.split()
            if len(parts) == 2 and parts[0] == "traffic" and "=" in parts[1]:
                key, value = parts[1].split("=")
                found[key] = int(value)
    except OSError:
        pass
    return found.get("dense_step_bytes"), found.get("sparse_step_bytes")


def finite(x, digits=4):
    """A device scalar as a JSON-safe float (None when not finite)."""
    x = float(x)
    return round(x, digits) if math.isfinite(x) else None


def timed_steps(step, warmup, steps, torch):
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    wall0 = time.perf_counter()
    for begin, end in events:
        begin.record()
        step()
        end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    per = [b.elapsed_time(e) for b, e in events]
    return per, wall


def bench_dense(args, torch, device):
    from exploration_amd import dense_attention
    from exploration_amd.workloads import CFG2, dense_config, dense_flops, dense_forward_flops

    q, k, v, pos, do, b = dense_config(CFG2, device=device)
    if args.dense_rows == "last":
        pos = torch.full_like(pos, k.shape[1] - 1)
    q, k, v = (t.requires_grad_() for t in (q, k, v))
    flops = dense_flops(pos, k.shape[1], q.shape[2], q.shape[3])
    fwd_flops = dense_forward_flops(pos, k.shape[1], q.shape[2], q.shape[3])
    phase = {"fwd": [], "bwd": []}

    def step(record=None):
        q.grad = k.grad = v.grad = None
        if record is not None:
            e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
            e0.record()
        out = dense_attention(q, k, v, pos, b)
        if record is not None:
            e1.record()
        out.backward(do)
        if record is not None:
            e2.record()
            record.append((e0, e1, e2))

    per, wall = timed_steps(step, args.warmup, args.steps, torch)
    # phase split (separate pass so the headline timing has no extra events)
    marks = []
    for _ in range(max(3, args.steps // 2)):
        step(marks)
    torch.cuda.synchronize()
    fwd_ms = statistics.median(a.elapsed_time(b_) for a, b_, _ in marks)
    bwd_ms = statistics.median(b_.elapsed_time(c) for _, b_, c in marks)
    ms = sum(per) / len(per)
    med = statistics.median(per)
    tflops = flops / (ms * 1e-3) / 1e12
    return {
        "ms_mean": ms, "ms_median": med, "ms_min": min(per), "wall_s": wall, "flops": flops,
        "tflops": tflops, "fwd_ms": fwd_ms, "bwd_ms": bwd_ms,
        "fwd_tflops": fwd_flops / (fwd_ms * 1e-3) / 1e12,
        "bwd_tflops": (flops - fwd_flops) / (bwd_ms * 1e-3) / 1e12,
        "peak_mem_gib": torch.cuda.max_memory_allocated() / 2**30,
    }


def bench_sparse(args, torch, device):
    from exploration_amd import sparse_attention
    from exploration_amd.workloads import CFG4, planted_sparse, sparse_bytes

    c = dict(CFG4)
    q, cache, pos, expected = planted_sparse(**c, device=device)
    torch.cuda.synchronize()
    out, sel = sparse_attention(q, cache, pos, c["block"], c["topk"], return_selection=True)
    exact = bool(torch.equal(sel["indices"], expected))
    nbytes = sparse_bytes(pos, sel["indices"], c["heads"], c["dim"], c["block"], 2)
    scan_bytes = c["heads"] * ((c["length"] - 1) // c["block"] - 1) * c["block"] * c["dim"] * 2

    def step():
        sparse_attention(q, cache, pos, c["block"], c["topk"])

    per, wall = timed_steps(step, args.warmup, args.steps, torch)
    ms = sum(per) / len(per)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"ms_mean": ms, "ms_median": statistics.median(per), "ms_min": min(per), "wall_s": wall,
            "bytes": nbytes, "scan_bytes": scan_bytes, "gbs": gbs, "ids_exact": exact}


# configs/stack_100m.json "runtime" (the reference's execution settings)
CFG5_RUNTIME = {"checkpoint_chunks": True, "encoder_chunk": 1024, "query_chunk": 0, "loss_chunk": 128}
# the same with whole-sequence chunks: one encoder chunk per layer, one dense
# operator call per step, one loss chunk (the chunks bound temporaries that
# the HIP operator never allocates; the math is chunk-invariant)
CFG5_RUNTIME_WHOLE = {"checkpoint_chunks": True, "encoder_chunk": 8192, "query_chunk": 8192, "loss_chunk": 8192}


def bench_model(args, torch, device):
    """cfg5: one training step of a stack_100m-shaped model (random init, bf16
    autocast, AdamW, checkpointed chunks) on uniform token ids, batch 1,
    length 8192, every position supervised; tokens/s over the timed steps
    (the reference engine's figure, st/runtime/engine.py:192). With the
    config's runtime settings the step runs eagerly first, then captured into
    one HIP graph and replayed (``GraphedStep``): ``tokens_per_s`` is the
    graphed figure. ``whole_chunks`` repeats the graphed step with
    whole-sequence chunks."""
    from exploration_amd.model import STACK_100M, build_model
    from exploration_amd.train import GraphedStep, make_optimizer, synthetic_lm_batch, train_step

    length = 8192
    ids, targets = synthetic_lm_batch(STACK_100M["vocab_size"], length, batch=1, seed=0, device=device)

    def graphed_run(model, opt):
        graphed = GraphedStep(model, opt, ids, targets, warmup=1)
        seen = []

        def replay():
            seen.append(graphed(ids, targets)[0].clone())

        per, wall = timed_steps(replay, 2, args.model_steps, torch)
        loss, _, count = graphed(ids, targets)
        if int(count) == 0:
            raise ValueError("batch has no supervised tokens")
        bad = int((~torch.isfinite(torch.stack(seen))).sum())
        return per, wall, finite(loss), bad

    torch.manual_seed(0)
    model = build_model(STACK_100M, execution=CFG5_RUNTIME, device=device)
    opt = make_optimizer(model, capturable=True)
    losses = []

    def eager():
        losses.append(train_step(model, opt, ids, targets, width=length)[0])

    per_e, wall_e = timed_steps(eager, 3, args.model_steps, torch)
    per, wall, loss, bad = graphed_run(model, opt)
    ms, ms_e = sum(per) / len(per), sum(per_e) / len(per_e)
    chunk = model._chunk_size(length)
    result = {"tokens_per_s": length / (ms * 1e-3), "ms_mean": ms, "ms_median": statistics.median(per),
              "wall_s": wall, "steps": args.model_steps, "warmup": 3, "graphed": True, "runtime": CFG5_RUNTIME,
              "eager_tokens_per_s": length / (ms_e * 1e-3), "eager_ms_mean": ms_e,
              "params": sum(p.numel() for p in model.parameters()),
              "dense_calls_per_step": -(-(length - 1) // chunk), "query_chunk": chunk,
              "loss_first": finite(losses[0]), "loss_last": loss, "nonfinite_steps": bad}
    del opt
    result["decode"] = bench_decode(model, torch)
    del model
    torch.cuda.empty_cache()
    torch.manual_seed(0)
    whole = build_model(STACK_100M, execution=CFG5_RUNTIME_WHOLE, device=device)
    opt = make_optimizer(whole, capturable=True)
    first = train_step(whole, opt, ids, targets, width=length)[0]  # same init and batch: same first loss
    per_w, wall_w, loss_w, bad_w = graphed_run(whole, opt)
    ms_w = sum(per_w) / len(per_w)
    result["whole_chunks"] = {"runtime": CFG5_RUNTIME_WHOLE, "tokens_per_s": round(length / (ms_w * 1e-3), 1),
                              "ms_mean": round(ms_w, 4), "ms_median": round(statistics.median(per_w), 4),
                              "wall_s": round(wall_w, 4), "dense_calls_per_step": 1,
                              "loss_first": finite(first), "loss_last": loss_w, "nonfinite_steps": bad_w}
    return result


def bench_decode(model, torch, context=131072, queries=16):
    """cfg5 tail: the trained model in bf16, streaming prefill of a 131,072-token
    prompt into an HBM page cache, then the sparse read (top-64 of 8,192
    blocks) for the 16 tail positions; decode = one iter_logits pass."""
    from exploration_amd.inference import InferenceSession
    from exploration_amd.train import synthetic_lm_batch

    model = model.to(torch.bfloat16).eval()
    ids, _ = synthetic_lm_batch(model.lm_head.out_features, context, batch=1, seed=1)
    positions = torch.arange(context - queries, context)[None]
    with InferenceSession(model) as session:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        session.prefill(ids, positions)
        torch.cuda.synchronize()
        prefill_s = time.perf_counter() - t0

        def decode():
            for _ in session.iter_logits():
                pass

        per, _ = timed_steps(decode, 2, 10, torch)
        plan = session.plan.to_dict()
    return {"context": context, "queries": queries, "topk": model.topk, "cache": plan["cache"],
            "prefill_s": prefill_s, "prefill_tokens_per_s": context / prefill_s,
            "decode_ms_mean": sum(per) / len(per), "decode_ms_median": statistics.median(per)}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_seconds(run, warmup, reps):
    """perf_counter median of ``reps`` runs after ``warmup`` untimed ones
    (the reference harness defaults are 3 and 10, st/tools/benchmark.py:66-67)."""
    for _ in range(warmup):
        run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def cpu_baseline(budget_s, torch):
    """The oracle's restatement of the reference's CPU paths, timed on this
    host's cores: cfg1 (B2 H4 N=Q=512 D64 b64, fp32, arange positions, seed 0)
    forward+backward in the eager Q x N form (st/tools/benchmark.py:27-43; the
    reported value) and in the bounded-memory chunked form with q_chunk 32 and
    kv_chunk 1024 (st/ops/attention.py:51-139), then one of cfg2's eight heads
    (N=Q=4096 D128 b128, fp32) in the eager form, if the budget allows."""
    from exploration_amd.workloads import CFG1, dense_config, dense_flops, dense_inputs
    from oracle import dense as od

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)

    def fwd_bwd(q, k, v, do, forward):
        def run():
            qg, kg, vg = (t.detach().requires_grad_() for t in (q, k, v))
            forward(qg, kg, vg).backward(do)
        return run

    q, k, v, pos, do, b = dense_config(CFG1)
    flops = dense_flops(pos, CFG1["length"], CFG1["heads"], CFG1["dim"])
    t0 = time.perf_counter()
    eager = _median_seconds(fwd_bwd(q, k, v, do, lambda a, c, e: od.eager_attention(a, c, e, pos, b)), 3, 10)
    chunked = _median_seconds(
        fwd_bwd(q, k, v, do, lambda a, c, e: od.chunked_attention(a, c, e, pos, b, 32, 1024)), 3, 10)
    line = {"value": flops / eager / 1e12, "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "cpu": _cpu_model(),
            "sample": "cfg1: B2 H4 N=Q=512 D64 b64 fp32, arange positions, q/k/v/dO ~ N(0,1) seed 0; "
                      "oracle eager forward+backward (Q x N form), 3 warmups, median of 10",
            "seconds_per_step": eager, "flop_per_step": flops,
            "chunked": {"value": flops / chunked / 1e12, "unit": "TFLOP/s", "seconds_per_step": chunked,
                        "q_chunk": 32, "kv_chunk": 1024,
                        "sample": "cfg1, oracle chunked bounded-memory forward+backward, 3 warmups, median of 10"}}
    if time.perf_counter() - t0 < budget_s:
        q, k, v, pos, do = dense_inputs(1, 4096, 4096, 1, 128, torch.float32, seed=0, scale=1 / math.sqrt(128))
        flops2 = dense_flops(pos, 4096, 1, 128)
        run = fwd_bwd(q, k, v, do, lambda a, c, e: od.eager_attention(a, c, e, pos, 128))
        first = time.perf_counter()
        run()
        reps = max(1, min(10, int((budget_s - (time.perf_counter() - t0)) / max(time.perf_counter() - first, 1e-3))))
        sec = _median_seconds(run, 2, reps)
        line["cfg2_one_head"] = {"value": flops2 / sec / 1e12, "unit": "TFLOP/s", "seconds_per_step": sec,
                                 "sample": f"cfg2 restricted to 1 of 8 heads (B1 H1 N=Q=4096 D128 b128 fp32, "
                                           f"causal), oracle eager forward+backward, 3 warmups, median of {reps}"}
    return line


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: multi-GPU paths are out of scope (asked for --gpus {args.gpus})",
              file=sys.stderr)
        sys.exit(2)
    import torch
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    dense = bench_dense(args, torch, device)
    sparse = None if args.no_sparse else bench_sparse(args, torch, device)
    model = None
    if not args.no_model:
        try:
            model = bench_model(args, torch, device)
        except Exception as exc:  # the headline line must still be printed
            print(f"cfg5 leg failed: {exc!r}", file=sys.stderr, flush=True)
            model = {"error": repr(exc)}
    cpu = None if args.no_cpu_baseline else cpu_baseline(args.cpu_seconds, torch)
    traffic = profiled_traffic()
    line = {
        "metric": METRIC, "value": round(dense["tflops"], 3), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(dense["ms_mean"], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "cfg2: dense gated attention forward+backward, bf16, B1 H8 N=Q=4096 D128 "
                               "block 128, " + ("causal" if args.dense_rows == "causal" else
                                                "every query at position 4095 (diagnostic)")
                               + ", q/k/v ~ N(0,1)/sqrt(128), dO ~ N(0,1)",
                   "global_batch": 1, "seq_len": 4096, "heads": 8, "head_dim": 128, "block_size": 128,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": "dense forward+backward, one step (dense_fwd_fast, "
                     "dense_fwd_merge, dense_bwd_dq_fast, dense_bwd_dkv_fast, dense_bwd_merge)",
                     "achieved": round(dense["tflops"], 3), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(dense["tflops"] / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": traffic[0],
                     "traffic_unit": "bytes per step (calibrated FETCH_SIZE + WRITE_SIZE)",
                     "algorithmic_flop": dense["flops"]},
        "dense": {k: (round(v, 4) if isinstance(v, float) else v) for k, v in dense.items()},
        "cpu_baseline": cpu,
    }
    if sparse is not None:
        line["sparse"] = {
            "workload": "cfg4: paged sparse top-k forward, bf16, B1 H8, 1,048,576 tokens in 128-token pages "
                        "(random page table), 16 tail queries, D128 block 128, top-64, 64 planted blocks/query",
            "value": round(sparse["gbs"], 2), "unit": "GB/s", "ms": round(sparse["ms_mean"], 4),
            "ids_bit_exact": sparse["ids_exact"],
            "roofline": {"bound": "hbm", "achieved": round(sparse["gbs"], 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(sparse["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic[1],
                         "traffic_unit": "bytes per forward (calibrated FETCH_SIZE + WRITE_SIZE)",
                         "algorithmic_bytes": sparse["bytes"]},
            **{k: (round(v, 4) if isinstance(v, float) else v) for k, v in sparse.items()},
        }
    if model is not None:
        line["cfg5"] = {
            "workload": "cfg5: stack_100m-shaped model (vocab 256, dim 1024, H16 D64, b16, arch Lx7,G, ffn 4.0), "
                        "random init, bf16 autocast, AdamW, batch 1, length 8192, uniform token ids, next-token "
                        "targets at every position",
            "metric": "training tokens/s", "value": round(model["tokens_per_s"], 1) if "tokens_per_s" in model else None,
            "unit": "tokens/s",
            **{k: (round(v, 4) if isinstance(v, float) else v) for k, v in model.items()},
        }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
