"""Dense gated attention: HIP kernels against the oracle on identical inputs.

Cases follow the reference's GPU validation matrix
(st/tools/validate.py:75-118: seed 772, q [2,5,2,D], positions with early,
block-boundary, last and padding rows) plus the BASELINE configurations:
cfg2 (bf16, B1 H8 N=Q=4096 D128 b128) at full size, cfg3 (fp32 ragged tail),
and a cfg5-shaped chunk (b16 D64). Tolerances: tests/helpers.py.
"""
import math

import pytest
import torch

from exploration_amd import _lib, dense_attention, launch_report
from exploration_amd.attention import dense_forward_stats
from exploration_amd.workloads import CFG1, CFG2, CFG3, dense_config
from oracle import dense as od
from tests.helpers import assert_close, error_metrics

pytestmark = pytest.mark.gpu

VALIDATE_CASES = [(17, 2, 16), (129, 16, 32), (257, 32, 64), (193, 64, 96), (385, 128, 128),
                  (131, 16, 256), (385, 128, 256)]
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _validate_case(n, b, d, dtype, seed=772):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(2, 5, 2, d, generator=g).to(dtype)
    k = torch.randn(2, n, 2, d, generator=g).to(dtype)
    v = torch.randn(2, n, 2, d, generator=g).to(dtype)
    probe = torch.randn(2, 5, 2, d, generator=g).to(dtype)
    pos = torch.tensor([[0, b - 1, min(2 * b + 1, n - 1), n - 1, -1], [n - 1, 0, n // 2, -1, n - 2]])
    return q, k, v, pos, probe


def _check_dense(q, k, v, pos, probe, b, device, dtype, oracle_device="cpu", label=""):
    """Forward output, saved statistics and all input gradients against the
    oracle (float64 on CPU, float32 when run on the GPU for large shapes)."""
    work = torch.float64 if oracle_device == "cpu" else torch.float32
    qo, ko, vo = (t.to(oracle_device, work) for t in (q, k, v))
    po, go = pos.to(oracle_device), probe.to(oracle_device, work)
    stats = od.forward_stats(qo, ko, vo, po, b)
    grads = od.backward_explicit(qo, ko, vo, po, b, go, stats)

    qg, kg, vg = (t.to(device).requires_grad_() for t in (q, k, v))
    out = dense_attention(qg, kg, vg, pos.to(device), b)
    dq, dk, dv = torch.autograd.grad(out, (qg, kg, vg), probe.to(device))
    hip_stats = dense_forward_stats(qg.detach(), kg.detach(), vg.detach(), pos.to(device), b)
    torch.cuda.synchronize()
    report = {name: error_metrics(a, e) for name, a, e in
              zip(("out", "dq", "dk", "dv"), (out, dq, dk, dv), (stats[0],) + tuple(grads))}
    print(f"{label} {dtype} errors {report}", flush=True)
    assert_close(out, stats[0], dtype, f"{label} out")
    assert torch.equal(hip_stats[0], out.detach())
    stat_dtype = torch.float32 if dtype == torch.float32 else dtype
    for name, a, e in zip(("rc", "pr", "zr", "z"), hip_stats[1:], stats[1:]):
        assert_close(a, e, stat_dtype, f"{label} {name}")
    for name, a, e in zip(("dq", "dk", "dv"), (dq, dk, dv), grads):
        assert_close(a, e, dtype, f"{label} {name}")


@pytest.mark.parametrize("dtype", DTYPES, ids=str)
@pytest.mark.parametrize("n,b,d", VALIDATE_CASES)
def test_validation_matrix(device, n, b, d, dtype):
    print(f"dense case n={n} b={b} d={d} {dtype}", flush=True)
    q, k, v, pos, probe = _validate_case(n, b, d, dtype)
    _check_dense(q, k, v, pos, probe, b, device, dtype, label=f"n={n} b={b} d={d}")


def test_cfg1_fp32_causal(device):
    """cfg1: fp32, B2 H4, N=Q=512 (positions arange), D=64, b=64, q/k/v/dO ~
    N(0,1) from seed 0 (the reference's CPU benchmark shape,
    st/tools/benchmark.py:27-43): forward, statistics and gradients against
    the float64 oracle."""
    print("dense cfg1", flush=True)
    q, k, v, pos, do, b = dense_config(CFG1)
    assert pos.shape == (2, 512) and pos[1].tolist() == list(range(512))
    _check_dense(q, k, v, pos, do, b, device, torch.float32, label="cfg1")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
@pytest.mark.parametrize("d", [40, 200, 20, 33, 130])
def test_head_dim_envelope(device, d, dtype):
    """Any head_dim up to 256 (the reference pads D inside its kernel,
    st/ops/kernels/dense.py:210): multiples of 8 run directly, others through
    zero-padded copies in the workspace; the scale stays 1/sqrt(head_dim)."""
    print(f"dense head_dim {d} {dtype}", flush=True)
    g = torch.Generator().manual_seed(40 + d)
    n, b = 300, 32
    q = torch.randn(2, 70, 2, d, generator=g).to(dtype)
    k = torch.randn(2, n, 2, d, generator=g).to(dtype)
    v = torch.randn(2, n, 2, d, generator=g).to(dtype)
    probe = torch.randn(2, 70, 2, d, generator=g).to(dtype)
    pos = torch.randint(-1, n, (2, 70), generator=g)
    _check_dense(q, k, v, pos, probe, b, device, dtype, label=f"d={d}")


def test_cfg3_fp32_ragged_tail(device):
    """cfg3: fp32, B1 H4, N=385, queries at 380..384, D=128, b=128; the last
    key block holds one token."""
    print("dense cfg3", flush=True)
    q, k, v, pos, do, b = dense_config(CFG3)
    assert pos.tolist() == [[380, 381, 382, 383, 384]]
    _check_dense(q, k, v, pos, do, b, device, torch.float32, label="cfg3")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
def test_unsorted_positions_and_padding(device, dtype):
    """Arbitrary (unsorted, repeated, padding) positions over several query
    tiles, batch 2, N not a multiple of any tile."""
    print(f"dense unsorted {dtype}", flush=True)
    g = torch.Generator().manual_seed(5)
    n, b, d = 1000, 32, 64
    q = torch.randn(2, 150, 3, d, generator=g).to(dtype)
    k = torch.randn(2, n, 3, d, generator=g).to(dtype)
    v = torch.randn(2, n, 3, d, generator=g).to(dtype)
    probe = torch.randn(2, 150, 3, d, generator=g).to(dtype)
    pos = torch.randint(-1, n, (2, 150), generator=g)
    _check_dense(q, k, v, pos, probe, b, device, dtype, label="unsorted")


FAST_CASES = [(64, 2), (64, 4), (64, 8), (64, 16), (64, 64), (64, 128), (128, 16), (128, 32), (128, 64),
              (128, 128)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=str)
@pytest.mark.parametrize("d,b", FAST_CASES)
def test_pipelined_path_block_sizes(device, d, b, dtype):
    """16-bit head_dim 64/128 (the pipelined kernels) at every block size:
    batch 2, 3 heads, 300 keys (a partial last key tile), 140 query rows
    (three 64-row tiles, the last partial) with unsorted positions, padding
    rows, a row at key 0 and rows past the last key."""
    print(f"dense pipelined d={d} b={b} {dtype}", flush=True)
    g = torch.Generator().manual_seed(11 + d + b)
    n, rows = 300, 140
    q = torch.randn(2, rows, 3, d, generator=g).to(dtype)
    k = torch.randn(2, n, 3, d, generator=g).to(dtype)
    v = torch.randn(2, n, 3, d, generator=g).to(dtype)
    probe = torch.randn(2, rows, 3, d, generator=g).to(dtype)
    pos = torch.randint(-1, n + 40, (2, rows), generator=g)
    pos[0, :4] = torch.tensor([0, -1, n - 1, n + 5])
    _check_dense(q, k, v, pos, probe, b, device, dtype, label=f"pipelined d={d} b={b}")


def test_cfg5_shaped_chunk(device):
    """cfg5 G-round shape: bf16, H16 D64 b16, 240 supervised query positions
    over N=8192 keys (oracle in float32 on the GPU)."""
    print("dense cfg5 chunk", flush=True)
    g = torch.Generator().manual_seed(8)
    n, d, b = 8192, 64, 16
    q = (torch.randn(1, 240, 16, d, generator=g) / 8).to(torch.bfloat16)
    k = (torch.randn(1, n, 16, d, generator=g) / 8).to(torch.bfloat16)
    v = torch.randn(1, n, 16, d, generator=g).to(torch.bfloat16)
    probe = torch.randn(1, 240, 16, d, generator=g).to(torch.bfloat16)
    pos = torch.sort(torch.randperm(n, generator=g)[:240]).values[None]
    _check_dense(q, k, v, pos, probe, b, device, torch.bfloat16, oracle_device=device, label="cfg5")


@pytest.mark.parametrize("heads,rows,pieces", [(16, 240, 8), (32, 256, 4), (48, 256, 2)])
def test_few_row_tiles_run_in_pieces(device, heads, rows, pieces):
    """Launches with few 128-row tiles (B*H*tiles well below the compute
    units: the cfg5 read chunks) run every row tile's key range as up to
    eight pieces, forward and dQ, whose partials merge kernels combine:
    consecutive positions near the end of N=8192 keys (D64 b16, bf16), with
    a padding row and a row at key 0. The launch record shows the piece
    count (workgroups = pieces x row tiles x heads); oracle in float32 on
    the GPU."""
    print(f"dense pieces heads={heads} rows={rows}", flush=True)
    g = torch.Generator().manual_seed(30 + heads)
    n, d, b = 8192, 64, 16
    q = (torch.randn(1, rows, heads, d, generator=g) / 8).to(torch.bfloat16)
    k = (torch.randn(1, n, heads, d, generator=g) / 8).to(torch.bfloat16)
    v = torch.randn(1, n, heads, d, generator=g).to(torch.bfloat16)
    probe = torch.randn(1, rows, heads, d, generator=g).to(torch.bfloat16)
    pos = torch.arange(n - 100 - rows, n - 100)[None].clone()
    pos[0, 0], pos[0, 1] = -1, 0
    _check_dense(q, k, v, pos, probe, b, device, torch.bfloat16, oracle_device=device, label=f"pieces{pieces}")
    tiles = -(-rows // 128)
    fwd = [r for r in launch_report() if r.get("kernel") == "dense_fwd_fast" and r.get("head_dim") == 64
           and r.get("block_size") == 16 and r.get("mode") == "slot"]
    assert fwd and fwd[-1]["workgroups"] == pieces * tiles * heads, fwd


@pytest.mark.parametrize("d,b,dtype", [(128, 32, torch.float16), (64, 128, torch.bfloat16), (64, 2, torch.bfloat16)],
                         ids=str)
def test_few_row_pieces_ragged(device, d, b, dtype):
    """The eight-piece path (6 row tiles for 256 compute units) with batch 2,
    3 heads, 130 query rows (a partial second row tile) at unsorted positions
    over 3,000 keys: padding rows, rows at key 0, rows past the last key, and
    pieces left without key tiles (oracle in float32 on the GPU)."""
    print(f"dense ragged pieces d={d} b={b} {dtype}", flush=True)
    g = torch.Generator().manual_seed(40 + d + b)
    n, rows = 3000, 130
    q = (torch.randn(2, rows, 3, d, generator=g) / math.sqrt(d)).to(dtype)
    k = (torch.randn(2, n, 3, d, generator=g) / math.sqrt(d)).to(dtype)
    v = torch.randn(2, n, 3, d, generator=g).to(dtype)
    probe = torch.randn(2, rows, 3, d, generator=g).to(dtype)
    pos = torch.randint(-1, n + 50, (2, rows), generator=g)
    pos[0, :5] = torch.tensor([0, -1, n - 1, n + 7, 1])
    pos[1, -3:] = torch.tensor([b, 2 * b - 1, 130])
    _check_dense(q, k, v, pos, probe, b, device, dtype, oracle_device=device, label=f"ragged d={d} b={b}")


def test_cfg2_full_size(device):
    """cfg2 at full size: bf16 B1 H8 N=Q=4096 D128 b128, causal; q/k/v ~
    N(0,1)/sqrt(128), dO ~ N(0,1) (oracle in float32 on the GPU)."""
    print("dense cfg2", flush=True)
    q, k, v, pos, do, b = dense_config(CFG2, device=device)
    _check_dense(q, k, v, pos, do, b, device, torch.bfloat16, oracle_device=device, label="cfg2")


def test_cfg2_every_row_at_the_last_position(device):
    """cfg2's tensors with every query at position 4095 (all keys visible, no
    causal structure: the `bench.py --dense-rows last` workload), in pair
    mode with equal-length row tiles (oracle in float32 on the GPU)."""
    print("dense cfg2 rows at the last position", flush=True)
    q, k, v, pos, do, b = dense_config(CFG2, device=device)
    pos = torch.full_like(pos, k.shape[1] - 1)
    _check_dense(q, k, v, pos, do, b, device, torch.bfloat16, oracle_device=device, label="cfg2-last")


@pytest.mark.parametrize("d,b", [(64, 32), (128, 64), (128, 128)])
def test_peaked_scores_bf16(device, d, b):
    """bf16 with blocks of 32+ keys, where the backward passes the (beta, eps)
    table to the dK/dV kernel as bf16 terms added by an MFMA: logits with a
    standard deviation of ~6 (peaked rows, large |beta| and eps), unsorted
    positions with padding rows and rows past the last key, a partial last
    key tile and a partial last row tile (oracle in float64 on the CPU)."""
    print(f"dense peaked d={d} b={b}", flush=True)
    g = torch.Generator().manual_seed(31 + d + b)
    n, rows = 520, 140
    q = (torch.randn(2, rows, 2, d, generator=g) * 2.5).to(torch.bfloat16)
    k = (torch.randn(2, n, 2, d, generator=g) * 2.5).to(torch.bfloat16)
    v = torch.randn(2, n, 2, d, generator=g).to(torch.bfloat16)
    probe = torch.randn(2, rows, 2, d, generator=g).to(torch.bfloat16)
    pos = torch.randint(-1, n + 20, (2, rows), generator=g)
    pos[1, :3] = torch.tensor([n - 1, -1, 0])
    _check_dense(q, k, v, pos, probe, b, device, torch.bfloat16, label=f"peaked d={d} b={b}")


@pytest.mark.parametrize("d,b,tiles", [(64, 64, 33), (128, 128, 32), (128, 16, 34)])
def test_causal_pair_mode(device, d, b, tiles):
    """Causal rows over enough 128-row tiles (B1 H8) that the forward pairs
    row tiles n-1-j and j across workgroups, splitting some long tiles: odd
    and even tile counts, with and without splits (oracle in float32 on the
    GPU)."""
    print(f"dense pair mode d={d} b={b} tiles={tiles}", flush=True)
    n = 128 * tiles
    g = torch.Generator().manual_seed(21 + tiles)
    q = (torch.randn(1, n, 8, d, generator=g) / math.sqrt(d)).to(torch.bfloat16)
    k = (torch.randn(1, n, 8, d, generator=g) / math.sqrt(d)).to(torch.bfloat16)
    v = torch.randn(1, n, 8, d, generator=g).to(torch.bfloat16)
    probe = torch.randn(1, n, 8, d, generator=g).to(torch.bfloat16)
    pos = torch.arange(n)[None]
    _check_dense(q, k, v, pos, probe, b, device, torch.bfloat16, oracle_device=device, label=f"pair{tiles}")


def test_native_library_is_the_path(device):
    """The kernels ran from the in-tree library, bound to torch's HIP runtime."""
    q = torch.randn(1, 8, 1, 64, device=device)
    out = dense_attention(q, q, q, torch.arange(8, device=device)[None], 4)
    torch.cuda.synchronize()
    assert out.shape == q.shape
    report = launch_report()
    assert any(r["kernel"] == "dense_fwd" and r["path"] == "hip" for r in report)
    native = [r for r in report if r["kernel"].startswith("dense_fwd") and "tile_m" in r]
    assert native and all(r["vgprs"] > 0 and r["workgroups"] > 0 for r in native), native
    runtimes = _lib.hip_runtimes_mapped()
    assert len(runtimes) == 1, runtimes
    maps = open("/proc/self/maps").read()
    assert _lib.LIB_PATH in maps
