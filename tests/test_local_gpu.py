"""The local blocks' fused window attention (exploration_amd.local) against
the same block's PyTorch path (the reference's computation,
st/models/blocks.py:102-179: rotary embedding, [previous ++ own] windows,
torch's scaled dot-product attention), which tests/test_model.py checks
against the float64 oracle on the CPU.

Output and the gradients of the input and of every parameter, fp32 (rtol
1e-5) and bf16 (rtol 2e-2 against the PyTorch path in fp32 on the same,
bf16-valued, parameters and inputs), over every instantiated (block,
head_dim):
chunks that fill their last block and chunks that do not, a chunk start
past zero, and with and without the previous block's halo.
"""
import copy

import pytest
import torch

import exploration_amd.model as M
from tests.helpers import assert_close

pytestmark = pytest.mark.gpu

SHAPES = [(16, 64, 4), (8, 64, 2), (4, 64, 3), (8, 32, 2), (4, 128, 1), (16, 128, 2), (32, 32, 3), (4, 32, 2), (8, 128, 1)]


def _block(dim, heads, b, device, dtype):
    torch.manual_seed(0)
    layer = M.HaloMemoryBlock(dim, heads, b, M.RotaryEmbedding(dim // heads), 2.0, 64).to(device, dtype)
    return layer


def _run(layer, x, previous, start, fused):
    layer.fused = fused
    layer.zero_grad(set_to_none=True)
    xi = x.detach().clone().requires_grad_()
    y = layer.forward_chunk(xi, previous, start)
    g = torch.randn(y.shape, generator=torch.Generator().manual_seed(5), dtype=torch.float32).to(y.device, y.dtype)
    (y.float() * g.float()).sum().backward()
    grads = {"x": xi.grad}
    grads.update({n: p.grad for n, p in layer.named_parameters()})
    return y.detach(), grads


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
@pytest.mark.parametrize("b,hd,heads", SHAPES)
@pytest.mark.parametrize("n,start,halo", [(96, 0, False), (83, 48, True), (37, 16, False), (5, 0, False)])
def test_fused_window_attention(device, b, hd, heads, n, start, halo, dtype):
    print(f"window attention b={b} hd={hd} heads={heads} n={n} start={start} halo={halo} {dtype}", flush=True)
    start = start // b * b
    dim = hd * heads
    layer = _block(dim, heads, b, device, dtype)
    gen = torch.Generator().manual_seed(b * 1000 + n)
    x = torch.randn(2, n, dim, generator=gen).to(device, dtype)
    previous = torch.randn(2, b, dim, generator=gen).to(device, dtype) if halo else None
    assert M.halo_supported(layer.qkv(layer.attn_norm(x)), b, hd)
    ref = copy.deepcopy(layer).float()
    want, gwant = _run(ref, x.float(), None if previous is None else previous.float(), start, fused=False)
    got, ggot = _run(layer, x, previous, start, fused=True)
    assert_close(got, want, dtype, "out")
    for name in gwant:
        assert_close(ggot[name], gwant[name], dtype, name)


@pytest.mark.parametrize("b,hd,heads", [(16, 64, 4), (8, 64, 2), (16, 128, 2)])
@pytest.mark.parametrize("n,start,halo", [(96, 0, False), (83, 48, True)])
def test_fused_window_attention_fp16(device, b, hd, heads, n, start, halo):
    """fp16 through the same kernels (MFMA at b 16, head_dim 64; VALU
    otherwise), against the PyTorch path in fp32."""
    test_fused_window_attention(device, b, hd, heads, n, start, halo, torch.float16)


def test_unsupported_shape_keeps_pytorch_path(device):
    """A head_dim without a kernel runs the PyTorch attention."""
    layer = _block(48, 2, 16, device, torch.float32)  # head_dim 24
    x = torch.randn(1, 40, 48, device=device)
    assert not M.halo_supported(layer.qkv(layer.attn_norm(x)), 16, 24)
    y = layer.forward_chunk(x)
    layer.fused = False
    torch.testing.assert_close(y, layer.forward_chunk(x))


def test_tables_built_under_inference_mode_serve_training(device):
    """The rotary tables are cached per shape; the first use may be an
    inference-mode prefill, and a later training step must still work."""
    from exploration_amd import local

    local._tables.clear()
    layer = _block(64, 1, 16, device, torch.float32)
    x = torch.randn(1, 40, 64, device=device)
    with torch.inference_mode():
        layer.forward_chunk(x)
    xi = x.clone().requires_grad_()
    layer.forward_chunk(xi).sum().backward()
    assert xi.grad is not None and torch.isfinite(xi.grad).all()
