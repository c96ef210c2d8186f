"""Inference planning on the CPU (st/runtime/memory.py:43-97): the chunk
sizes for a stack_100m-shaped bf16 model with the default 256 MiB workspace,
derived by hand from the reference's bounds."""
import pytest
import torch

import exploration_amd.model as M
from exploration_amd.inference import plan_inference


def test_plan_chunks_stack_100m():
    m = M.build_model(M.STACK_100M, device="meta", dtype=torch.bfloat16)
    plan = plan_inference(m, 1, 131072, cache="cpu")
    ws = 256 << 20
    assert plan.cache == "cpu"
    assert plan.cache_bytes == 2 * 131072 * 1024 * 2
    # page: min(65536, ws / (2*1*1024*2)) = 65536; encoder: ws / (24*1024*2) = 5461 -> 4096
    assert plan.page_tokens == min(65536, ws // (2 * 1024 * 2)) // 16 * 16 == 65536
    assert plan.encoder_chunk == 4096
    # query chunk: min(16, ws / (16 heads * 64 topk * 16 b * 4)); score tile: min(page, ws / (4*16*16*4))
    assert plan.query_chunk == 16
    assert plan.score_tokens == 65536
    assert plan.head_chunk == 16


def test_plan_rejects():
    m = M.build_model(M.STACK_100M, device="meta", dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        plan_inference(m, 1, 1024, memory_fraction=1.5)
    with pytest.raises(ValueError):
        plan_inference(m, 1, 1024, cache="tape")
    with pytest.raises(NotImplementedError):
        plan_inference(m, 1, 1024, cache="disk")
    with pytest.raises(MemoryError):
        plan_inference(m, 1, 1024, cache="cuda")  # parameters not on a GPU
