"""Inference planning and the KV cache tiers on the CPU
(st/runtime/memory.py:43-97, st/runtime/inference.py:19-62): the chunk
sizes for a stack_100m-shaped bf16 model with the default 256 MiB
workspace, derived by hand from the reference's bounds; the disk tier's
file mapping, its writes and its removal on close (the reference's
tests/test_framework.py:54-70 checks the directory is left empty)."""
import os

import pytest
import torch

import exploration_amd.model as M
from exploration_amd.inference import InferencePlan, KVCache, plan_inference


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
    with pytest.raises(ValueError):
        plan_inference(m, 1, 1024, cache="disk")  # no cache_dir
    with pytest.raises(MemoryError):
        plan_inference(m, 1, 1024, cache="cuda")  # parameters not on a GPU


def test_plan_disk(tmp_path):
    m = M.build_model(M.STACK_100M, device="meta", dtype=torch.bfloat16)
    plan = plan_inference(m, 1, 4096, cache="disk", cache_dir=str(tmp_path / "kv"))
    assert plan.cache == "disk" and os.path.isdir(tmp_path / "kv")
    with pytest.raises(MemoryError):
        plan_inference(m, 1, 1 << 40, cache="disk", cache_dir=str(tmp_path))  # 4 PiB of K/V


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=str)
def test_disk_cache_roundtrip_and_cleanup(tmp_path, dtype):
    plan = InferencePlan("disk", 0, 0, 64, 64, 4, 64, 4, None)
    g = torch.Generator().manual_seed(1)
    cache = KVCache(2, 100, 3, 8, dtype, "cpu", plan, offset=128, cache_dir=str(tmp_path))
    (sub,) = os.listdir(tmp_path)
    assert os.path.getsize(tmp_path / sub / "kv.bin") == 2 * 2 * 100 * 3 * 8 * dtype.itemsize
    k, v = torch.randn(2, 2, 100, 3, 8, generator=g).to(dtype)
    cache.write(128, k[:, :60], v[:, :60])
    cache.write(188, k[:, 60:], v[:, 60:])
    assert torch.equal(cache.k, k) and torch.equal(cache.v, v)
    # the page protocol reads back what was written
    pages = list(cache.pages("cpu"))
    assert [p[0] for p in pages] == [128, 192]
    assert torch.equal(torch.cat([p[1] for p in pages], 1), k)
    with pytest.raises(ValueError):
        cache.write(100, k[:, :10], v[:, :10])  # before the shard
    with pytest.raises(ValueError):
        cache.write(200, k, v)  # past its end
    cache.close()
    assert os.listdir(tmp_path) == []
    with KVCache(1, 16, 1, 4, dtype, "cpu", plan, cache_dir=str(tmp_path)):
        assert len(os.listdir(tmp_path)) == 1
    assert os.listdir(tmp_path) == []
