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
    """stack_100m (dim 1024, H16 hd64, b16, top-64, FFN 4096, vocab 256), bf16,
    one 131,072-token prompt on the pinned host tier, 256 MiB workspace."""
    m = M.build_model(M.STACK_100M, device="meta", dtype=torch.bfloat16)
    plan = plan_inference(m, 1, 131072, cache="cpu")
    ws = 256 << 20
    assert plan.cache == "cpu"
    assert plan.cache_bytes == 2 * 131072 * 16 * 64 * 2
    # encoder: (9*1024 + 2*4096) elements * 2 bytes = 34,816 B per token -> 7710 tokens fit,
    # capped at the requested 4096 (a multiple of lcm(16, 128))
    assert ws // ((9 * 1024 + 2 * 4096) * 2) == 7710 and plan.encoder_chunk == 4096
    # one read of 16 queries: 8 MiB of scores (256 rows x 8192 blocks) + partials + outputs
    read16 = 4 * 256 * 8192 + 4 * 256 * 17 * 66 + 256 * (12 * 64 + 4 + 64 * 2)
    assert plan.query_chunk == 16 and plan.read_bytes == read16
    assert plan.head_chunk == 16
    # score chunk: two device K buffers of 2,048 B per token -> 65,536 tokens
    assert plan.score_tokens == plan.page_tokens == 65536
    assert plan.pool_pages == 0


def test_plan_small_workspace_clamps_every_chunk():
    m = M.build_model(M.STACK_100M, device="meta", dtype=torch.bfloat16)
    plan = plan_inference(m, 1, 131072, cache="cpu", workspace_mb=1)
    assert plan.encoder_chunk == 128       # 30 tokens fit: one unit of 128
    assert plan.query_chunk == 1           # two queries need 1 MiB of scores alone
    assert plan.head_chunk == 1
    assert plan.score_tokens == 256        # 1 MiB / (2 x 2,048 B)


def test_available_host_memory_takes_the_cgroup_limit(monkeypatch):
    import exploration_amd.inference as inf
    monkeypatch.setattr(inf, "_meminfo_available", lambda: 10 << 30)
    monkeypatch.setattr(inf, "_cgroup_room", lambda: 3 << 30)
    assert inf.available_host_memory() == 3 << 30
    monkeypatch.setattr(inf, "_cgroup_room", lambda: None)
    assert inf.available_host_memory() == 10 << 30
    monkeypatch.setattr(inf, "_meminfo_available", lambda: None)
    assert inf.available_host_memory() is None


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
