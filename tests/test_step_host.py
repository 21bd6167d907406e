"""Host logic of the decode step (llmpager_amd.step), on the CPU: which
shapes the fused launches take (head_dim 128, an fp16 cache, 1, 2, 4, 8 or
16 query heads per KV head, at most 16 KV heads, hidden and heads x
head_dim at most 4096, hidden a multiple of 8), so a shape outside them
runs the reference's launch sequence instead of failing on the device."""
import pytest

from llmpager_amd.step import StepShape, check_step, fusable


@pytest.mark.parametrize("kw,ok", [
    (dict(hidden=2048, heads=32, kv_heads=4, head_dim=128), True),    # Qwen3-30B-A3B
    (dict(hidden=4096, heads=64, kv_heads=4, head_dim=128), False),   # 235B: heads x head_dim 8192
    (dict(hidden=4096, heads=32, kv_heads=2, head_dim=128), True),    # 16 query heads per KV head
    (dict(hidden=2048, heads=32, kv_heads=4, head_dim=64), False),    # head_dim 64
    (dict(hidden=2048, heads=24, kv_heads=4, head_dim=128), False),   # 6 query heads per KV head
    (dict(hidden=2048, heads=32, kv_heads=32, head_dim=128), False),  # 32 KV heads
    (dict(hidden=2047, heads=8, kv_heads=8, head_dim=128), False),    # hidden not a multiple of 8
    (dict(hidden=8192, heads=32, kv_heads=4, head_dim=128), False),   # hidden past 4096
    (dict(hidden=256, heads=4, kv_heads=2, head_dim=128), True),      # the GPU test's shape
])
def test_fusable(kw, ok):
    assert fusable(StepShape(vocab=100, max_seq=16, **kw)) == ok
    # an fp32 cache always takes the reference's sequence
    assert not fusable(StepShape(vocab=100, max_seq=16, kv_f16=False, **kw))


@pytest.mark.parametrize("token,pos,ok", [
    (0, 0, True), (99, 15, True),
    (100, 0, False), (-1, 0, False),   # outside the embedding table
    (0, 16, False), (0, -1, False),    # outside the KV cache
])
def test_step_token_and_position_checked(token, pos, ok):
    S = StepShape(hidden=256, heads=4, kv_heads=2, head_dim=128, vocab=100, max_seq=16)
    if ok:
        check_step(S, token, pos)
    else:
        with pytest.raises(ValueError):
            check_step(S, token, pos)
