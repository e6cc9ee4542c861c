"""Host-side checks of the GPU-resident KV cache (no device memory touched):
the step and constructor validation of smollm2_triton/model.py:197-214 and
:256-268, with the reference's messages."""

import pytest

from triton_llm.kv_cache import GpuKVCache, check_step


def test_check_step_mirrors_the_model():
    assert check_step(0, 7, 8) == 7
    assert check_step(7, 1, 8) == 8
    with pytest.raises(ValueError, match=r"Decode mode requires seq=1, got seq=2"):
        check_step(3, 2, 8)
    with pytest.raises(ValueError, match=r"Total sequence length 9 exceeds pre-allocated cache size \(8\)"):
        check_step(8, 1, 8)
    with pytest.raises(ValueError, match=r"Total sequence length 9 exceeds"):
        check_step(0, 9, 8)


def test_constructor_validation_before_allocation():
    with pytest.raises(ValueError, match="max_seq must be a positive integer, got 0"):
        GpuKVCache(2, 9, 3, 64, max_seq=0)
    with pytest.raises(ValueError, match=r"max_seq \(100\) cannot exceed model's max_position_embeddings \(64\)"):
        GpuKVCache(2, 9, 3, 64, max_seq=100, max_position_embeddings=64)
    with pytest.raises(ValueError, match="bad head counts"):
        GpuKVCache(2, 10, 3, 64, max_seq=16)
