"""CPU checks of host-side dispatch rules in exact_amd.ops."""
import os

import pytest

from exact_amd import _lib


@pytest.mark.skipif(not os.path.exists(_lib.LIB_PATH), reason="library not built")
def test_norm_gemv_one_block_per_cu_reads_the_kernel_split():
    """The model fuses the attention norm into the q|k|v GEMV only where exact_gemv_g128_norm_acc runs one 8-wave block
    per CU: rows wider than 1024 whose group-split tasks (ceil(N / 64) row blocks x min(G, ceil(4096 / row blocks)))
    fit one round of 8-wave blocks, or do with the split capped at 8 CUs / row blocks when that is at least 8. The
    split is the library's own query (no launch, no GPU needed with an explicit CU count); a device with fewer CUs
    gets fewer one-round shapes."""
    from exact_amd import ops
    assert ops.norm_gemv_one_block_per_cu(4608, 3584, cus=256)          # 7B q|k|v: 72 x 28 = 2016 tasks, 252 blocks
    assert ops.norm_gemv_one_block_per_cu(4608, 3584, cus=240)          # ... 240 CUs: split capped at 26 (1872 tasks)
    assert ops.norm_gemv_one_block_per_cu(7168, 5120, cus=256)          # 14B q|k|v: 112 x 37 tasks, capped at 112 x 18
    assert not ops.norm_gemv_one_block_per_cu(7168, 5120, cus=96)       # ... a cap of 6 parts: 4-wave blocks
    assert not ops.norm_gemv_one_block_per_cu(37888, 3584, cus=256)     # 7B gate|up: 592 row blocks, cap 3
    assert ops.norm_gemv_one_block_per_cu(300, 6144, cus=256)           # 5 x 48 = 240 tasks
    assert ops.norm_gemv_one_block_per_cu(6144, 2048, cus=256)          # MoE q|k|v: 96 x 16 = 1536 tasks, 192 blocks
    assert not ops.norm_gemv_one_block_per_cu(4608, 1024, cus=256)      # rows of 1024 and less keep 4-wave blocks
    assert not ops.norm_gemv_one_block_per_cu(1152, 896, cus=256)       # (the 0.5B's 896)
    assert ops.norm_gemv_one_block_per_cu(4608, 3584, R=2, cus=256)
    assert not ops.norm_gemv_one_block_per_cu(4608, 3584, R=3, cus=256)      # the launch takes at most 2 rows
    assert _lib.load().exact_gemv_g128_norm_acc_blockwaves(1, 4608, 100, 256) == 0   # K % 128: refused
