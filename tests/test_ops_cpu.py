"""CPU checks of host-side dispatch rules in exact_amd.ops."""


def test_norm_gemv_one_block_per_cu_matches_the_kernel_split():
    """The model fuses the attention norm into the q|k|v GEMV only where exact_gemv_g128_norm_acc runs one 8-wave block
    per CU: rows wider than 2048 whose group-split tasks (ceil(N / 64) row blocks x min(G, ceil(4096 / row blocks)))
    fit 256 blocks of 8."""
    from exact_amd import ops
    assert ops.norm_gemv_one_block_per_cu(4608, 3584)          # 7B q|k|v: 72 x 28 = 2016 tasks, 252 blocks
    assert not ops.norm_gemv_one_block_per_cu(7168, 5120)      # 14B q|k|v: 112 x 37 = 4144 tasks, 518 blocks
    assert ops.norm_gemv_one_block_per_cu(300, 6144)           # 5 x 48 = 240 tasks
    assert not ops.norm_gemv_one_block_per_cu(4608, 2048)      # rows of 2048 keep 4-wave blocks
    assert ops.norm_gemv_one_block_per_cu(4608, 3584, R=2)
    assert not ops.norm_gemv_one_block_per_cu(4608, 3584, R=3)      # the launch takes at most 2 rows
