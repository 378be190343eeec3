"""Properties that fix the moe_align layout uniquely (used by the CPU oracle
tests and the GPU tests): for route ids over `experts` experts and blocks of
`block_m` rows,
  * blocks hold experts in ascending order, each expert e in exactly
    ceil(count_e / block_m) consecutive blocks (count_e = its valid pairs),
    and every block past the last holds expert -1;
  * every valid pair index appears exactly once, in a block of its own
    expert, and each expert's pairs appear in ascending pair index;
  * every other row holds the sentinel `pairs`, and within an expert's
    blocks all sentinels come after its last pair;
  * padded = number of blocks * block_m."""
import numpy as np


def check_moe_align(sorted_ids, expert_ids, padded, ids, experts, block_m):
    flat = np.asarray(ids, np.int64).reshape(-1)
    pairs = flat.size
    sorted_ids = np.asarray(sorted_ids, np.int64)
    expert_ids = np.asarray(expert_ids, np.int64)
    valid = (flat >= 0) & (flat < experts)
    counts = np.bincount(flat[valid], minlength=experts)
    blocks_per = (counts + block_m - 1) // block_m
    nblocks = int(blocks_per.sum())
    assert padded == nblocks * block_m, (padded, nblocks)
    assert np.array_equal(expert_ids[:nblocks], np.repeat(np.arange(experts), blocks_per))
    assert np.all(expert_ids[nblocks:] == -1)
    assert np.all(sorted_ids[padded:] == pairs)
    seen = np.zeros(pairs, np.int64)
    start = 0
    for e in range(experts):
        rows = sorted_ids[start * block_m:(start + blocks_per[e]) * block_m]
        real = rows[rows != pairs]
        assert real.size == counts[e], e
        assert np.all(rows[:real.size] != pairs) and np.all(rows[real.size:] == pairs), e
        assert np.all(np.diff(real) > 0), e
        assert np.all(flat[real] == e), e
        seen[real] += 1
        start += blocks_per[e]
    assert np.array_equal(seen, valid.astype(np.int64))
