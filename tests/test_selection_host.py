"""The product's host-side selection helpers against the reference tests' known answers and the oracle.

`lazykv_amd.selection.blocks_for_budget` and `current_block_mask` run no kernel, so they are checked
here on the CPU: the budget rule of lazykv/selection.py:72-74 (tests/test_selection.py:38-44) and
the current-block mask of lazykv/selection.py:65-69 (tests/test_selection.py:98).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from lazykv_amd.selection import blocks_for_budget, current_block_mask
from oracle import reference as R


def test_blocks_for_budget_leaves_room_for_sink_and_current_block() -> None:
    """tests/test_selection.py:38-44, and the workloads' budgets under the reference's rule."""
    for frac in (0.75, 0.25, 0.0625):
        k = blocks_for_budget(frac, 32768, 64)
        assert (k + 2) * 64 <= frac * 32768
    assert blocks_for_budget(0.0625, 131072, 16) == 510  # 8B, 128K, 6.25%
    assert blocks_for_budget(0.25, 32768, 16) == 510  # 1B, 32K, 25%
    assert blocks_for_budget(0.25, 65536, 16) == 1022  # 1B, 64K, 25%
    assert blocks_for_budget(0.5, 131072, 16) == 4094
    # At least one block, however small the budget.
    assert blocks_for_budget(0.0, 32768, 16) == 1
    assert blocks_for_budget(0.001, 1024, 64) == 1


def test_blocks_for_budget_equals_the_oracle_over_a_sweep() -> None:
    gen = np.random.default_rng(5)
    for _ in range(2000):
        frac = float(gen.uniform(0.0, 1.0))
        tokens = int(gen.integers(1, 1 << 20))
        bs = int(gen.choice([4, 8, 16, 32, 64, 128, 256]))
        k = blocks_for_budget(frac, tokens, bs)
        assert k == R.blocks_for_budget(frac, tokens, bs)
        assert k >= 1
        if k > 1:
            # K is the largest count for which sink + K + current fit in the budget.
            assert (k + 2) * bs <= frac * tokens * (1 + 1e-12)
            assert (k + 3) * bs > frac * tokens * (1 - 1e-12)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_current_block_mask_hides_the_unfilled_tail(dtype: torch.dtype) -> None:
    """tests/test_selection.py:98: K = 3, 5 live tokens of the current block, positions 4*BS+5 on masked."""
    bs, k = 8, 3
    total = (k + 2) * bs
    mask = current_block_mask(total, bs, 5, dtype, torch.device("cpu"))
    assert mask.shape == (1, 1, 1, total) and mask.dtype == dtype
    assert (mask[0, 0, 0, : 4 * bs + 5] == 0).all() and torch.isinf(mask[0, 0, 0, 4 * bs + 5 :]).all()
    assert (mask[0, 0, 0, 4 * bs + 5 :] < 0).all()
    assert np.array_equal(mask[0, 0, 0].float().numpy(), R.current_block_mask(total, bs, 5))


def test_current_block_mask_reuses_its_buffer_for_every_fill() -> None:
    """A reused mask is cleared first, so a larger fill unmasks what a smaller one hid."""
    bs, total = 16, 5 * 16
    buf = current_block_mask(total, bs, 1, torch.float32, torch.device("cpu"))
    for fill in (3, 16, 1, 9):
        out = current_block_mask(total, bs, fill, torch.float32, torch.device("cpu"), reuse=buf)
        assert out.data_ptr() == buf.data_ptr()
        assert np.array_equal(out[0, 0, 0].numpy(), R.current_block_mask(total, bs, fill))
    full = current_block_mask(total, bs, bs, torch.float32, torch.device("cpu"))
    assert (full == 0).all()  # a full current block hides nothing
