"""Host logic of the fp16 projection wrapper (``nori_amd.projection``): the row grids it hands
the kernel address every row of x and of the output, in order, for the strided views the model
passes (no GPU needed: only the addressing is checked)."""

from __future__ import annotations

import itertools

import pytest
import torch

from nori_amd.projection import _common_grid


def grid_offsets(grid, strides):
    no, nm, ni = grid
    return [o * strides[0] + j * strides[1] + i * strides[2] for o in range(no) for j in range(nm) for i in range(ni)]


def row_offsets(t):
    lead = t.shape[:-1]
    return [sum(a * b for a, b in zip(ix, t.stride()[:-1])) for ix in itertools.product(*[range(n) for n in lead])]


CELLS = torch.empty(3, 5, 4, 16)  # [table, row, group, width]
TOKENS = torch.empty(7, 6, 16)


@pytest.mark.parametrize(
    "x,y",
    [
        (CELLS.transpose(1, 2), torch.empty(3, 4, 5, 8)),              # transposed view, contiguous out
        (CELLS.transpose(1, 2)[:, :, :3], torch.empty(3, 4, 3, 8)),    # its first rows (the K/V operand)
        (TOKENS[:, :4], torch.empty(7, 6, 32)[:, :4, :8]),              # token subset into a stacked slice
        (torch.empty(100, 16), torch.empty(100, 8)),
        (torch.empty(4, 5, 16), torch.empty(20, 8).view(4, 5, 8)),
        (torch.empty(2, 3, 4, 16), torch.empty(2, 12, 8).view(2, 3, 4, 8)),
    ],
)
def test_common_grid_addresses_every_row_in_order(x, y):
    grid = _common_grid(x, y)
    assert grid is not None
    levels, sx, sy = grid
    assert grid_offsets(levels, sx) == row_offsets(x)
    assert grid_offsets(levels, sy) == row_offsets(y)


def test_four_levels_are_refused():
    x = torch.empty(2, 3, 4, 5, 16).permute(0, 2, 1, 3, 4)[:, :, :, :3]
    assert _common_grid(x, torch.empty(2, 4, 3, 3, 8)) is None
