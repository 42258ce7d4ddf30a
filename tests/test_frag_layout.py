"""The fragment order of decode activations (``FragRows``), on the CPU: the
layout is the closed-form offset the kernels use, and the round trip is the
identity. The kernels that write and read it are compared with the row-major
ones in ``test_gpu_projections.py``."""
import pytest
import torch

from litemoe_amd.linear import FragRows, frag_row_blocks


def offset(r, k, mb):
    """Element (r, k): k steps of 32, then 16-row blocks, then the MFMA A
    operand's 64 lanes (row r%16, k group (k%32)//8), 8 values each."""
    return ((k // 32) * mb + r // 16) * 512 + ((k % 32) // 8) * 128 + (r % 16) * 8 + k % 8


@pytest.mark.parametrize("rows,cols", [(1, 32), (5, 64), (16, 96), (17, 1536), (40, 128), (64, 3072 // 8), (100, 64), (128, 32)])
def test_fragment_order_is_the_closed_form_and_round_trips(rows, cols):
    a = torch.arange(rows * cols, dtype=torch.float32).view(rows, cols).to(torch.bfloat16)
    a = torch.randn(rows, cols).to(torch.bfloat16) if rows * cols > 256 else a
    f = FragRows.from_rows(a)
    mb = frag_row_blocks(rows)
    assert f.mb == mb and f.data.numel() == 16 * mb * cols
    flat = f.data
    g = torch.Generator().manual_seed(rows + cols)
    for _ in range(64):
        r = int(torch.randint(0, rows, (1,), generator=g))
        k = int(torch.randint(0, cols, (1,), generator=g))
        assert flat[offset(r, k, mb)].view(torch.int16) == a[r, k].view(torch.int16)
    # every element once, padding rows zero
    idx = torch.tensor([offset(r, k, mb) for r in range(16 * mb) for k in range(cols)])
    assert idx.unique().numel() == 16 * mb * cols and int(idx.max()) == 16 * mb * cols - 1
    pad = torch.tensor([offset(r, k, mb) for r in range(rows, 16 * mb) for k in range(cols)], dtype=torch.long)
    if pad.numel():
        assert bool((flat[pad] == 0).all())
    assert torch.equal(f.to_rows(), a)


def test_row_blocks_and_limits():
    assert [frag_row_blocks(r) for r in (1, 16, 17, 32, 33, 64, 65, 128)] == [1, 1, 2, 2, 4, 4, 8, 8]
    with pytest.raises(ValueError):
        frag_row_blocks(129)
    with pytest.raises(ValueError):
        FragRows(4, 48, "cpu")
