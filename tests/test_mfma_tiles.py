"""The MFMA tile order of the weight copies the batched kernel streams
(``mk_weights.mfma_tiles``), checked element by element against the layout
the kernel's loads assume: for matrix [N][K], 1 KiB block
(row // 16) * (K // 32) + col // 32, 16-byte slot ((col % 32) // 8) * 16 + row % 16,
element col % 8 -- the B operand of v_mfma_f32_16x16x32_bf16 (lane = slot:
row lane % 16, columns (lane // 16) * 8 .. +7 of the k-step)."""

import pytest
import torch

from mk_weights import mfma_tiles


def expected_index(r, c, K):
    block = (r // 16) * (K // 32) + c // 32
    slot = ((c % 32) // 8) * 16 + r % 16
    return block * 512 + slot * 8 + c % 8


@pytest.mark.parametrize("shape", [(16, 32), (48, 96), (2, 32, 64)])
def test_tile_order_matches_kernel_offsets(shape):
    n, k = shape[-2], shape[-1]
    lead = 1 if len(shape) == 2 else shape[0]
    w = torch.arange(lead * n * k, dtype=torch.float32).reshape(shape)
    t = mfma_tiles(w)
    assert t.shape == w.shape
    flat_w = w.reshape(lead, n * k)
    flat_t = t.reshape(lead, n * k)
    for b in range(lead):
        for r in range(n):
            for c in range(k):
                assert flat_t[b, expected_index(r, c, k)] == flat_w[b, r * k + c]


def test_tile_is_a_permutation_of_bf16_bits():
    g = torch.Generator().manual_seed(5)
    w = torch.randn(64, 128, generator=g).to(torch.bfloat16)
    t = mfma_tiles(w)
    assert torch.equal(torch.sort(t.reshape(-1).view(torch.int16))[0], torch.sort(w.reshape(-1).view(torch.int16))[0])
    # one block = one MFMA B operand: lane l of block (0, 1) holds row l % 16, columns 32 + (l // 16) * 8 .. +7
    blk = t.reshape(-1)[512:1024].reshape(64, 8)
    for lane in range(64):
        assert torch.equal(blk[lane], w[lane % 16, 32 + (lane // 16) * 8: 32 + (lane // 16) * 8 + 8])


def test_untileable_shapes_rejected():
    with pytest.raises(ValueError):
        mfma_tiles(torch.zeros(24, 32))
    with pytest.raises(ValueError):
        mfma_tiles(torch.zeros(16, 48))
