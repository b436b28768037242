"""The streaming copy the memory-bound kernels are measured against copies every byte, for sizes
that end inside a 32 KiB chunk, exactly one chunk, and many chunks with a ragged tail."""

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [16, 32768, 32768 + 16, 10 * (1 << 20) + 48])
def test_stream_copy_is_exact(pkg, dev, nbytes):
    g = torch.Generator(device=dev).manual_seed(nbytes % 1000)
    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=dev, generator=g)
    dst = torch.zeros(nbytes + 64, dtype=torch.uint8, device=dev)
    pkg._lib.hbm_stream_copy(dst[:nbytes], src)
    torch.cuda.synchronize()
    assert torch.equal(dst[:nbytes], src)
    assert not bool(dst[nbytes:].any())  # nothing past the end is written


def test_stream_copy_rejects_ragged_sizes(pkg, dev):
    src = torch.zeros(24, dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError, match="multiple of 16"):
        pkg._lib.hbm_stream_copy(torch.zeros_like(src), src)


@pytest.mark.parametrize("chunks", [1, 3, 257])
def test_stream_fold_xors_the_word_pairs(pkg, dev, chunks):
    """The read-2-write-1 pass: output slot 256 i + t of chunk k is word 256 (2 i) + t xor word
    256 (2 i + 1) + t of the chunk's 2048 16-byte words."""
    n = chunks * 32768
    g = torch.Generator(device=dev).manual_seed(chunks)
    src = torch.randint(-2**31, 2**31 - 1, (n // 4,), dtype=torch.int32, device=dev, generator=g)
    dst = torch.zeros(n // 8 + 16, dtype=torch.int32, device=dev)
    pkg._lib.hbm_stream_fold(dst[: n // 8], src)
    torch.cuda.synchronize()
    w = src.view(chunks, 4, 2, 256, 4)  # [chunk, i, pair, t, word]
    ref = (w[:, :, 0] ^ w[:, :, 1]).reshape(-1)
    assert torch.equal(dst[: n // 8], ref)
    assert not bool(dst[n // 8:].any())


def test_stream_fold_rejects_partial_chunks(pkg, dev):
    src = torch.zeros(32768 + 16, dtype=torch.uint8, device=dev)
    with pytest.raises(ValueError, match="multiple of 32768"):
        pkg._lib.hbm_stream_fold(torch.zeros(src.numel() // 2, dtype=torch.uint8, device=dev), src)
