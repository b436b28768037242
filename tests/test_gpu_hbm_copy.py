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
