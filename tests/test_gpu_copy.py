"""aigpu_copy_device, the streaming copy behind the bench's achievable-
bandwidth line: every byte arrives, including a ragged tail past the last
16-byte piece, nothing past the end is touched, and misaligned or overlapping
buffers are refused before any launch."""
import numpy as np
import pytest

from gpu_util import say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [16, 4096 * 8 + 16, (1 << 26) + 7, 5])
def test_copy_moves_every_byte(gpu, nbytes):
    import torch
    rng = np.random.default_rng(nbytes)
    src_h = rng.integers(0, 256, nbytes + 64, dtype=np.uint8)
    src = torch.from_numpy(src_h).cuda()
    dst = torch.zeros(nbytes + 64, dtype=torch.uint8, device="cuda")
    say("copy", dict(nbytes=nbytes))
    gpu.copy_device(dst, src, nbytes)
    got = dst.cpu().numpy()
    np.testing.assert_array_equal(got[:nbytes], src_h[:nbytes])
    assert not got[nbytes:].any(), "bytes past the copy were written"


def test_copy_refuses_misaligned_and_overlapping_buffers(gpu):
    import torch
    buf = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    with pytest.raises(gpu.AiGpuError, match="aligned"):
        gpu.copy_device(buf[8:], buf[2048:], 1024)
    with pytest.raises(gpu.AiGpuError, match="overlap"):
        gpu.copy_device(buf[16:], buf, 1024)
