"""lia_hbm_read, the contiguous-read ceiling the bench measures beside the attention kernel:
every byte is read (each workgroup's word is the XOR of its share), ragged sizes included."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes,wgs", [(16, 1), (4096, 3), (1 << 20, 256), ((1 << 20) + 48, 7),
                                        (96546828 // 16 * 16, 1024)])
def test_hbm_read_folds_every_word(lia, nbytes, wgs):
    g = torch.Generator(device="cuda")
    g.manual_seed(nbytes)
    src = torch.randint(-2**31, 2**31 - 1, (nbytes // 4,), generator=g, dtype=torch.int32, device="cuda")
    sink = torch.zeros(wgs, dtype=torch.int32, device="cuda")
    lia.hbm_read(src, wgs, sink)
    torch.cuda.synchronize()
    words = src.cpu().numpy().view(np.uint32)
    share = -(-(nbytes // 16) // wgs) * 4  # words per workgroup (16-byte units split evenly)
    want = [np.bitwise_xor.reduce(words[i * share:(i + 1) * share]) if i * share < len(words) else 0
            for i in range(wgs)]
    got = sink.cpu().numpy().view(np.uint32)
    assert np.array_equal(got, np.array(want, np.uint32))
