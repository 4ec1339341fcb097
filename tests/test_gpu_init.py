"""Device set-up: lia_init resolves the library's kernels on the device (the counterpart of
loading the kernels' module once, src/gpu/llama_attention.rs:24,163) and every launch after
it runs through hipModuleLaunchKernel on those functions."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

E_HIP = -30


def test_init_resolves_kernels_and_reports_cus(lia):
    L = lia.lib()
    assert L.lia_init(0) == 0
    assert L.lia_init(0) == 0  # idempotent
    assert L.lia_device_cus() == torch.cuda.get_device_properties(0).multi_processor_count


def test_init_rejects_a_device_that_does_not_exist(lia):
    L = lia.lib()
    assert L.lia_init(torch.cuda.device_count() + 7) == E_HIP
    # the failed call leaves the current device usable
    assert L.lia_init(0) == 0


def test_launch_after_init_runs_the_kernel(lia):
    assert lia.lib().lia_init(0) == 0
    src = torch.arange(64 * 12, dtype=torch.float32, device="cuda").reshape(64, 12)
    idx = torch.tensor([5, 0, 63, 5], dtype=torch.int32, device="cuda")
    dst = torch.zeros(4, 12, dtype=torch.float32, device="cuda")
    lia.gather_rows(idx, src, dst)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(dst.cpu().numpy(), src.cpu().numpy()[[5, 0, 63, 5]])
