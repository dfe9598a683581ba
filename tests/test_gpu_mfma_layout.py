"""Lane layout of v_mfma_f32_32x32x16_f16 on gfx950, as the dense large-M kernel
uses it (operand k ranges 8 (lane / 32) .. + 7, result row 8 (r / 4) + 4 (lane / 32)
+ r % 4): one instruction on integer-valued operands, whose product is exact in
fp32, compared with the plain product."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def test_mfma_32x32x16_lane_layout():
    import bench

    lib = bench.load_probe()
    lib.marlin_probe_mfma_32x32x16.restype = ctypes.c_int
    lib.marlin_probe_mfma_32x32x16.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int, ctypes.c_void_p]
    rng = np.random.default_rng(7)
    A = rng.integers(-8, 8, (32, 16)).astype(np.float16)
    B = rng.integers(-8, 8, (16, 32)).astype(np.float16)
    a, b = torch.from_numpy(A).to(DEV), torch.from_numpy(B).to(DEV)
    d = torch.full((32, 32), float("nan"), dtype=torch.float32, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.marlin_probe_mfma_32x32x16(a.data_ptr(), b.data_ptr(), d.data_ptr(), 0, ctypes.c_void_p(stream)) == 0
    torch.cuda.synchronize()
    assert np.array_equal(d.cpu().numpy(), A.astype(np.float32) @ B.astype(np.float32))
