"""The library rounds fp32 -> bf16 with gfx950's v_cvt_pk_bf16_f32. This checks, on the GPU, that it gives the bits
of the integer round-to-nearest-even rule (NaN -> quiet NaN) for every one of the 2^32 fp32 inputs."""
import ctypes
import os

import pytest
import torch

pytestmark = pytest.mark.gpu
LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "hip", "libbf16_selfcheck.so")


def test_bf16_rounding_exhaustive(dev):
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is missing: run __graft_entry__.build() first")
    lib = ctypes.CDLL(LIB)
    lib.gpic_selfcheck_bf16.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    mismatch = torch.zeros(1, dtype=torch.int64, device=dev)
    rc = lib.gpic_selfcheck_bf16(mismatch.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert mismatch.item() == 0
