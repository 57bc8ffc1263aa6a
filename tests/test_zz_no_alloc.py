"""gpic_fp8_tcast_noalloc (the cast with its workspace in the library's static device array) through the C ABI:
the same bytes and scale as gpic_fp8_tcast on the same inputs, on consecutive calls with a smaller input second
(the array keeps the previous call's state), both single-pass and two-pass sizes, and equal to the oracle."""
import numpy as np
import pytest
import torch

import gpic_fp8 as G
from gpic_fp8 import _lib as L
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def noalloc(x):
    """x (contiguous bf16 / fp32 on the GPU) -> (e4m3 bytes, dequant) from gpic_fp8_tcast_noalloc."""
    q = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    s = torch.empty(1, dtype=torch.float32, device=x.device)
    rc = L.lib().gpic_fp8_tcast_noalloc(x.data_ptr(), L.DTYPE_CODE[x.dtype], x.numel(), q.data_ptr(), s.data_ptr(),
                                        L.stream_ptr(x.device))
    assert rc == 0, L.lib().gpic_fp8_status_string(rc)
    return q, s


def host(x):
    return (x.view(torch.int16).cpu().numpy().view(np.uint16) if x.dtype == torch.bfloat16
            else x.cpu().numpy())


@pytest.mark.parametrize("shapes,dtype", [
    (((32768, 1024), (3000, 1000)), torch.bfloat16),        # single pass: full grid, then a smaller grid with a tail
    (((5000, 4096), (777, 1024)), torch.float32),           # fp32 single pass, then smaller
    (((16384, 16384), (1000, 8)), torch.bfloat16),          # past the single pass (two-pass), then a tiny one
])
def test_noalloc_matches_tcast(dev, shapes, dtype):
    g = torch.Generator(device=dev).manual_seed(sum(shapes[0]))
    for i, shape in enumerate(shapes):
        x = (torch.randn(*shape, generator=g, device=dev) * (10.0 if i == 0 else 0.01)).to(dtype)
        q, s = noalloc(x)
        q0, s0 = G.tcast(x)
        torch.cuda.synchronize()
        assert s.item() == s0.item(), (shape, s.item(), s0.item())
        assert torch.equal(q, q0.view(torch.uint8)), f"{shape}: bytes differ from gpic_fp8_tcast"
        if x.numel() <= 1 << 26:
            oq, od, _ = O.tcast(host(x))
            assert s.item() == od and np.array_equal(q.cpu().numpy(), oq)


def test_noalloc_argument_errors(dev):
    """Invalid arguments come back as status codes (nothing launched), as from gpic_fp8_tcast."""
    x = torch.randn(64, device=dev).to(torch.bfloat16)
    q = torch.empty(64, dtype=torch.uint8, device=dev)
    s = torch.empty(1, dtype=torch.float32, device=dev)
    lib, st = L.lib(), L.stream_ptr(dev)
    assert lib.gpic_fp8_tcast_noalloc(x.data_ptr() + 2, 0, 32, q.data_ptr(), s.data_ptr(), st) == -4
    assert lib.gpic_fp8_tcast_noalloc(x.data_ptr(), 7, 64, q.data_ptr(), s.data_ptr(), st) == -2
    assert lib.gpic_fp8_tcast_noalloc(x.data_ptr(), 0, -1, q.data_ptr(), s.data_ptr(), st) == -1
    assert lib.gpic_fp8_tcast_noalloc(x.data_ptr(), 0, 64, q.data_ptr(), None, st) == -1
