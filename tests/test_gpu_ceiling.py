"""The MFMA ceiling measurement (tests/hip/mfma_ceiling.hip): every SIMD issuing FP8 MFMAs back to back, in the
16 x 16 x 128 form the GEMM uses and in the 32 x 32 x 64 form. Checks that the loop is MFMA-bound cycle for cycle and
that its FLOP rate agrees with the clock the waves measured; prints the rates on constant and on random e4m3 operands
(random ones draw enough power that the clock drops: that rate, not the published peak, is what a GEMM on real data
can reach)."""
import ctypes
import os

import pytest
import torch

LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "hip", "libmfma_ceiling.so")
FLOPS_PER_CYCLE_PER_SIMD = 2 * 32 * 32 * 64 / 64    # either form: 2048 FP8 FLOP per cycle and SIMD


def probe(shape, random, src=None, steps=8000):
    lib = ctypes.CDLL(LIB)
    d = ctypes.c_double
    lib.gpic_probe_mfma_ceiling.argtypes = ([ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int] +
                                            [ctypes.POINTER(d)] * 4)
    ms, tf, ghz, busy = d(), d(), d(), d()
    rc = lib.gpic_probe_mfma_ceiling(shape, int(random), None if src is None else src.data_ptr(),
                                     0 if src is None else src.numel(), steps, ms, tf, ghz, busy)
    assert rc == 0, rc
    return ms.value, tf.value, ghz.value, busy.value


@pytest.mark.gpu
@pytest.mark.parametrize("shape", [16, 32], ids=["16x16x128", "32x32x64"])
@pytest.mark.parametrize("data", ["const", "random", "tcast"])
def test_mfma_ceiling(shape, data):
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is missing: run __graft_entry__.build()")
    torch.cuda.init()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    src = None
    if data == "tcast":   # the e4m3 bytes of an N(0, 1) tensor, as a GEMM's operands
        import gpic_fp8 as G
        g = torch.Generator(device="cuda").manual_seed(0)
        src = G.tcast(torch.randn(2048, 4096, generator=g, device="cuda").to(torch.bfloat16))[0].view(torch.uint8)
    ms, tf, ghz, busy = probe(shape, data == "random", src)
    print(f"\n{shape}x{shape}x{2048 // shape} {data} e4m3: {tf:.0f} TFLOP/s, clock {ghz:.2f} GHz, "
          f"MFMA busy {busy:.3f} ({ms:.2f} ms)", flush=True)
    assert busy > 0.95                       # the loop keeps every SIMD's MFMA pipe busy
    expect = ghz * 1e9 * busy * cus * 4 * FLOPS_PER_CYCLE_PER_SIMD / 1e12
    assert abs(tf / expect - 1) < 0.05, (tf, expect)

    with pytest.raises(AssertionError):      # a form the probe does not know is refused
        probe(24, False, None, 2)


@pytest.mark.gpu
def test_hbm_floor_probe(dev):
    """tests/hip/hbm_floor.hip: one read launch and one write launch over 64 / 32 MiB, in every launch shape; bench.py
    reports the config-2 cast against their times. The read returns each workgroup's maximum word (all ones here: the
    bits of 1.0f), so the probe is seen to read what it claims."""
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "hip", "libhbm_floor.so")
    lib = ctypes.CDLL(path)
    lib.gpic_probe_hbm.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p,
                                   ctypes.c_void_p]
    lib.gpic_probe_hbm_groups.argtypes = [ctypes.c_int, ctypes.c_uint64]
    nb = 64 * 1024 * 1024
    src = torch.ones(nb // 4, dtype=torch.float32, device=dev)
    dst = torch.zeros(nb // 8, dtype=torch.float32, device=dev)
    st = torch.cuda.current_stream(dev).cuda_stream
    for cfg in range(4):
        g = lib.gpic_probe_hbm_groups(cfg, nb)
        out = torch.zeros(g, dtype=torch.int32, device=dev)
        assert lib.gpic_probe_hbm(1, cfg, src.data_ptr(), nb, out.data_ptr(), st) == 0
        assert lib.gpic_probe_hbm(0, cfg, dst.data_ptr(), nb // 2, None, st) == 0
        torch.cuda.synchronize()
        assert bool((out == 0x3F800000).all()), cfg
        assert bool((dst.view(torch.int32) == 0x38383838).all()), cfg
    lib.gpic_probe_hbm_rw.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_void_p]
    for cfg in range(4):   # the read-and-write launch: 8 bytes per 16-byte word (here 1.0f x 4: zeros)
        dst.fill_(7.0)
        assert lib.gpic_probe_hbm_rw(cfg, src.data_ptr(), nb, dst.data_ptr(), st) == 0
        torch.cuda.synchronize()
        assert bool((dst == 0).all()), cfg
    assert lib.gpic_probe_hbm(1, 9, src.data_ptr(), nb, out.data_ptr(), st) == -1
    assert lib.gpic_probe_hbm(1, 0, src.data_ptr(), 17, out.data_ptr(), st) == -1
