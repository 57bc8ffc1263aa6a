"""The MFMA ceiling measurement (tests/hip/mfma_ceiling.hip): every SIMD issuing v_mfma_f32_32x32x64_f8f6f4 back to
back on LDS-fed operands. Checks that the loop is MFMA-bound cycle for cycle and that its FLOP rate agrees with the
clock the waves measured; prints the rates on constant and on random e4m3 operands (random ones draw enough power
that the clock drops: that rate, not the published peak, is what a GEMM on real data can reach)."""
import ctypes
import os

import pytest
import torch

LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "hip", "libmfma_ceiling.so")
FLOPS_PER_MFMA = 2 * 32 * 32 * 64
CYCLES_PER_MFMA = 64


def probe(random, steps=8000):
    lib = ctypes.CDLL(LIB)
    d = ctypes.c_double
    lib.gpic_probe_mfma_ceiling.argtypes = [ctypes.c_int, ctypes.c_int] + [ctypes.POINTER(d)] * 4
    ms, tf, ghz, busy = d(), d(), d(), d()
    rc = lib.gpic_probe_mfma_ceiling(int(random), steps, ms, tf, ghz, busy)
    assert rc == 0, rc
    return ms.value, tf.value, ghz.value, busy.value


@pytest.mark.gpu
@pytest.mark.parametrize("random", [False, True], ids=["const", "random"])
def test_mfma_ceiling(random):
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} is missing: run __graft_entry__.build()")
    torch.cuda.init()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    ms, tf, ghz, busy = probe(random)
    print(f"\n{'random' if random else 'const'} e4m3: {tf:.0f} TFLOP/s, clock {ghz:.2f} GHz, MFMA busy {busy:.3f} "
          f"({ms:.2f} ms)", flush=True)
    assert busy > 0.95                       # the loop issues an MFMA every 64 cycles on every SIMD
    expect = ghz * 1e9 * busy * cus * 4 * FLOPS_PER_MFMA / CYCLES_PER_MFMA / 1e12
    assert abs(tf / expect - 1) < 0.05, (tf, expect)
