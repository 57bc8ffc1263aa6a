"""GPU parity of the cast kernels (gpic_fp8_tcast / gpic_fp8_tcast_t) against the pinned oracle and the golden vectors.
The bar is bit-exact: every e4m3 byte and every fp32 scale."""
import os

import numpy as np
import pytest
import torch

import gpic_fp8 as G
from gpic_fp8 import _lib as L
from oracle import oracle as O
from parity import once_state

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLD, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def to_bf16(h, dev):
    return torch.from_numpy(np.ascontiguousarray(h).view(np.int16)).view(torch.bfloat16).to(dev)


def bits(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def qb(t):
    return t.contiguous().view(torch.uint8).cpu().numpy()


def config2_input(rows=32768, cols=1024, seed=1):
    """fp32 randn (seed 1), round(0.01 * cols) outlier columns x50 in fp32, rounded once to bf16."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, cols, generator=g)
    c = torch.randperm(cols, generator=g)[:round(0.01 * cols)]
    x[:, c] *= 50.0
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("name", ["cast_bf16", "cast_tail", "cast_range"])
def test_golden_bf16(dev, gold, name):
    q, s = G.tcast(to_bf16(gold[f"{name}_x"], dev))
    assert np.array_equal(qb(q), gold[f"{name}_q"])
    assert s.item() == gold[f"{name}_s"][0]


def test_golden_f32_weight(dev, gold):
    q, s = G.tcast(torch.from_numpy(gold["cast_f32_x"]).to(dev))
    assert np.array_equal(qb(q), gold["cast_f32_q"]) and s.item() == gold["cast_f32_s"][0]


def test_golden_zero_and_empty(dev, gold):
    q, s = G.tcast(torch.zeros(16, 16, dtype=torch.bfloat16, device=dev))
    assert np.array_equal(qb(q), gold["cast_zero_q"]) and s.item() == gold["cast_zero_s"][0]
    q, s = G.tcast(torch.empty(0, 64, dtype=torch.bfloat16, device=dev))
    assert q.shape == (0, 64) and s.item() == np.float32(np.float32(1e-12) / np.float32(448.0))


def test_golden_cast_t(dev, gold):
    q, qt, s = G.tcast_t(to_bf16(gold["cast_t_x"], dev))
    assert np.array_equal(qb(q), gold["cast_t_q"]) and np.array_equal(qb(qt), gold["cast_t_qt"])
    assert s.item() == gold["cast_t_s"][0]


def test_config2_full_size_bitexact(dev):
    """[32768 x 1024] bf16 with 1% outlier channels: bytes and scale equal the oracle's."""
    x = config2_input()
    xh = bits(x)
    q, s = G.tcast(x.to(dev))
    oq, od, _ = O.tcast(xh)
    assert s.item() == od
    assert np.array_equal(qb(q), oq)


def test_config2_fp32_bitexact(dev):
    x = config2_input(rows=4096).float() * 0.37
    q, s = G.tcast(x.to(dev))
    oq, od, _ = O.tcast(x.numpy())
    assert s.item() == od and np.array_equal(qb(q), oq)


def test_hw_e4m3_conversion_exhaustive(dev):
    """Every fp32 magnitude in [0, 448], both signs, through the product cast: the input's amax is 448, so the scale
    is exactly 1 and each byte is e4m3(x) -- gfx950's conversion against the oracle's (itself equal to torch's)."""
    top = int(np.float32(448.0).view(np.uint32)) + 1
    chunk = 1 << 28
    for sign_bit in (0, 1 << 31):
        for s0 in range(0, top, chunk):
            s1 = min(s0 + chunk, top)
            u = torch.arange(s0, s1, dtype=torch.int64, device=dev).bitwise_or(sign_bit).to(torch.int32)
            x = torch.cat([u.view(torch.float32), torch.tensor([448.0], device=dev)])
            q, s = G.tcast(x)
            assert s.item() == 1.0
            f = (np.arange(s0, s1, dtype=np.uint32) | np.uint32(sign_bit)).view(np.float32)
            bad = np.flatnonzero(qb(q)[:-1] != O.e4m3(f))
            assert bad.size == 0, f"first mismatch at fp32 {f[bad[0]]!r}"
            del u, x, q


def test_tcast_t_matches_oracle(dev):
    g = torch.Generator().manual_seed(11)
    for rows, cols, dt in ((1000, 1024, torch.bfloat16), (77, 48, torch.float32), (3, 16, torch.bfloat16)):
        x = (torch.randn(rows, cols, generator=g) * 7).to(dt)
        q, qt, s = G.tcast_t(x.to(dev))
        xn = bits(x) if dt == torch.bfloat16 else x.numpy()
        oq, od, _ = O.tcast(xn)
        r16 = (rows + 15) // 16 * 16
        assert s.item() == od and np.array_equal(qb(q), oq)
        qtn = qb(qt)
        assert qtn.shape == (cols, r16)
        assert np.array_equal(qtn[:, :rows], oq.T) and not qtn[:, rows:].any()


@pytest.mark.parametrize("rows,cols", [(4099, 4112), (8193, 16400)])
def test_tcast_t_large_ragged(dev, rows, cols):
    """Both bf16 transposing kernels: 1089 tiles on the persistent grid (some workgroups take two tiles, the second
    prefetched) and 8385 tiles, past the persistent limit (one tile per workgroup). q equals the flat cast's bytes,
    qt its transpose with zero padding."""
    g = torch.Generator(device=dev).manual_seed(rows)
    x = (torch.randn(rows, cols, generator=g, device=dev) * 5).to(torch.bfloat16)
    q, qt, s = G.tcast_t(x)
    qf, sf = G.tcast(x)
    r16 = (rows + 15) // 16 * 16
    assert s.item() == sf.item() and torch.equal(q.view(torch.uint8), qf.view(torch.uint8))
    qtb = qt.view(torch.uint8)
    assert qtb.shape == (cols, r16) and torch.equal(qtb[:, :rows], q.view(torch.uint8).t())
    assert not qtb[:, rows:].any()


def test_transpose_invariant(dev):
    """tcast_t(w).qt == tcast(w.t().contiguous()).q: the reference casts the transposed weight (fp8_native.py:259)."""
    w = (torch.randn(1024, 4096, device=dev) / 64).to(torch.bfloat16)
    _, qt, s1 = G.tcast_t(w, False)
    q2, s2 = G.tcast(w.t().contiguous())
    assert s1.item() == s2.item() and torch.equal(qt.view(torch.uint8), q2.view(torch.uint8))


def test_misaligned_and_strided_inputs(dev):
    base = config2_input(rows=64, cols=256).to(dev)
    x = base.view(-1)[3:3 + 5000]             # 6-byte offset: not 16-byte aligned
    q, s = G.tcast(x)
    oq, od, _ = O.tcast(bits(x))
    assert s.item() == od and np.array_equal(qb(q), oq)
    xs = base[:, ::2]                          # non-contiguous view
    q, s = G.tcast(xs)
    oq, od, _ = O.tcast(bits(xs))
    assert s.item() == od and np.array_equal(qb(q), oq)


def test_nan_and_inf_rules(dev):
    x = config2_input(rows=16, cols=64)
    x[3, 5] = float("nan")
    x[9, 1] = -float("nan")
    q, s = G.tcast(x.to(dev))
    oq, od, _ = O.tcast(bits(x))
    assert s.item() == od and np.array_equal(qb(q), oq)
    x[0, 0] = float("inf")                     # amax inf -> scale 0: finite values -> 0, inf * 0 -> -448
    q, s = G.tcast(x.to(dev))
    oq, od, _ = O.tcast(bits(x))
    assert np.isinf(s.item()) and np.isinf(od) and np.array_equal(qb(q), oq)


def test_other_float_dtypes_widen(dev):
    x = torch.randn(333, 17, device=dev).to(torch.float16)
    q, s = G.tcast(x)
    q2, s2 = G.tcast(x.float())
    assert s.item() == s2.item() and torch.equal(q.view(torch.uint8), q2.view(torch.uint8))


@pytest.fixture
def single_pass_default():
    L.set_single_pass(True, -1)
    yield
    L.set_single_pass(True, -1)


def test_single_pass_taken_when_the_tensor_fits(dev, single_pass_default):
    """Config 2 ([32768 x 1024] bf16) fits the single-pass kernels (the flat cast's wide kernel holds 100 MiB in
    registers and LDS, the transposing one 64 MiB in registers): the flat and the transposing cast each write new
    tagged partials and match the oracle; a tensor of 3x the size takes the flat hybrid (held + streamed, new tags)
    with the oracle's bytes; one of 15x (960 MiB, past the hybrid's 8 x 100 MiB) takes the two-pass path (the partial
    words unchanged): five copies of the 3x tensor, so its bytes are five copies of the 3x result. No partial had to
    be computed from x."""
    x = config2_input()
    xh = bits(x)
    oq, od, _ = O.tcast(xh)
    xd = x.to(dev)
    w0, f0 = once_state(dev)
    q, s = G.tcast(xd)
    w1, _ = once_state(dev)
    assert w1 >> 32 != w0 >> 32
    assert s.item() == od and np.array_equal(qb(q), oq)
    q, qt, s = G.tcast_t(xd)
    w2, f2 = once_state(dev)
    assert w2 >> 32 != w1 >> 32 and f2 == f0
    assert s.item() == od and np.array_equal(qb(q), oq)
    assert torch.equal(qt.view(torch.uint8), q.view(torch.uint8).t())
    big = torch.cat([xd, xd * 2, xd * 0.5], dim=1)
    q, s = G.tcast(big)
    w3, f3 = once_state(dev)
    assert w3 >> 32 != w2 >> 32 and f3 == f0
    oq, od, _ = O.tcast(bits(big.cpu()))
    assert s.item() == od and np.array_equal(qb(q), oq)
    huge = big.repeat(1, 5)
    qh, sh = G.tcast(huge)
    w4, f4 = once_state(dev)
    assert w4 == w3 and f4 == f0
    assert sh.item() == s.item()
    assert torch.equal(qh.view(torch.uint8).view(32768, 5, 3072), q.view(torch.uint8).unsqueeze(1).expand(-1, 5, -1))


def test_single_pass_direct_fallback_and_two_pass_agree(dev, single_pass_default):
    """The same tensors through the single pass with its normal wait, with a zero wait (every partial not yet
    published is computed by the waiting workgroup from x: the path that keeps the single pass exact when other work
    holds CUs) and through the forced two-pass path: identical bytes and scales, equal to the oracle's."""
    g = torch.Generator(device=dev).manual_seed(3)
    cases = [(torch.randn(4096, 1024, generator=g, device=dev) * 3).to(torch.bfloat16),
             (torch.randn(777, 4096, generator=g, device=dev) / 64),                      # fp32 weight
             (torch.randn(1_000_003, generator=g, device=dev)).to(torch.bfloat16)]         # flat with a tail
    cases[0][17, 5] = float("nan")
    cases[2][999_999] = -88.0
    for x in cases:
        xn = bits(x.cpu()) if x.dtype == torch.bfloat16 else x.cpu().numpy()
        oq, od, _ = O.tcast(xn)
        outs = []
        for enabled, wait in ((True, -1), (True, 0), (False, -1)):
            L.set_single_pass(enabled, wait)
            _, f0 = once_state(dev)
            q, s = G.tcast(x)
            _, f1 = once_state(dev)
            if enabled and wait == 0:
                assert f1 > f0          # the direct computation did run
            outs.append((qb(q), s.item()))
            if x.dim() == 2 and x.dtype == torch.bfloat16:
                q2, qt2, s2 = G.tcast_t(x)
                assert np.array_equal(qb(q2), qb(q)) and s2.item() == s.item()
                assert torch.equal(qt2.view(torch.uint8)[:, :x.shape[0]], q2.view(torch.uint8).t())
        L.set_single_pass(True, -1)
        for q, s in outs:
            assert s == od and np.array_equal(q, oq)


@pytest.mark.parametrize("n", [41_000_007, 1_000_003])
def test_nan_inf_tail_both_paths(dev, n):
    """NaNs (ignored by the amax), an odd tail (n % 16 != 0) and a planted maximum, on a flat bf16 tensor above the
    single-pass capacity (the hybrid: held words + streamed ones) and one below it (single pass): bytes and scale equal
    the oracle's."""
    g = torch.Generator(device=dev).manual_seed(n)
    x = (torch.randn(n, generator=g, device=dev) * 3).to(torch.bfloat16)
    x[::1_000_001] = float("nan")
    x[n // 3] = -float("nan")
    x[n - 2] = 977.0                       # the maximum sits in the tail
    q, s = G.tcast(x)
    oq, od, _ = O.tcast(bits(x))
    assert s.item() == od and np.array_equal(qb(q), oq)


def test_fp32_weight_both_paths(dev):
    """fp32 (DDP) weights: [2048 x 4096] fits the single-pass fp32 kernel, [5000 x 4096] takes its hybrid."""
    for rows in (2048, 5000):
        w = torch.randn(rows, 4096, device=dev) / 64
        w[rows // 2, 7] = -3.5
        q, s = G.tcast(w)
        oq, od, _ = O.tcast(w.cpu().numpy())
        assert s.item() == od and np.array_equal(qb(q), oq)


def test_single_pass_back_to_back_calls(dev):
    """Forty stream-ordered calls with no host synchronisation between them, alternating single-pass tensors of
    different amax with two-pass ones on the same workspace: each result is checked afterwards against the first by
    the power-of-two scale invariance (same bytes, dequant scale times 2^k)."""
    g = torch.Generator(device=dev).manual_seed(5)
    x = (torch.randn(4096, 1024, generator=g, device=dev) * 2).to(torch.bfloat16)
    y = (torch.randn(6000, 8192, generator=g, device=dev)).to(torch.bfloat16)   # 49M elements: the flat hybrid
    outs = []
    for i in range(40):
        k = i % 5 - 2
        if i % 4 == 3:
            outs.append(("y", G.tcast(y)))
        else:
            outs.append((k, G.tcast_t(x * 2.0 ** k)))
    q0, qt0, s0 = G.tcast_t(x)
    qy, sy = G.tcast(y)
    for k, out in outs:
        if k == "y":
            assert torch.equal(out[0].view(torch.uint8), qy.view(torch.uint8)) and out[1].item() == sy.item()
        else:
            q, qt, s = out
            assert torch.equal(q.view(torch.uint8), q0.view(torch.uint8))
            assert torch.equal(qt.view(torch.uint8), qt0.view(torch.uint8))
            assert s.item() == s0.item() * 2.0 ** k


def test_single_pass_concurrent_streams(dev, single_pass_default):
    """Two streams (default priority, separate workspaces) cast config-2-size tensors at the same time, so the two
    single-pass grids compete for the CUs and not every workgroup is resident while the others wait: waits run out,
    missing partial maxima are computed from x and shared between the waiters, and every result equals the one
    computed alone (bytes and scale), flat and transposing."""
    g = torch.Generator(device=dev).manual_seed(21)
    xs = [(torch.randn(32768, 1024, generator=g, device=dev) * (1 + 3 * i)).to(torch.bfloat16) for i in range(3)]
    ref = [G.tcast(x) for x in xs]
    ref_t = [G.tcast_t(x) for x in xs]
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)
    out1, out2 = [], []
    with torch.cuda.stream(s1):
        for _ in range(3):
            for x in xs:
                out1.append(G.tcast(x))
    with torch.cuda.stream(s2):
        for _ in range(3):
            for x in reversed(xs):
                out2.append(G.tcast_t(x))
    torch.cuda.synchronize()
    for i, (q, s) in enumerate(out1):
        rq, rs = ref[i % 3]
        assert s.item() == rs.item() and torch.equal(q.view(torch.uint8), rq.view(torch.uint8))
    for i, (q, qt, s) in enumerate(out2):
        rq, rqt, rs = ref_t[2 - i % 3]
        assert s.item() == rs.item() and torch.equal(q.view(torch.uint8), rq.view(torch.uint8))
        assert torch.equal(qt.view(torch.uint8), rqt.view(torch.uint8))


def test_single_pass_beside_a_persistent_gemm(dev, single_pass_default):
    """A persistent GEMM (one workgroup holding all 160 KiB of LDS on every CU) runs on one stream while single-pass
    casts run on another: the casts' workgroups find CUs only as the GEMM's leave them, so their grids start piecemeal
    and the bounded waits run out. Every result equals the one computed alone (bytes and scale), for casts issued
    before, during and after the GEMMs."""
    g = torch.Generator(device=dev).manual_seed(23)
    xs = [(torch.randn(32768, 1024, generator=g, device=dev) * (1 + 2 * i)).to(torch.bfloat16) for i in range(3)]
    ref = [G.tcast(x) for x in xs]
    a = torch.randn(32768, 1024, generator=g, device=dev).to(torch.bfloat16)
    b = (torch.randn(8192, 1024, generator=g, device=dev) / 32).to(torch.bfloat16)
    aq, sa = G.tcast(a)
    bq, sb = G.tcast(b)
    y0 = G.fp8_gemm(aq, sa, bq, sb)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)
    outs, ys = [], []
    for order in range(3):
        if order == 0:          # casts first, the GEMMs right behind them
            with torch.cuda.stream(s2):
                outs += [G.tcast(x) for x in xs]
            with torch.cuda.stream(s1):
                ys += [G.fp8_gemm(aq, sa, bq, sb) for _ in range(2)]
        else:                   # GEMMs first (order 1) or between two casts (order 2)
            with torch.cuda.stream(s1):
                ys += [G.fp8_gemm(aq, sa, bq, sb) for _ in range(2)]
            with torch.cuda.stream(s2):
                outs += [G.tcast(x) for x in (xs if order == 1 else reversed(xs))]
        torch.cuda.synchronize()
    for i, (q, s) in enumerate(outs):
        rq, rs = ref[i % 3] if i < 6 else ref[2 - i % 3]
        assert s.item() == rs.item() and torch.equal(q.view(torch.uint8), rq.view(torch.uint8)), i
    for y in ys:
        assert torch.equal(y.view(torch.int16), y0.view(torch.int16))


@pytest.mark.parametrize("shape,dtype", [((32768, 3072), torch.bfloat16), ((41_000_009,), torch.bfloat16),
                                         ((100_000_007,), torch.bfloat16), ((8192, 4096), torch.float32),
                                         ((6_553_600 * 8 * 8,), torch.bfloat16)])
def test_flat_hybrid_matches_two_pass(dev, shape, dtype, single_pass_default):
    """Flat bf16 casts above 48 MiB take the wide single-pass kernel (one 1024-thread workgroup per CU holding
    100 MiB in registers and LDS), and past its capacity, up to 8x it, its hybrid (every workgroup holds its share,
    the rest is streamed twice); fp32 above 48 MiB the 256-thread kernel's hybrid. The same bytes and scale as the
    forced two-pass path and as the zero-wait path (missing partials, streamed part included, computed from x), with
    a NaN, an infinity and an odd tail: the [32768 x 3072] dY of qkv (also against the oracle), 41M elements (held
    whole, a tail of 1), 100M (a hybrid with a tail of 7), an fp32 weight-gradient-sized tensor and the wide hybrid's
    exact 8x edge (419M elements, 800 MiB)."""
    g = torch.Generator(device=dev).manual_seed(len(shape) + shape[0])
    x = (torch.randn(*shape, generator=g, device=dev) * 4).to(dtype)
    flat = x.view(-1)
    flat[flat.numel() // 3] = float("nan")
    flat[flat.numel() - 1] = 1.0e4
    flat[flat.numel() // 2] = -float("inf") if dtype == torch.float32 else -3.0e3
    outs = []
    for enabled, wait in ((True, -1), (False, -1), (True, 0)):
        L.set_single_pass(enabled, wait)
        _, f0 = once_state(dev)
        q, s = G.tcast(x)
        _, f1 = once_state(dev)
        if enabled and wait == 0:
            assert f1 > f0
        outs.append((q.view(torch.uint8).clone(), s.item()))
        del q
    L.set_single_pass(True, -1)
    q0, s0 = outs[0]
    for q, s in outs[1:]:
        assert s == s0 and torch.equal(q, q0)
    if shape == (32768, 3072):
        oq, od, _ = O.tcast(bits(x.cpu()))
        assert s0 == od and np.array_equal(q0.cpu().numpy(), oq)


@pytest.mark.parametrize("rows,cols", [(5000, 7008), (9000, 9008), (32768, 3072), (32768, 4096)])
def test_tcast_t_hybrid_matches_two_pass(dev, rows, cols, single_pass_default):
    """Transposing casts of 2049..8192 tiles take the hybrid single pass (two tiles per workgroup held in registers,
    the rest streamed twice): the same bytes and scale as the forced two-pass path and as the zero-wait path (missing
    partials computed from x), ragged in both dimensions, with a NaN and an infinity planted; the [32768 x 3072] dY of
    qkv also against the oracle."""
    g = torch.Generator(device=dev).manual_seed(rows + cols)
    x = (torch.randn(rows, cols, generator=g, device=dev) * 4).to(torch.bfloat16)
    x[rows // 3, cols // 5] = float("nan")
    x[rows - 1, cols - 1] = 1.0e4
    outs = []
    for enabled, wait in ((True, -1), (False, -1), (True, 0)):
        L.set_single_pass(enabled, wait)
        q, qt, s = G.tcast_t(x)
        outs.append((q.view(torch.uint8).clone(), qt.view(torch.uint8).clone(), s.item()))
        del q, qt
    L.set_single_pass(True, -1)
    q0, qt0, s0 = outs[0]
    r16 = (rows + 15) // 16 * 16
    assert qt0.shape == (cols, r16) and torch.equal(qt0[:, :rows], q0.t()) and not qt0[:, rows:].any()
    for q, qt, s in outs[1:]:
        assert s == s0 and torch.equal(q, q0) and torch.equal(qt, qt0)
    if (rows, cols) == (32768, 3072):
        oq, od, _ = O.tcast(bits(x.cpu()))
        assert s0 == od and np.array_equal(q0.cpu().numpy(), oq)
