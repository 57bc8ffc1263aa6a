"""GPU parity of the SwiGLU kernels (gpic_fp8_swiglu_tcast / _bwd and their transposing variants) against the oracle
(bit-exact) and the torch-written golden vectors (bit-exact for the product cast, within 1 bf16 ulp for dz, whose
sigmoid is this build's definition)."""
import os

import numpy as np
import pytest
import torch

import gpic_fp8 as G
from oracle import oracle as O

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


def rand_bf16(shape, scale, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def test_golden_product_cast(dev, gold):
    q, s = G.swiglu_tcast(to_bf16(gold["swiglu_z"], dev))
    assert np.array_equal(qb(q), gold["swiglu_q"]) and s.item() == gold["swiglu_s"][0]


def test_golden_bwd(dev, gold):
    dz, dzq, s = G.swiglu_bwd(to_bf16(gold["swiglu_z"], dev), to_bf16(gold["bwd_da"], dev))
    diff = np.abs(bits(dz).astype(np.int32) - gold["bwd_dz"].astype(np.int32))
    assert diff.max() <= 1 and (diff == 0).mean() > 0.99
    oz, oq, od, _ = O.swiglu_bwd(gold["swiglu_z"], gold["bwd_da"])
    assert np.array_equal(bits(dz), oz) and np.array_equal(qb(dzq), oq) and s.item() == od


def test_sigmoid_exhaustive_all_bf16(dev):
    """z1 = every bf16 value, z2 = da = 1: d2 = bf16(1 * sl) = sl and d1 = bf16(1 * g) expose the device's
    sl(z1) = bf16(z1 * sigmoid(z1)) and g(z1) = sigmoid * (1 + z1 * (1 - sigmoid)) for all 65536 inputs."""
    H = 256
    z1 = np.arange(65536, dtype=np.uint16).reshape(-1, H)
    M = z1.shape[0]
    z = np.concatenate([z1, np.full((M, H), 0x3F80, np.uint16)], axis=1)
    da = np.full((M, H), 0x3F80, np.uint16)
    dz, _, _ = G.swiglu_bwd(to_bf16(z, dev), to_bf16(da, dev))
    oz, _, _, _ = O.swiglu_bwd(z, da)
    d = bits(dz)
    nan_o = np.isnan(O.bf16_to_f32(oz))
    assert np.array_equal(np.isnan(O.bf16_to_f32(d)), nan_o)
    assert np.array_equal(d[~nan_o], oz[~nan_o])
    # and the forward product: a = bf16(sl * 1) = sl, through the cast with a common scale
    q, s = G.swiglu_tcast(to_bf16(np.where(np.isfinite(O.bf16_to_f32(z)), z, 0).astype(np.uint16), dev))
    oq, od, _ = O.swiglu_tcast(np.where(np.isfinite(O.bf16_to_f32(z)), z, 0).astype(np.uint16))
    assert s.item() == od and np.array_equal(qb(q), oq)


@pytest.mark.parametrize("M,H", [(256, 512), (33, 64), (1, 8)])
def test_product_cast_matches_oracle(dev, M, H):
    z = rand_bf16((M, 2 * H), 3.0, seed=M + H)
    q, s = G.swiglu_tcast(z.to(dev))
    oq, od, _ = O.swiglu_tcast(bits(z))
    assert s.item() == od and np.array_equal(qb(q), oq)


def test_product_cast_row_stride(dev):
    """z as a column slice of a wider tensor (row stride > 2H), as the reference allows (fp8_native.py:135)."""
    wide = rand_bf16((128, 3 * 256), 2.0, seed=5).to(dev)
    z = wide[:, :512]
    q, s = G.swiglu_tcast(z)
    oq, od, _ = O.swiglu_tcast(bits(z))
    assert s.item() == od and np.array_equal(qb(q), oq)


def test_product_cast_d12_rows(dev):
    """4096 tokens of d12's SwiGLU (H = 4096)."""
    z = rand_bf16((4096, 8192), 1.5, seed=12)
    q, s = G.swiglu_tcast(z.to(dev))
    oq, od, _ = O.swiglu_tcast(bits(z))
    assert s.item() == od and np.array_equal(qb(q), oq)


@pytest.mark.parametrize("M,H", [(200, 256), (17, 16)])
def test_bwd_matches_oracle(dev, M, H):
    z = rand_bf16((M, 2 * H), 3.0, seed=M)
    da = rand_bf16((M, H), 0.05, seed=M + 1)
    dz, dzq, s = G.swiglu_bwd(z.to(dev), da.to(dev))
    oz, oq, od, _ = O.swiglu_bwd(bits(z), bits(da))
    assert np.array_equal(bits(dz), oz) and np.array_equal(qb(dzq), oq) and s.item() == od


@pytest.mark.parametrize("M,H", [(300, 512), (33, 8), (4096, 4096)])
def test_flat_product_cast_paths_agree(dev, M, H):
    """The flat product casts give the same bytes and scale: the op's, gpic_fp8_swiglu_tcast (no product buffer) and
    gpic_fp8_swiglu_tcast_t with qt = NULL and no buffer -- all three the single pass here -- and
    gpic_fp8_swiglu_tcast_t into a strided q (the two-pass cast recomputing the product). H = 8: one word per row."""
    from gpic_fp8 import _lib as L
    z = rand_bf16((M, 2 * H), 3.0, seed=M + 3 * H).to(dev)
    q0, s0 = G.swiglu_tcast(z)
    lib, ws, st = L.lib(), L.cast_workspace(z.device), L.stream_ptr(z.device)
    outs = []
    for mode in ("plain", "t_nobuf", "t_strided"):
        sq = H + 16 if mode == "t_strided" else H
        q = torch.zeros(M, sq, dtype=torch.uint8, device=dev)
        s = torch.empty(1, device=dev)
        a = torch.empty(M, H, dtype=torch.bfloat16, device=dev) if mode == "t_strided" else None
        if mode == "plain":
            rc = lib.gpic_fp8_swiglu_tcast(z.data_ptr(), M, H, 2 * H, q.data_ptr(), sq, s.data_ptr(), ws.data_ptr(), st)
        else:
            rc = lib.gpic_fp8_swiglu_tcast_t(z.data_ptr(), M, H, 2 * H, L.ptr(a), q.data_ptr(), sq, None, 0,
                                             s.data_ptr(), ws.data_ptr(), st)
        assert rc == 0
        outs.append((mode, q[:, :H], s))
    for mode, q, s in outs:
        assert s.item() == s0.item(), mode
        assert torch.equal(q, q0.view(torch.uint8)), mode
    oq, od, _ = O.swiglu_tcast(bits(z))
    assert s0.item() == od and np.array_equal(qb(q0), oq)


@pytest.fixture
def single_pass_default():
    from gpic_fp8 import _lib as L
    L.set_single_pass(True, -1)
    yield
    L.set_single_pass(True, -1)


# (M, H): one workgroup; rows of 130 words across groups of 1024; 8 words per thread (registers only); the grid's
# exact capacity on 256 CUs (24 words per thread, 8 of them in LDS); hybrids at 1.33x, d12 (2.67x) and d18 (4.67x)
# past it.
@pytest.mark.parametrize("M,H", [(33, 64), (4100, 1040), (4096, 4096), (12288, 4096), (16384, 4096), (32768, 4096),
                                 (32768, 7168)])
def test_single_pass_product_cast(dev, M, H, single_pass_default):
    """The single-pass product cast (one launch: the product held in registers and LDS, past the grid's capacity
    streamed through the product buffer) against the forced two-pass path and the zero-wait path (a partial not yet
    published is computed by the waiting workgroup from z, streamed part included): the same bytes and scale, with a
    NaN product (excluded from the amax) and an outlier planted; the call writes a new tag. Up to 12288 rows also
    against the oracle; gpic_fp8_swiglu_tcast (no product buffer) agrees wherever the product fits."""
    from gpic_fp8 import _lib as L
    from parity import once_state
    g = torch.Generator(device=dev).manual_seed(M + H)
    z = (torch.randn(M, 2 * H, generator=g, device=dev) * 2).to(torch.bfloat16)
    z[M // 3, H // 5] = float("nan")                   # z1 NaN: a NaN product
    z[M - 1, 2 * H - 1] = 300.0                         # z2 outlier: the largest product
    outs = []
    for enabled, wait in ((True, -1), (True, 0), (False, -1)):
        L.set_single_pass(enabled, wait)
        w0, f0 = once_state(dev)
        q, s = G.swiglu_tcast(z)
        w1, f1 = once_state(dev)
        if enabled:
            assert w1 >> 32 != w0 >> 32                  # the single pass ran
        else:
            assert w1 == w0
        if enabled and wait == 0 and M * H // 8 > 512:
            assert f1 > f0                               # the direct computation did run (more than one workgroup)
        outs.append((q.view(torch.uint8).clone(), s.item()))
        del q
    L.set_single_pass(True, -1)
    q0, s0 = outs[0]
    for q, s in outs[1:]:
        assert s == s0 and torch.equal(q, q0)
    if M * H <= 4096 * 12288:
        oq, od, _ = O.swiglu_tcast(bits(z))
        assert s0 == od and np.array_equal(q0.cpu().numpy(), oq)
    if M * H // 8 <= 12288 * 512:
        q = torch.zeros(M, H, dtype=torch.uint8, device=dev)
        s = torch.empty(1, device=dev)
        assert L.lib().gpic_fp8_swiglu_tcast(z.data_ptr(), M, H, 2 * H, q.data_ptr(), H, s.data_ptr(),
                                             L.cast_workspace(dev).data_ptr(), L.stream_ptr(dev)) == 0
        assert s.item() == s0 and torch.equal(q, q0)


# (M, H): one workgroup; rows of 258 units across groups of 1024; 2 units per thread (registers only); the grid's
# exact capacity on 256 CUs (10 units per thread, 4 of them in LDS); hybrids at 1.6x, d12 (6.4x) and d18 (11.2x) past
# it.
@pytest.mark.parametrize("M,H", [(33, 16), (1000, 2064), (8192, 512), (5120, 4096), (8192, 4096), (32768, 4096),
                                 (32768, 7168)])
def test_single_pass_bwd_cast(dev, M, H, single_pass_default):
    """The single-pass cast of dz without dz in memory (one launch: dz held in registers and LDS, past the grid's
    capacity computed for the maximum and again after the fold) against the forced two-pass path (an amax pass, then
    the recomputing cast) and the zero-wait path: the same bytes and scale, with NaN and infinity planted in z and da;
    the call writes a new tag. Up to 5120 x 4096 also against the oracle."""
    from gpic_fp8 import _lib as L
    from parity import once_state
    g = torch.Generator(device=dev).manual_seed(M + 2 * H)
    z = (torch.randn(M, 2 * H, generator=g, device=dev) * 2).to(torch.bfloat16)
    da = (torch.randn(M, H, generator=g, device=dev) * 0.01).to(torch.bfloat16)
    z[M // 3, H // 5] = float("nan")
    da[M // 2, H - 1] = float("inf")
    z[M - 1, 2 * H - 1] = 300.0
    outs = []
    for enabled, wait in ((True, -1), (True, 0), (False, -1)):
        L.set_single_pass(enabled, wait)
        w0, f0 = once_state(dev)
        q, s = G.swiglu_bwd_q(z, da)
        w1, f1 = once_state(dev)
        if enabled:
            assert w1 >> 32 != w0 >> 32                  # the single pass ran
        else:
            assert w1 == w0
        if enabled and wait == 0 and M * H // 8 > 1024:
            assert f1 > f0                               # the direct computation did run (more than one workgroup)
        outs.append((q.view(torch.uint8).clone(), s.item()))
        del q
    L.set_single_pass(True, -1)
    q0, s0 = outs[0]
    for q, s in outs[1:]:
        assert s == s0 and torch.equal(q, q0)
    if M * H <= 5120 * 4096:
        _, oq, od, _ = O.swiglu_bwd(bits(z), bits(da))
        assert s0 == od and np.array_equal(q0.cpu().numpy(), oq)


@pytest.mark.parametrize("M,H", [(1024, 1040), (16384, 4096)])
def test_single_pass_casts_strided_rows(dev, M, H, single_pass_default):
    """z and da as column slices of wider tensors (row strides 2H + 72 and H + 40, as a view of a fused projection
    would give): both single passes -- held whole, and past the grid's capacity (the product's hybrid through its
    buffer, dz computed twice) -- give the bytes and scale of the same values made contiguous; the smaller also
    against the oracle."""
    g = torch.Generator(device=dev).manual_seed(M + H + 7)
    zw = (torch.randn(M, 2 * H + 72, generator=g, device=dev) * 2).to(torch.bfloat16)
    dw = (torch.randn(M, H + 40, generator=g, device=dev) * 0.01).to(torch.bfloat16)
    z, da = zw[:, 8:8 + 2 * H], dw[:, 16:16 + H]
    assert z.stride(0) == 2 * H + 72 and da.stride(0) == H + 40
    q, s = G.swiglu_tcast(z)
    q0, s0 = G.swiglu_tcast(z.contiguous())
    assert s.item() == s0.item() and torch.equal(q.view(torch.uint8), q0.view(torch.uint8))
    dq, sd = G.swiglu_bwd_q(z, da)
    dq0, sd0 = G.swiglu_bwd_q(z.contiguous(), da.contiguous())
    assert sd.item() == sd0.item() and torch.equal(dq.view(torch.uint8), dq0.view(torch.uint8))
    if M * H <= 1024 * 1040:
        oq, od, _ = O.swiglu_tcast(bits(z))
        assert s.item() == od and np.array_equal(qb(q), oq)
        _, oq, od, _ = O.swiglu_bwd(bits(z), bits(da))
        assert sd.item() == od and np.array_equal(qb(dq), oq)


def test_single_pass_casts_beside_a_persistent_gemm(dev, single_pass_default):
    """The single-pass SwiGLU casts (one 1024-thread workgroup per CU, all of its LDS) on one stream while a
    persistent GEMM holds every CU from another: their workgroups start only as the GEMM's leave, the bounded waits
    run out and missing partials are computed from z (and da). Every result equals the one computed alone -- product
    casts of a product that fits and of one that streams, the backward's cast of a hybrid -- issued before and after
    the GEMMs."""
    g = torch.Generator(device=dev).manual_seed(29)
    zs = [(torch.randn(m, 8192, generator=g, device=dev) * (1 + i)).to(torch.bfloat16)
          for i, m in enumerate((4096, 16384))]
    da = (torch.randn(8192, 4096, generator=g, device=dev) * 0.01).to(torch.bfloat16)
    calls = [lambda: G.swiglu_tcast(zs[0]), lambda: G.swiglu_tcast(zs[1]), lambda: G.swiglu_bwd_q(zs[1][:8192], da)]
    ref = [f() for f in calls]
    a = torch.randn(32768, 1024, generator=g, device=dev).to(torch.bfloat16)
    b = (torch.randn(8192, 1024, generator=g, device=dev) / 32).to(torch.bfloat16)
    aq, sa = G.tcast(a)
    bq, sb = G.tcast(b)
    y0 = G.fp8_gemm(aq, sa, bq, sb)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)
    outs, ys = [], []
    for order in range(2):
        if order == 0:          # casts first, the GEMMs right behind them
            with torch.cuda.stream(s2):
                outs += [f() for f in calls]
            with torch.cuda.stream(s1):
                ys += [G.fp8_gemm(aq, sa, bq, sb) for _ in range(2)]
        else:                   # GEMMs first
            with torch.cuda.stream(s1):
                ys += [G.fp8_gemm(aq, sa, bq, sb) for _ in range(2)]
            with torch.cuda.stream(s2):
                outs += [f() for f in calls]
        torch.cuda.synchronize()
    for i, (q, s) in enumerate(outs):
        rq, rs = ref[i % len(calls)]
        assert s.item() == rs.item() and torch.equal(q.view(torch.uint8), rq.view(torch.uint8)), i
    for y in ys:
        assert torch.equal(y.view(torch.int16), y0.view(torch.int16))


def test_transposing_variants(dev):
    M, H = 300, 512
    z = rand_bf16((M, 2 * H), 2.0, seed=9).to(dev)
    da = rand_bf16((M, H), 0.1, seed=10).to(dev)
    q, s = G.swiglu_tcast(z)
    q2, qt, s2 = G.swiglu_tcast_t(z)
    m16 = (M + 15) // 16 * 16
    assert s.item() == s2.item() and torch.equal(q.view(torch.uint8), q2.view(torch.uint8))
    assert qt.shape == (H, m16) and torch.equal(qt.view(torch.uint8)[:, :M], q.view(torch.uint8).t())
    assert not qt.view(torch.uint8)[:, M:].any()
    dz, dq, sd = G.swiglu_bwd(z, da)
    dz2, dq2, dqt, sd2 = G.swiglu_bwd_t(z, da)
    assert torch.equal(dz.view(torch.int16), dz2.view(torch.int16)) and sd.item() == sd2.item()
    assert torch.equal(dq.view(torch.uint8), dq2.view(torch.uint8))
    assert torch.equal(dqt.view(torch.uint8)[:, :M], dq.view(torch.uint8).t())
    assert not dqt.view(torch.uint8)[:, M:].any()


@pytest.mark.parametrize("M,H", [(300, 512), (33, 16), (1000, 2064), (4100, 1040)])
def test_bwd_t_without_dz_matches(dev, M, H):
    """swiglu_bwd_t(want_dz=False) never writes dz: it casts dz recomputed from z and da, tile by tile for both halves.
    Same dzq, dzqt and scale as the path through dz, and as the oracle; ragged M and H (partial 128-tiles in both)."""
    z = rand_bf16((M, 2 * H), 3.0, seed=M + H)
    da = rand_bf16((M, H), 0.05, seed=M + H + 1)
    z[0, :5] = torch.tensor([0.0, -0.0, 1e-30, 300.0, -300.0]).to(torch.bfloat16)   # sigmoid outside the table range
    zd, dad = z.to(dev), da.to(dev)
    dz, dq, dqt, s = G.swiglu_bwd_t(zd, dad)
    dz0, dq0, dqt0, s0 = G.swiglu_bwd_t(zd, dad, False)
    assert dz0.numel() == 0 and s0.item() == s.item()
    assert torch.equal(dq0.view(torch.uint8), dq.view(torch.uint8))
    assert torch.equal(dqt0.view(torch.uint8), dqt.view(torch.uint8))
    _, oq, od, _ = O.swiglu_bwd(bits(z), bits(da))
    assert np.array_equal(qb(dq0), oq) and s0.item() == od


@pytest.mark.parametrize("M,H", [(300, 512), (33, 16), (1000, 2064), (4100, 1040)])
def test_bwd_flat_without_dz_matches(dev, M, H):
    """swiglu_bwd_q never writes dz: the flat cast recomputes dz from z and da. Same dzq and scale as the path through
    dz (swiglu_bwd), and as the oracle; row counts that leave the 4-row batches with a remainder."""
    z = rand_bf16((M, 2 * H), 3.0, seed=M + 2 * H)
    da = rand_bf16((M, H), 0.05, seed=M + 2 * H + 1)
    z[0, :5] = torch.tensor([0.0, -0.0, 1e-30, 300.0, -300.0]).to(torch.bfloat16)   # sigmoid outside the table range
    zd, dad = z.to(dev), da.to(dev)
    dz, dq, s = G.swiglu_bwd(zd, dad)
    dq0, s0 = G.swiglu_bwd_q(zd, dad)
    assert s0.item() == s.item()
    assert torch.equal(dq0.view(torch.uint8), dq.view(torch.uint8))
    _, oq, od, _ = O.swiglu_bwd(bits(z), bits(da))
    assert np.array_equal(qb(dq0), oq) and s0.item() == od


def test_bwd_flat_without_dz_full_size(dev):
    """The d12 shape (M 32768, H 4096) with NaN and inf planted: the flat cast without dz gives the bytes of the
    path through dz."""
    g = torch.Generator(device=dev).manual_seed(13)
    z = (torch.randn(32768, 8192, generator=g, device=dev) * 2).to(torch.bfloat16)
    da = (torch.randn(32768, 4096, generator=g, device=dev) * 0.01).to(torch.bfloat16)
    z[7, 5] = float("nan")
    da[200, 9] = -float("inf")
    z[30000, 100] = float("inf")
    dz, dq, s = G.swiglu_bwd(z, da)
    dq0, s0 = G.swiglu_bwd_q(z, da)
    assert s0.item() == s.item()
    assert torch.equal(dq0.view(torch.uint8), dq.view(torch.uint8))


def test_bwd_t_without_dz_full_size(dev):
    """The d12 shape (M 32768, H 4096) with NaN and inf planted in z and da: both paths give the same bytes."""
    g = torch.Generator(device=dev).manual_seed(12)
    z = (torch.randn(32768, 8192, generator=g, device=dev) * 2).to(torch.bfloat16)
    da = (torch.randn(32768, 4096, generator=g, device=dev) * 0.01).to(torch.bfloat16)
    z[5, 7] = float("nan")
    da[100, 3] = float("inf")
    z[31000, 4100] = -float("inf")
    dz, dq, dqt, s = G.swiglu_bwd_t(z, da)
    _, dq0, dqt0, s0 = G.swiglu_bwd_t(z, da, False)
    assert s0.item() == s.item()
    assert torch.equal(dq0.view(torch.uint8), dq.view(torch.uint8))
    assert torch.equal(dqt0.view(torch.uint8), dqt.view(torch.uint8))


@pytest.mark.parametrize("M,H", [(1000, 256), (33, 16)])
def test_tcast_t_with_and_without_product_buffer(dev, M, H):
    """gpic_fp8_swiglu_tcast_t either writes the product a and casts it, or recomputes it inside the cast: the same
    bytes and scale; the written product equals the oracle's."""
    from gpic_fp8 import _lib as L
    z = rand_bf16((M, 2 * H), 3.0, seed=M + 31).to(dev)
    m16 = (M + 15) // 16 * 16
    out = []
    for with_a in (True, False):
        a = torch.empty(M, H, dtype=torch.bfloat16, device=dev)
        q = torch.empty(M, H, dtype=torch.uint8, device=dev)
        qt = torch.empty(H, m16, dtype=torch.uint8, device=dev)
        s = torch.empty(1, dtype=torch.float32, device=dev)
        ws = L.cast_workspace(dev)
        rc = L.lib().gpic_fp8_swiglu_tcast_t(z.data_ptr(), M, H, z.stride(0), a.data_ptr() if with_a else None,
                                             q.data_ptr(), H, qt.data_ptr(), m16, s.data_ptr(), ws.data_ptr(),
                                             L.stream_ptr(dev))
        assert rc == 0
        torch.cuda.synchronize()
        out.append((a, q, qt, s.item()))
    (a, q1, qt1, s1), (_, q2, qt2, s2) = out
    assert s1 == s2 and torch.equal(q1, q2) and torch.equal(qt1, qt2)
    assert np.array_equal(bits(a), O.swiglu_product(bits(z.cpu())))


def test_bwd_matches_eager_torch_within_one_ulp(dev):
    """The eager phase-1 backward (fp8_native.py:226-231, torch.sigmoid) agrees with the kernel's dz within 1 ulp."""
    M, H = 512, 1024
    z = rand_bf16((M, 2 * H), 3.0, seed=21).to(dev)
    da = rand_bf16((M, H), 0.1, seed=22).to(dev)
    dz, _, _ = G.swiglu_bwd(z, da)
    z1, z2 = z.float().chunk(2, dim=-1)
    sg = torch.sigmoid(z1)
    dz1 = (da.float() * z2 * (sg * (1 + z1 * (1 - sg)))).to(torch.bfloat16)
    dz2 = da * (z1 * sg).to(torch.bfloat16)
    ref = torch.cat([dz1, dz2], -1)
    diff = (dz.view(torch.int16).int() - ref.view(torch.int16).int()).abs()
    assert diff.max().item() <= 1 and (diff == 0).float().mean().item() > 0.99


def test_q_only_product_buffer_contract(dev):
    """The contract of `a` in gpic_fp8_swiglu_tcast_t with qt = NULL and sq == H (include/gpic_fp8.h): the single
    pass uses `a` as scratch for the rows that do not fit on chip, so a product that fits leaves `a` as it was; with
    the single pass disabled the amax pass writes the whole product there. The bytes and scale are the same and equal
    the oracle's either way."""
    from gpic_fp8 import _lib as L
    M, H = 512, 256
    z = rand_bf16((M, 2 * H), 3.0, seed=77).to(dev)
    oq, od, _ = O.swiglu_tcast(bits(z.cpu()))
    try:
        for single in (True, False):
            L.set_single_pass(single, -1)
            a = torch.full((M, H), 7.0, dtype=torch.bfloat16, device=dev)
            q = torch.empty(M, H, dtype=torch.uint8, device=dev)
            s = torch.empty(1, dtype=torch.float32, device=dev)
            rc = L.lib().gpic_fp8_swiglu_tcast_t(z.data_ptr(), M, H, z.stride(0), a.data_ptr(), q.data_ptr(), H, None,
                                                 0, s.data_ptr(), L.cast_workspace(dev).data_ptr(), L.stream_ptr(dev))
            assert rc == 0
            torch.cuda.synchronize()
            assert s.item() == od and np.array_equal(qb(q), oq)
            if single:
                assert bool((a == 7.0).all()), "the single pass wrote a product that fits on chip"
            else:
                assert np.array_equal(bits(a), O.swiglu_product(bits(z.cpu())))
    finally:
        L.set_single_pass(True, -1)
