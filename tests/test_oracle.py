"""Pins the CPU oracle (oracle/) before it is trusted to check the HIP kernels.

Each oracle function is checked against something independent of it: torch's own CPU routines (the float8 conversion,
IEEE division, sigmoid, matmul), the committed golden vectors (tests/golden, written with torch ops only), closed
forms and invariants (transpose, power-of-two scaling, exact integer GEMMs). Mutants of the oracle's rules (a truncating
e4m3 rounding, the eager reciprocal * 448 scale, a dropped clamp, a transposed operand) are shown to fail these checks.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")
E4 = torch.float8_e4m3fn


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLD, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def torch_e4m3(f):
    return torch.from_numpy(np.ascontiguousarray(f, dtype=np.float32)).to(E4).view(torch.uint8).numpy()


# ---------------------------------------------------------------- e4m3 rounding

def test_e4m3_exhaustive_against_torch():
    """Every fp32 magnitude up to 464 (the last value that still rounds to 448), both signs: 2.28e9 values."""
    top = int(np.float32(464.0).view(np.uint32)) + 1
    chunk = 1 << 26
    bad = 0
    for s in range(0, top, chunk):
        f = np.arange(s, min(s + chunk, top), dtype=np.uint32).view(np.float32)
        ref = torch_e4m3(f)
        bad += int((O.e4m3(f) != ref).sum())
        bad += int((O.e4m3(-f) != (ref | 0x80)).sum())
    assert bad == 0


def test_e4m3_specials():
    f = np.array([np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0, 448.0, 464.0, 465.0, 2.0 ** -9, 2.0 ** -10,
                  1.5 * 2.0 ** -9, 2.0 ** -6], dtype=np.float32)
    ours, ref = O.e4m3(f), torch_e4m3(f)
    # NaN payload bits aside, torch and the oracle agree on every special value
    assert (ours == ref).all(), (ours, ref)


def test_e4m3_decode_all_bytes():
    b = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(b).view(E4).float().numpy()
    ours = O.e4m3_to_f32(b)
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    m = ~np.isnan(ref)
    assert (ours[m] == ref[m]).all()
    assert O.e4m3_to_f32(np.uint8(0x7E)) == 448.0 and O.e4m3_to_f32(np.uint8(0x01)) == 2.0 ** -9


def test_e4m3_mutant_truncation_fails():
    """A truncating (round-toward-zero) e4m3 disagrees with torch on many values: the check above has teeth."""
    f = np.random.default_rng(0).standard_normal(100000).astype(np.float32) * 10
    f = np.clip(f, -448, 448)
    u = f.view(np.uint32)
    trunc = O.e4m3_to_f32(O.e4m3(((u >> 20) << 20).view(np.float32)))   # chop the mantissa to 3 bits
    assert (O.e4m3(trunc) != torch_e4m3(f)).mean() > 0.1


# ---------------------------------------------------------------- amax and scales

def test_scales_ieee_division():
    rng = np.random.default_rng(1)
    amax = np.concatenate([rng.uniform(0, 1000, 50000), np.exp(rng.uniform(-40, 40, 50000)),
                           [0.0, 1e-13, 1e-12, 448.0]]).astype(np.float32)
    s = np.empty_like(amax)
    d = np.empty_like(amax)
    for i, a in enumerate(amax):
        s[i], d[i] = O.scales(int(np.float32(a).view(np.uint32)))
    at = torch.clamp_min(torch.from_numpy(amax), 1e-12)
    assert np.array_equal(s, torch.div(torch.tensor(448.0), at).numpy())
    assert np.array_equal(d, torch.div(at, torch.tensor(448.0)).numpy())
    # the eager 448.0 / a (reciprocal(a) * 448) is a different rule: it disagrees on a sizeable share of values
    eager = (448.0 / at).numpy()
    assert (eager != s).mean() > 0.05


def test_amax_closed_form():
    rng = np.random.default_rng(2)
    x = rng.standard_normal(10001).astype(np.float32)
    h = O.f32_to_bf16(x)
    assert O.amax_bits(h) == int(np.abs(O.bf16_to_f32(h)).max().view(np.uint32))
    assert O.amax_bits(x) == int(np.abs(x).max().view(np.uint32))
    x[17] = np.nan                                   # tl.max (maxnum) ignores NaN
    assert O.amax_bits(x) == int(np.nanmax(np.abs(x)).view(np.uint32))
    assert O.amax_bits(np.zeros(0, np.uint16)) == 0


@pytest.mark.parametrize("name", ["cast_bf16", "cast_tail", "cast_f32", "cast_range"])
def test_tcast_golden(gold, name):
    q, d, _ = O.tcast(gold[f"{name}_x"])
    assert np.array_equal(q, gold[f"{name}_q"])
    assert d == gold[f"{name}_s"][0]


def test_tcast_zero_golden(gold):
    q, d, am = O.tcast(np.zeros((16, 16), np.uint16))
    assert np.array_equal(q, gold["cast_zero_q"]) and d == gold["cast_zero_s"][0] and am == 0
    q, d, _ = O.tcast(np.zeros(0, np.uint16))
    assert q.size == 0 and d == np.float32(np.float32(1e-12) / np.float32(448.0))


def test_tcast_mutant_eager_scale_fails(gold):
    """Casting config-2-like data with the eager reciprocal * 448 scale changes bytes for some amax values."""
    rng = np.random.default_rng(3)
    changed = 0
    for _ in range(40):
        x = O.f32_to_bf16(rng.standard_normal(4096).astype(np.float32) * rng.uniform(0.1, 100))
        q, _, am = O.tcast(x)
        a = torch.tensor(np.uint32(am).view(np.float32)).clamp_min(1e-12)
        q2 = O.cast(x, np.float32((448.0 / a).item()))
        changed += int((q2 != q).any())
    assert changed > 0


def test_transpose_invariant():
    rng = np.random.default_rng(4)
    x = O.f32_to_bf16(rng.standard_normal((48, 80)).astype(np.float32))
    q, d, _ = O.tcast(x)
    qt, dt, _ = O.tcast(np.ascontiguousarray(x.T))
    assert np.array_equal(qt, q.T) and d == dt


def test_tcast_heads_is_the_permuted_cast():
    """tcast_heads: byte (b N + n, h D + d) is byte (b, h, n, d) of the cast of o in its own order, with its scale
    (one amax for any order; bytes elementwise). A mutant that merges without the transpose fails."""
    rng = np.random.default_rng(6)
    B, H, N, D = 2, 3, 5, 16
    o = O.f32_to_bf16(rng.standard_normal((B, H, N, D)).astype(np.float32))
    q, d, am = O.tcast_heads(o)
    q0, d0, am0 = O.tcast(o)
    assert d == d0 and am == am0 and q.shape == (B * N, H * D)
    for b in range(B):
        for h in range(H):
            for n in range(N):
                assert np.array_equal(q[b * N + n, h * D:(h + 1) * D], q0[b, h, n])
    assert not np.array_equal(O.tcast(o.reshape(B * N, H * D))[0], q)


def test_pow2_scale_invariant():
    rng = np.random.default_rng(5)
    x = rng.standard_normal(5000).astype(np.float32)
    q, d, _ = O.tcast(x)
    for k in (-20, -3, 1, 7, 30):
        qk, dk, _ = O.tcast((x * np.float32(2.0 ** k)).astype(np.float32))
        assert np.array_equal(qk, q) and dk == np.float32(d * np.float32(2.0 ** k))


def test_cast_clamp_and_nan_rule():
    """x * scale beyond +-448 saturates (tl.minimum / tl.maximum); a NaN product saturates to -448 (maxNum)."""
    x = np.array([1.0, -1.0, 500.0, -500.0, np.nan, np.inf, -np.inf], np.float32)
    q = O.cast(x, np.float32(448.0))
    assert list(q) == [0x7E, 0xFE, 0x7E, 0xFE, 0xFE, 0x7E, 0xFE]


# ---------------------------------------------------------------- SwiGLU

def test_exp_accuracy_all_bf16():
    h = np.arange(65536, dtype=np.uint16)
    f = O.bf16_to_f32(h)
    ok = np.isfinite(f) & (f > -87) & (f < 88)
    e = O.exp(f[ok]).astype(np.float64)
    ex = np.array([math.exp(v) for v in f[ok].astype(np.float64)])
    ulp = np.abs(e - ex) / np.spacing(ex.astype(np.float32)).astype(np.float64)
    assert ulp.max() <= 1.0
    assert O.exp(np.float32([0.0]))[0] == 1.0 and O.exp(np.float32([-np.inf]))[0] == 0.0


def test_sigmoid_against_torch_all_bf16():
    f = O.bf16_to_f32(np.arange(65536, dtype=np.uint16))
    fin = np.isfinite(f)
    ours = O.sigmoid(f[fin])
    ref = torch.sigmoid(torch.from_numpy(f[fin])).numpy()
    ulp = np.abs(ours.astype(np.float64) - ref) / np.maximum(np.spacing(np.abs(ref)), 1e-45)
    assert ulp.max() <= 2 and (ours == ref).mean() > 0.99


def test_silu_table_equals_torch_all_bf16():
    """sl = bf16(z1 * sigmoid(z1)) equals torch's eager value for every finite bf16 z1 (so the SwiGLU product, a
    function of sl and z2, is torch's to the bit)."""
    h = np.arange(65536, dtype=np.uint16)
    fin = np.isfinite(O.bf16_to_f32(h))
    z1 = torch.from_numpy(h.view(np.int16)).view(torch.bfloat16).float()
    ref = (z1 * torch.sigmoid(z1)).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.swiglu_table()[fin], ref[fin])


def test_swiglu_tcast_golden(gold):
    z = gold["swiglu_z"]
    assert np.array_equal(O.swiglu_product(z), gold["swiglu_a"])
    q, d, _ = O.swiglu_tcast(z)
    assert np.array_equal(q, gold["swiglu_q"]) and d == gold["swiglu_s"][0]


def test_swiglu_bwd_golden(gold):
    z, da = gold["swiglu_z"], gold["bwd_da"]
    dz, dzq, d, _ = O.swiglu_bwd(z, da)
    ref = gold["bwd_dz"]
    diff = np.abs(dz.astype(np.int32) - ref.astype(np.int32))
    assert diff.max() <= 1 and (diff == 0).mean() > 0.99          # within 1 bf16 ulp of torch's sigmoid
    q2, d2, _ = O.tcast(dz)                                         # the bytes are the cast of dz itself
    assert np.array_equal(q2, dzq) and d2 == d


def test_swiglu_bwd_mutant_fused_fails():
    """Fusing 1 + z1 * (1 - sg) into one fma changes some dz values: the bwd rounding order is pinned. (Such a change
    moves g by an fp32 ulp, which flips dz's bf16 rounding about once per 3e4 elements: 4M elements are checked.)"""
    rng = np.random.default_rng(6)
    M, H = 1024, 4096
    z = O.f32_to_bf16(rng.standard_normal((M, 2 * H)).astype(np.float32) * 3)
    da = O.f32_to_bf16(rng.standard_normal((M, H)).astype(np.float32))
    dz, _, _, _ = O.swiglu_bwd(z, da)
    sg_tab = O.sigmoid(O.bf16_to_f32(np.arange(65536, dtype=np.uint16)))
    z1 = O.bf16_to_f32(z[:, :H])
    z2 = O.bf16_to_f32(z[:, H:])
    dav = O.bf16_to_f32(da)
    sg = sg_tab[z[:, :H]]
    unfused = (np.float32(1) + z1 * (np.float32(1) - sg)).astype(np.float32)
    fused = (z1.astype(np.float64) * (np.float32(1) - sg).astype(np.float64) + 1).astype(np.float32)
    d1u = O.f32_to_bf16((dav * z2) * (sg * unfused))
    d1f = O.f32_to_bf16((dav * z2) * (sg * fused))
    assert np.array_equal(d1u, dz[:, :H])          # the oracle is the unfused expression
    assert (d1f != dz[:, :H]).sum() > 0


# ---------------------------------------------------------------- GEMM

def test_mm_exact_golden(gold):
    c = O.mm(gold["gemm_a"], gold["gemm_sa"][0], gold["gemm_b"], gold["gemm_sb"][0])
    assert np.array_equal(c, gold["gemm_c"])
    cb = O.mm(gold["gemm_a"], gold["gemm_sa"][0], gold["gemm_b"], gold["gemm_sb"][0], gold["gemm_bias"])
    assert np.array_equal(cb, gold["gemm_cbias"])


def test_mm_mutant_transposed_operand_fails(gold):
    a, b = gold["gemm_a"], gold["gemm_b"]
    c = O.mm(a, 1.0, b, 1.0)
    # a swapped-operand result is C^T: a different matrix
    ct = O.mm(b, 1.0, a, 1.0)
    assert ct.shape != c.shape or not np.array_equal(ct, c)


def test_mm_identity():
    rng = np.random.default_rng(7)
    a = O.e4m3(rng.standard_normal((32, 64)).astype(np.float32) * 20)
    eye = O.e4m3(np.eye(64, dtype=np.float32))
    c = O.mm(a, np.float32(0.5), eye, np.float32(2.0))
    assert np.array_equal(c, O.f32_to_bf16(O.e4m3_to_f32(a)))


def test_mm_against_torch_fp32():
    rng = np.random.default_rng(8)
    a = O.e4m3(np.clip(rng.standard_normal((64, 256)) * 50, -448, 448).astype(np.float32))
    b = O.e4m3(np.clip(rng.standard_normal((80, 256)) * 50, -448, 448).astype(np.float32))
    ref = (torch.from_numpy(a).view(E4).float() * 0.01) @ (torch.from_numpy(b).view(E4).float() * 0.02).t()
    assert O.rel_fro(O.mm64(a, np.float32(0.01), b, np.float32(0.02)), ref.numpy()) < 1e-6


def test_linear_forward_golden(gold):
    y = O.linear_forward(gold["lin_x"], gold["lin_w"], gold["lin_b"])
    ref = O.bf16_to_f32(gold["lin_y"])
    assert O.rel_fro(O.bf16_to_f32(y), ref) < 5e-3


# ---------------------------------------------------------------- the torch-CPU restatement (the CPU baseline)

def _u16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_torch_tcast_equals_c_oracle(dtype):
    """The CPU baseline's cast (torch ops, torch.div scales) gives the C oracle's bytes and scale, outliers included."""
    g = torch.Generator().manual_seed(7)
    x = torch.randn(3000, 1024, generator=g)
    x[:, :10] *= 50.0
    x = x.to(dtype)
    q, s = O.torch_tcast(x)
    oq, od, _ = O.tcast(_u16(x) if dtype == torch.bfloat16 else x.numpy())
    assert s.item() == od and np.array_equal(q.view(torch.uint8).numpy(), oq)


def test_torch_mm_equals_reference_formula_and_c_oracle(gold):
    """The baseline's GEMM is reference()'s fp32 product of the dequantized bytes: on the exact integer golden GEMM it
    gives the golden bf16 bits, and on random bytes it is within 1e-2 of the oracle's float64 product."""
    a = torch.from_numpy(gold["gemm_a"]).view(E4)
    b = torch.from_numpy(gold["gemm_b"]).view(E4)
    c = O.torch_mm(a, torch.tensor(gold["gemm_sa"]), b, torch.tensor(gold["gemm_sb"]))
    assert np.array_equal(_u16(c), gold["gemm_c"])
    g = torch.Generator().manual_seed(8)
    a = (torch.randn(300, 512, generator=g) * 30).clamp(-448, 448).to(E4)
    b = (torch.randn(200, 512, generator=g) * 30).clamp(-448, 448).to(E4)
    c = O.torch_mm(a, torch.tensor(0.01), b, torch.tensor(0.02))
    ref = O.mm64(a.view(torch.uint8).numpy(), np.float32(0.01), b.view(torch.uint8).numpy(), np.float32(0.02))
    assert O.rel_fro(c.float().numpy(), ref) < 4e-3


def test_torch_swiglu_equals_c_oracle():
    """The baseline's SwiGLU product cast equals the C oracle's bytes (sl = bf16(z1 sigmoid(z1)) agrees with torch's
    for every finite bf16 input); its backward's dz is within one bf16 ulp of the oracle's (sigmoid definitions)."""
    g = torch.Generator().manual_seed(9)
    z = (torch.randn(256, 2048, generator=g) * 3).to(torch.bfloat16)
    da = (torch.randn(256, 1024, generator=g) * 0.1).to(torch.bfloat16)
    q, s = O.torch_swiglu_tcast(z)
    oq, od, _ = O.swiglu_tcast(_u16(z))
    assert s.item() == od and np.array_equal(q.view(torch.uint8).numpy(), oq)
    dz, dzq, sdz = O.torch_swiglu_bwd(z, da)
    odz, _, _, _ = O.swiglu_bwd(_u16(z), _u16(da))
    diff = np.abs(_u16(dz).astype(np.int32) - odz.astype(np.int32))
    assert diff.max() <= 1 and (diff == 0).mean() > 0.99
    q2, s2 = O.torch_tcast(dz)
    assert s2.item() == sdz.item() and torch.equal(q2.view(torch.uint8), dzq.view(torch.uint8))


# ---------------------------------------------------------------- the norm sites' producer (fused_norm.py:64-91)

def _norm_inputs(B, N, C, seed, res=True, k=1.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(B, N, C, generator=g) * k).to(torch.bfloat16)
    a = torch.randn(B, N, C, generator=g).to(torch.bfloat16)
    gate = (torch.randn(B, 1, C, generator=g) * 0.2).to(torch.bfloat16)
    sh = (torch.randn(B, 1, C, generator=g) * 0.1).to(torch.bfloat16)
    sc = (torch.randn(B, 1, C, generator=g) * 0.1).to(torch.bfloat16)
    w = 1 + 0.1 * torch.randn(C, generator=g)
    return x, (a if res else None), (gate if res else None), w, sh, sc


def _oracle_norm(x, a, gate, w, sh, sc, eps):
    B, N, C = x.shape
    return O.mod_rmsnorm(_u16(x).reshape(-1, C), w.numpy(), _u16(sh).reshape(B, C), _u16(sc).reshape(B, C), N, eps,
                         None if a is None else _u16(a).reshape(-1, C),
                         None if gate is None else _u16(gate).reshape(B, C))


@pytest.mark.parametrize("res", [False, True])
@pytest.mark.parametrize("C", [100, 256, 768, 896, 1024, 1152, 1792])
def test_norm_against_torch(res, C):
    """x_new equals torch's x + gate * a in fp32 rounded once to bf16 (the reference kernel's, fused_norm.py:82); rstd
    is within 2 fp32 ulp of torch.rsqrt(mean(x_new^2) + eps); h equals torch's n = bf16(w * (x_new * rstd)),
    bf16(n * (1 + scale) + shift) (fused_norm.py:85-89) bit for bit when fed the oracle's rstd, the multiply-add
    evaluated exactly (float64, exact for these operands) and rounded once to fp32, as a fused multiply-add does."""
    B, N, eps = 3, 40, 1e-6
    x, a, gate, w, sh, sc = _norm_inputs(B, N, C, C + res, res)
    xn, h, rstd = _oracle_norm(x, a, gate, w, sh, sc, eps)
    xs = (x.float() + gate.float() * a.float()).to(torch.bfloat16) if res else x
    if res:
        assert np.array_equal(xn, _u16(xs).reshape(-1, C))
    rs_t = torch.rsqrt(xs.float().pow(2).mean(-1) + eps).reshape(-1).numpy()
    assert np.abs(rstd.astype(np.float64) / rs_t - 1).max() <= 2.5e-7
    r = torch.from_numpy(rstd).view(B, N, 1)
    n = (w * (xs.float() * r)).to(torch.bfloat16).float()
    ht = (n.double() * (1 + sc.float()).double() + sh.double()).float().to(torch.bfloat16)
    assert np.array_equal(h, _u16(ht).reshape(-1, C))


def test_norm_multiply_add_is_fused():
    """h's n * (1 + scale) + shift is one fused multiply-add: with scales near 2^-16 (1 + scale then has up to 24
    significant bits, so the product rounds in fp32) and shift = -1 (cancellation), the oracle equals the exact value
    rounded once and differs from the separately rounded product and sum. (x + gate * a and the sum of squares take
    products of bf16 values, exact in fp32, so fusing does not change their bits.)"""
    B, N, C = 2, 256, 1024
    g = torch.Generator().manual_seed(3)
    x = torch.randn(B, N, C, generator=g).to(torch.bfloat16)
    w = torch.ones(C)
    sc = (torch.randn(B, 1, C, generator=g) * 2.0 ** -16).to(torch.bfloat16)
    sh = torch.full((B, 1, C), -1.0).to(torch.bfloat16)
    _, h, rstd = _oracle_norm(x, None, None, w, sh, sc, 1e-6)
    n = (w * (x.float() * torch.from_numpy(rstd).view(B, N, 1))).to(torch.bfloat16).float()
    fused = (n.double() * (1 + sc.float()).double() + sh.double()).float().to(torch.bfloat16)
    unfused = (n * (1 + sc.float()) + sh.float()).to(torch.bfloat16)
    assert np.array_equal(h, _u16(fused).reshape(-1, C))
    assert (h != _u16(unfused).reshape(-1, C)).sum() > 50


@pytest.mark.parametrize("C", [1024, 1152])
def test_norm_power_of_two_invariance(C):
    """With eps = 0, scaling x by 2^k leaves h unchanged bit for bit (the sum of squares, the square root and the
    division scale exactly): a check of the sum's structure that does not restate it (C = 1152: rows whose last
    group of 256 columns is half full)."""
    x, _, _, w, sh, sc = _norm_inputs(2, 33, C, 5, False)
    _, h0, r0 = _oracle_norm(x, None, None, w, sh, sc, 0.0)
    for k in (-3, 2, 7):
        _, h1, r1 = _oracle_norm((x.float() * 2.0 ** k).to(torch.bfloat16), None, None, w, sh, sc, 0.0)
        assert np.array_equal(h0, h1) and np.array_equal(r1 * np.float32(2.0 ** k), r0)


def test_norm_mutant_unrounded_n_fails():
    """A restatement that skips the bf16 rounding of n (fused_norm.py:86) is caught by the torch comparison above."""
    x, _, _, w, sh, sc = _norm_inputs(2, 40, 1024, 6, False)
    _, h, rstd = _oracle_norm(x, None, None, w, sh, sc, 1e-6)
    r = torch.from_numpy(rstd).view(2, 40, 1)
    n_unrounded = w * (x.float() * r)
    hm = (n_unrounded.double() * (1 + sc.float()).double() + sh.double()).float().to(torch.bfloat16)
    assert not np.array_equal(h, _u16(hm).reshape(-1, 1024))


def test_norm_q_is_tcast_of_h():
    """mod_rmsnorm_q's bytes and scale are the tcast of its h (the cast rule pinned above)."""
    x, a, gate, w, sh, sc = _norm_inputs(2, 64, 1024, 7, True)
    B, N, C = x.shape
    xn, h, rstd, hq, d = O.mod_rmsnorm_q(_u16(x).reshape(-1, C), w.numpy(), _u16(sh).reshape(B, C),
                                         _u16(sc).reshape(B, C), N, 1e-6, _u16(a).reshape(-1, C),
                                         _u16(gate).reshape(B, C))
    q2, d2, _ = O.tcast(h)
    assert d == d2 and np.array_equal(hq, q2)
