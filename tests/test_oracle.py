"""Pins for the CPU oracle (``oracle/``): every oracle function is checked here against
something other than its own formula -- torch's casts, brute-force loops, exact integer
arithmetic, algebraically different formulations, and planted mistakes that must fail."""
import numpy as np
import pytest
import torch

from oracle import gemm as og
from oracle import layout as ol
from oracle import numerics as on
from oracle import quant as oq


# ---------------------------------------------------------------- numerics
def test_e4m3fn_known_values():
    d = on.e4m3fn_decode(np.array([0x7E, 0x08, 0x01, 0x38, 0x00, 0x80, 0xFE, 0x07], dtype=np.uint8))
    assert d[0] == 448.0 and d[1] == 2.0 ** -6 and d[2] == 2.0 ** -9 and d[3] == 1.0
    assert d[4] == 0.0 and d[5] == 0.0 and np.signbit(d[5]) and d[6] == -448.0
    assert d[7] == 7 * 2.0 ** -9
    assert np.isnan(on.e4m3fn_decode(np.array([0x7F, 0xFF], dtype=np.uint8))).all()


def test_e4m3fn_decode_matches_torch_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    t = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).float().numpy()
    d = on.e4m3fn_decode(codes)
    assert np.array_equal(np.isnan(t), np.isnan(d))
    ok = ~np.isnan(t)
    assert np.array_equal(t[ok].view(np.uint32), d[ok].view(np.uint32))


def test_e4m3fn_encode_roundtrip_and_ties():
    codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], dtype=np.uint8)
    assert np.array_equal(on.e4m3fn_encode(on.e4m3fn_decode(codes)), codes)
    # exact midpoints between neighbouring positive codes round to the even code
    pos = on.e4m3fn_decode(np.arange(0, 0x7E, dtype=np.uint8)).astype(np.float64)
    nxt = on.e4m3fn_decode(np.arange(1, 0x7F, dtype=np.uint8)).astype(np.float64)
    mid = ((pos + nxt) / 2).astype(np.float32)
    enc = on.e4m3fn_encode(mid)
    lo = np.arange(0, 0x7E)
    want = np.where(lo % 2 == 0, lo, lo + 1)
    assert np.array_equal(enc, want.astype(np.uint8))


def test_e4m3fn_encode_matches_torch_cast():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        (rng.standard_normal(1_000_000) * 50).astype(np.float32),
        (rng.standard_normal(100_000) * 1e-3).astype(np.float32),
        np.array([0.0, -0.0, 448.0, -448.0, 460.0, 464.0, 470.0, 479.9, 480.0, 1e9, np.inf, -np.inf, np.nan],
                 dtype=np.float32),
    ])
    pos = on.e4m3fn_decode(np.arange(0, 0x7E, dtype=np.uint8)).astype(np.float64)
    nxt = on.e4m3fn_decode(np.arange(1, 0x7F, dtype=np.uint8)).astype(np.float64)
    x = np.concatenate([x, ((pos + nxt) / 2).astype(np.float32), -((pos + nxt) / 2).astype(np.float32)])
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = on.e4m3fn_encode(x)
    # NaN payload/sign may differ; compare NaN-ness, then exact codes elsewhere
    ref_nan = np.isnan(on.e4m3fn_decode(ref))
    got_nan = np.isnan(on.e4m3fn_decode(got))
    assert np.array_equal(ref_nan, got_nan)
    assert np.array_equal(ref[~ref_nan], got[~got_nan])


def test_bf16_rne_matches_torch():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(200_000).astype(np.float32) * 1e3,
                        rng.integers(0, 2 ** 32, 200_000, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    x = x[np.isfinite(x)]
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(on.bf16_rne(x), ref)
    exact = on.bf16_to_f32(ref)
    assert np.array_equal(on.bf16_rne(exact), ref)


def test_bf16_trunc_is_round_toward_zero():
    """Truncation to bf16 (the reference's weight conversion) is rounding toward zero on the
    bf16 grid: the result is the bf16 value of largest magnitude not above |x| with x's sign --
    checked against math.frexp-based rounding of every value -- it keeps bf16 values unchanged,
    and its relative error stays below 2^-7."""
    import math
    rng = np.random.default_rng(11)
    x = np.concatenate([rng.standard_normal(20_000).astype(np.float32) * 37.0,
                        np.array([1.0, -1.0, 3.0, 0.0, -0.0, 1.0 + 2 ** -7, 1.0 + 2 ** -8, -(1.0 + 2 ** -8)],
                                 dtype=np.float32)])
    got = on.bf16_to_f32(on.bf16_trunc(x))
    for v, t in zip(x[:2000].tolist() + x[-8:].tolist(), got[:2000].tolist() + got[-8:].tolist()):
        if v == 0:
            assert t == 0
            continue
        m, e = math.frexp(abs(v))                     # |v| = m * 2^e, m in [0.5, 1)
        want = math.floor(m * 256) / 256 * 2.0 ** e   # 8 significant bits, toward zero
        assert t == math.copysign(want, v), (v, t)
    assert np.array_equal(on.bf16_trunc(got), on.bf16_trunc(x))
    nz = x != 0
    assert np.all(np.abs(got[nz]) <= np.abs(x[nz])) and np.all(np.abs(got[nz] - x[nz]) < 2.0 ** -7 * np.abs(x[nz]))


# ---------------------------------------------------------------- quantizers
@pytest.mark.parametrize("kind", ["fp8", "int8", "int4"])
def test_quant_rows_invariants(kind):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((64, 512)).astype(np.float32)
    x[3] = 0.0
    q, s = oq.quant_rows(x, kind)
    qmax = oq.QMAX[kind]
    v = on.e4m3fn_decode(q) if kind == "fp8" else q.astype(np.float32)
    assert np.all(np.abs(v) <= qmax)
    assert s[3] == 1.0 and np.all(v[3] == 0)
    # the row's amax maps to +-qmax exactly
    i = np.abs(x).argmax(axis=1)
    peak = np.abs(v[np.arange(64), i])
    assert np.all(peak[np.arange(64) != 3] == qmax)
    err = np.abs(v * s[:, None] - x)
    if kind == "fp8":
        # half an fp8 ulp at the value's binade (3 mantissa bits), plus subnormal quantum
        y = np.abs(x / s[:, None])
        ulp = 2.0 ** (np.maximum(np.floor(np.log2(np.maximum(y, 1e-30))), -6) - 3)
        assert np.all(np.abs(v - x / s[:, None]) <= ulp / 2 + 1e-6)
    else:
        assert np.all(err <= s[:, None] / 2 * (1 + 1e-5))


@pytest.mark.parametrize("kind", ["fp8", "int8"])
def test_quant_rows_matches_product_quantizer(kind):
    from flydsl_amd import quant as pq
    g = torch.Generator().manual_seed(7)
    x = torch.randn(96, 384, generator=g)
    qd = pq.FP8 if kind == "fp8" else torch.int8
    q_t, s_t = pq.pertoken_quant(x, quant_dtype=qd)
    q_o, s_o = oq.quant_rows(x.numpy(), kind)
    assert np.array_equal(s_t.view(-1).numpy(), s_o)
    assert np.array_equal(q_t.view(torch.int8).numpy().view(np.uint8), q_o.view(np.uint8))


def test_quant_int4_matches_product_quantizer():
    from flydsl_amd import quant as pq
    g = torch.Generator().manual_seed(8)
    x = torch.randn(64, 256, generator=g) * 0.02
    q_t, s_t = pq.pertoken_quant(x, quant_dtype=torch.int8, dtypeMax=7)
    q_o, s_o = oq.quant_rows(x.numpy(), "int4")
    assert np.array_equal(s_t.view(-1).numpy(), s_o)
    assert np.array_equal(q_t.numpy(), q_o)


def test_reference_int8_cast_truncates():
    """The reference's own int8 cast (``.to(torch.int8)``) truncates; the product offers it as
    rounding='trunc' and defaults to round-half-even."""
    from flydsl_amd import quant as pq
    x = torch.tensor([[127.0, 1.7, 2.5, -1.7, -2.5, 0.4]])
    q_tr, _ = pq.pertoken_quant(x, quant_dtype=torch.int8, rounding="trunc")
    q_rn, _ = pq.pertoken_quant(x, quant_dtype=torch.int8)
    assert q_tr.tolist() == [[127, 1, 2, -1, -2, 0]]
    assert q_rn.tolist() == [[127, 2, 2, -2, -2, 0]]


def _f32_round(v):
    """Exact round-to-nearest-even of a rational to float32 (normal range), returned as a
    Fraction: an implementation independent of numpy's float32 arithmetic."""
    from fractions import Fraction
    if v == 0:
        return Fraction(0)
    neg = v < 0
    a = -v if neg else v
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    m = a / Fraction(2) ** (e - 23)          # in [2^23, 2^24)
    fl = m.numerator // m.denominator
    rem = m - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    r = Fraction(fl) * Fraction(2) ** (e - 23)
    return -r if neg else r


def _trunc(fr):
    q = abs(fr.numerator) // fr.denominator
    return -q if fr < 0 else q


def test_quant_rows_recip_exact_rational():
    """The reference device kernel's q = fptosi(x * f32(1 / f32(amax / 127))) recomputed with
    exact rationals and explicit float32 rounding, on the reference test's own data
    distribution (np.random.seed(42), uniform(-5, 5) in fp16; test_quant.py:306-307)."""
    from fractions import Fraction
    np.random.seed(42)
    x = np.random.uniform(-5.0, 5.0, size=(3, 700)).astype(np.float16)
    q, s = oq.quant_rows_recip(x)
    for r in range(x.shape[0]):
        amax = max(abs(Fraction(float(v))) for v in x[r])
        scale = _f32_round(amax / 127)
        assert Fraction(float(s[r])) == scale
        inv = _f32_round(1 / scale)
        want = [_trunc(_f32_round(Fraction(float(v)) * inv)) for v in x[r]]
        assert q[r].tolist() == want


def test_quant_rows_recip_vs_division_known_answers():
    """Values where truncating x * (1/s) and x / s give different integers: the device-kernel
    oracle must follow the reciprocal, the pertoken_quant oracle the quotient."""
    from fractions import Fraction
    rng = np.random.default_rng(11)
    found = 0
    for _ in range(400):
        row = rng.uniform(-5, 5, 64).astype(np.float32)
        row[0] = np.float32(rng.uniform(3, 5))  # amax position
        amax = max(abs(Fraction(float(v))) for v in row)
        scale = _f32_round(amax / 127)
        inv = _f32_round(1 / scale)
        for k, v in enumerate(row):
            fv = Fraction(float(v))
            a, b = _trunc(_f32_round(fv * inv)), _trunc(_f32_round(fv / scale))
            if a != b:
                found += 1
                q_r, _ = oq.quant_rows_recip(row[None, :])
                q_d, _ = oq.quant_rows(row[None, :], "int8", rounding="truncate")
                assert q_r[0, k] == a and q_d[0, k] == b
        if found >= 3:
            break
    assert found >= 3


def test_quant_rows_recip_reference_criterion_and_invariants():
    """The reference test's own acceptance (|q - (x/scale).astype(int8)| <= 1, scales equal to
    amax/127; test_quant.py:309-316, 339-349) plus truncation invariants."""
    np.random.seed(42)
    x = np.random.uniform(-5.0, 5.0, size=(64, 8192)).astype(np.float16)
    xf = x.astype(np.float32)
    q, s = oq.quant_rows_recip(x)
    amax = np.max(np.abs(xf), axis=1)
    ref_scale = amax / 127.0
    ref_scale[ref_scale == 0] = 1.0
    assert np.max(np.abs(s - ref_scale)) == 0.0
    ref_q = (xf / ref_scale[:, None]).astype(np.int8)
    assert np.max(np.abs(q.astype(np.int32) - ref_q.astype(np.int32))) <= 1
    y = xf / s[:, None]
    assert np.all(np.abs(q) <= 127)
    assert np.all(np.abs(q.astype(np.float64)) <= np.abs(y) * (1 + 1e-6))   # toward zero
    assert np.all(np.abs(y) - np.abs(q) < 1 + 1e-4)
    assert np.all((q == 0) | (np.sign(q) == np.sign(xf)))
    z, sz = oq.quant_rows_recip(np.zeros((2, 16), np.float16))
    assert np.all(sz == 1.0) and np.all(z == 0)


def test_quant_rows_truncate_matches_torch_cast():
    """pertoken_quant's int8 cast is torch's .to(int8) of the float32 quotient (tests/utils.py:71)."""
    g = torch.Generator().manual_seed(12)
    x = torch.randn(50, 300, generator=g) * 3
    x[4] = 0
    x[5, 7] = float("inf")
    x[6, 9] = float("nan")
    q, s = oq.quant_rows(x.numpy(), "int8", rounding="truncate")
    xs = torch.nan_to_num(x, nan=0.0, posinf=127.0, neginf=-127.0)
    st = torch.maximum(xs.amax(-1, keepdim=True), -xs.amin(-1, keepdim=True)) / 127.0
    st[st == 0] = 1
    qt = (xs / st).to(torch.int8)
    assert np.array_equal(s, st.view(-1).numpy())
    assert np.array_equal(q, qt.numpy())


def test_quant_blocks_reduces_to_rows_and_matches_product():
    from flydsl_amd import quant as pq
    rng = np.random.default_rng(3)
    x = rng.standard_normal((32, 256)).astype(np.float32)
    qb, sb = oq.quant_blocks(x, 1, 256)
    qr, sr = oq.quant_rows(x, "fp8")
    assert np.array_equal(qb, qr) and np.array_equal(sb.reshape(-1), sr)
    for br, bc in [(1, 128), (128, 128)]:
        xx = rng.standard_normal((256, 384)).astype(np.float32)
        q_o, s_o = oq.quant_blocks(xx, br, bc)
        q_t, s_t = pq.blockscale_quant(torch.from_numpy(xx), br, bc)
        assert np.array_equal(s_t.numpy(), s_o)
        assert np.array_equal(q_t.view(torch.uint8).numpy(), q_o)


# ---------------------------------------------------------------- layouts
def test_shuffle_bruteforce_and_inverse():
    N, K = 48, 96
    b = (np.arange(N * K) % 251).astype(np.uint8).reshape(N, K)
    flat = ol.shuffle_weight(b)
    for n in range(N):
        for k in range(K):
            assert flat[ol.shuffle_index(n, k, K)] == b[n, k]
    assert np.array_equal(ol.unshuffle_weight(flat, N, K), b)


def test_shuffle_matches_product():
    from flydsl_amd import quant as pq
    rng = np.random.default_rng(4)
    b = rng.integers(-128, 128, (64, 256), dtype=np.int8)
    got = pq.shuffle_weight(torch.from_numpy(b)).numpy().reshape(-1)
    assert np.array_equal(got, ol.shuffle_weight(b))


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_shuffle_2byte_bruteforce(dt):
    """2-byte elements: the reference groups 8 elements per 16-byte chunk
    (tests/utils.py:83-90: view(-1, N/16, 16, K/32, 4, 8).permute(0, 1, 3, 4, 2, 5)); element
    (n, k) lands at [n//16][k//32][(k//8)%4][n%16][k%8] -- checked element by element."""
    N, K = 32, 96
    x = (torch.randn(N, K) * 5).to(dt)
    bits = x.view(torch.int16).numpy().view(np.uint16)
    got = ol.shuffle_weight(bits).view(np.uint16)
    want = np.empty(N * K, dtype=np.uint16)
    for n in range(N):
        for k in range(K):
            idx = (((n // 16) * (K // 32) + k // 32) * 4 + (k // 8) % 4) * 128 + (n % 16) * 8 + k % 8
            want[idx] = bits[n, k]
    assert np.array_equal(got, want)
    from flydsl_amd import quant as pq
    assert np.array_equal(pq.shuffle_weight(x).contiguous().view(torch.int16).numpy().view(np.uint16).reshape(-1), got)


@pytest.mark.parametrize("kind,dt", [("bf16", torch.bfloat16), ("fp16", torch.float16)])
def test_run_torch_16bit_matches_torch_and_loop(kind, dt):
    g = torch.Generator().manual_seed(4)
    a = (torch.randn(9, 64, generator=g) * 3).to(dt)
    b = (torch.randn(20, 64, generator=g) * 3).to(dt)
    ab = a.view(torch.int16).numpy().view(np.uint16)
    bb = b.view(torch.int16).numpy().view(np.uint16)
    ref32 = og.run_torch(ab, bb, None, None, kind)
    # float32 BLAS (numpy vs torch) differs only by accumulation rounding: bound by K ulps of sum|a||b|
    mag = (a.float().abs() @ b.float().abs().T).numpy()
    assert np.all(np.abs(ref32 - (a.float() @ b.float().T).numpy()) <= 64 * 2.0 ** -23 * mag)
    ref64 = og.run_torch(ab, bb, None, None, kind, "f64")
    af, bf = a.double().numpy(), b.double().numpy()
    loop = np.array([[sum(af[m, k] * bf[n, k] for k in range(64)) for n in range(20)] for m in range(9)])
    assert np.allclose(ref64, loop, rtol=1e-12, atol=1e-12)
    # the decode itself: every 16-bit pattern that is finite
    allbits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    t = torch.from_numpy(allbits.view(np.int16).copy()).view(dt).float().numpy()
    d = on.bf16_to_f32(allbits) if kind == "bf16" else on.f16_to_f32(allbits)
    fin = np.isfinite(t)
    assert np.array_equal(np.isfinite(d), fin) and np.array_equal(t[fin].view(np.uint32), d[fin].view(np.uint32))


def test_int4_pack_unpack_exhaustive():
    from flydsl_amd import quant as pq
    vals = np.arange(-8, 8, dtype=np.int8)
    # every value in every one of the 8 positions of a packing group
    groups = []
    for pos in range(8):
        for v in vals:
            g = np.zeros(8, dtype=np.int8)
            g[pos] = v
            g[(pos + 3) % 8] = -v - 1 if v != -8 else 7
            groups.append(g)
    x = np.concatenate(groups)
    packed = ol.pack_int4(x)
    assert packed.size == x.size // 2
    assert np.array_equal(ol.unpack_int4(packed), x)
    assert np.array_equal(pq.pack_int4(torch.from_numpy(x)).numpy(), packed)
    # the nibble placement the kernel relies on: byte j = u[j] | u[j+4] << 4
    g = np.array([1, 2, 3, 4, -1, -2, -3, -4], dtype=np.int8)
    assert ol.pack_int4(g).view(np.uint8).tolist() == [0xF1, 0xE2, 0xD3, 0xC4]


# ---------------------------------------------------------------- GEMM oracles
def _brute(a, b):
    M, K = a.shape
    N = b.shape[0]
    out = np.zeros((M, N), dtype=np.float64)
    for m in range(M):
        for n in range(N):
            s = 0.0
            for k in range(K):
                s += float(a[m, k]) * float(b[n, k])
            out[m, n] = s
    return out


def test_acc_int_exact():
    rng = np.random.default_rng(5)
    a = rng.integers(-127, 128, (5, 64), dtype=np.int8)
    b = rng.integers(-127, 128, (7, 64), dtype=np.int8)
    assert np.array_equal(og.acc_int(a, b), _brute(a, b).astype(np.int32))
    a = rng.integers(-127, 128, (64, 1024), dtype=np.int8)
    b = rng.integers(-127, 128, (48, 1024), dtype=np.int8)
    ref = torch._int_mm(torch.from_numpy(a), torch.from_numpy(b).t().contiguous()).numpy()
    assert np.array_equal(og.acc_int(a, b), ref)
    # extreme magnitudes: all -127 x -127 over a long K stays exact
    a = np.full((2, 8192), -127, dtype=np.int8)
    assert og.acc_int(a, a)[0, 0] == 127 * 127 * 8192


def test_run_torch_matches_bruteforce_and_f32():
    rng = np.random.default_rng(6)
    x = rng.standard_normal((6, 128)).astype(np.float32)
    w = rng.standard_normal((5, 128)).astype(np.float32)
    qa, sa = oq.quant_rows(x, "fp8")
    qb, sb = oq.quant_rows(w, "fp8")
    da = on.e4m3fn_decode(qa).astype(np.float64) * sa[:, None]
    db = on.e4m3fn_decode(qb).astype(np.float64) * sb[:, None]
    ref = og.run_torch(qa, qb, sa, sb, "fp8", "f64")
    assert np.allclose(ref, _brute(da, db), rtol=1e-6, atol=1e-6)
    f32 = og.run_torch(qa, qb, sa, sb, "fp8", "f32")
    tt = torch.mm(torch.from_numpy(on.e4m3fn_decode(qa)) * torch.from_numpy(sa)[:, None],
                  (torch.from_numpy(on.e4m3fn_decode(qb)) * torch.from_numpy(sb)[:, None]).T).numpy()
    assert np.allclose(f32, tt, rtol=1e-5, atol=1e-5)


def test_epilogue_int_matches_torch():
    rng = np.random.default_rng(7)
    acc = rng.integers(-2 ** 26, 2 ** 26, (16, 32)).astype(np.int32)
    sa = rng.random(16).astype(np.float32) * 0.01
    sb = rng.random(32).astype(np.float32) * 0.01
    ref = ((torch.from_numpy(acc).float() * torch.from_numpy(sa)[:, None]) * torch.from_numpy(sb)[None, :])
    ref = ref.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(og.epilogue_int_bf16(acc, sa, sb), ref)


def test_blockscale_two_formulations_agree():
    rng = np.random.default_rng(8)
    M, N, K = 8, 272, 384  # N not a multiple of 128 -> last scale block partial
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = rng.standard_normal((N, K)).astype(np.float32)
    qx, sx = oq.quant_blocks(x, 1, 128)
    wp = np.concatenate([w, np.zeros(((-N) % 128, K), np.float32)])
    qw, sw = oq.quant_blocks(wp, 128, 128)
    qw = qw[:N]
    a = og.run_torch_blockscale(qx, qw, sx, sw, "f64")
    b = og.blockscale_per_block(qx, qw, sx, sw)
    # the reference rounds each dequantized element to fp32 before the product; the
    # per-block form scales exact partial sums: they agree to fp32 rounding
    assert np.allclose(a, b, rtol=1e-5, atol=1e-4)
    # uniform per-row / per-column scales reduce blockscale to the per-token GEMM
    sx_u = np.repeat(sx[:, :1], K // 128, axis=1)
    sw_u = np.repeat(sw[:, :1], K // 128, axis=1)
    c = og.run_torch_blockscale(qx, qw, sx_u, sw_u, "f64")
    sbn = sw_u[np.arange(N) // 128, 0]
    d = og.run_torch(qx, qw, sx_u[:, 0], sbn, "fp8", "f64")
    assert np.allclose(c, d, rtol=1e-9, atol=1e-9)


def test_bar_rejects_planted_mistakes():
    """Plausible kernel mistakes, planted in the oracle, must fail the acceptance bar."""
    rng = np.random.default_rng(9)
    M, N, K = 32, 64, 512
    qa, sa = oq.quant_rows(rng.standard_normal((M, K)).astype(np.float32), "fp8")
    qb, sb = oq.quant_rows(rng.standard_normal((N, K)).astype(np.float32), "fp8")
    ref = og.run_torch(qa, qb, sa, sb, "fp8", "f64")
    assert og.within_bar(og.run_torch(qa, qb, sa, sb, "fp8", "f32"), ref)[0]
    bad = {
        "dropped_scale_b": og.run_torch(qa, qb, sa, np.ones_like(sb), "fp8", "f64"),
        "swapped_scales": og.run_torch(qa, qb, sb[:M], sa.repeat(2)[:N], "fp8", "f64"),
        "sign": -ref,
        "last_k_tile_dropped": og.run_torch(qa[:, :K - 128], qb[:, :K - 128], sa, sb, "fp8", "f64"),
        "k_chunks_misaligned": og.run_torch(qa, np.roll(qb, 16, axis=1), sa, sb, "fp8", "f64"),
        "columns_shifted": np.roll(ref, 1, axis=1),
    }
    for name, out in bad.items():
        assert not og.within_bar(out, ref)[0], name
    # blockscale: A scale indexed [m][kb] instead of the transposed layout
    x = rng.standard_normal((128, 256)).astype(np.float32)
    w = rng.standard_normal((128, 256)).astype(np.float32)
    qx, sx = oq.quant_blocks(x, 1, 128)
    qw, sw = oq.quant_blocks(w, 128, 128)
    good = og.run_torch_blockscale(qx, qw, sx, sw, "f64")
    wrong = og.run_torch_blockscale(qx, qw, sx.T.reshape(sx.shape), sw, "f64")
    assert not og.within_bar(wrong, good)[0]


# ---------------------------------------------------------------- MXFP4
from oracle import mxfp4 as om  # noqa: E402

_OCP_E2M1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]   # OCP MX spec v1.0, FP4 E2M1 magnitudes


def test_e2m1_decode_matches_spec_table():
    codes = np.arange(16, dtype=np.uint8)
    want = np.array(_OCP_E2M1 + [-v for v in _OCP_E2M1], dtype=np.float32)
    got = om.e2m1_decode(codes)
    assert np.array_equal(got, want) and np.signbit(got[8])
    from flydsl_amd import fp4
    packed = torch.tensor([0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE], dtype=torch.uint8)
    assert np.array_equal(fp4.mxfp4_to_f32(packed).numpy(), want)
    assert np.array_equal(om.unpack(packed.numpy()).reshape(-1), np.arange(16))


def _nearest_e2m1_bruteforce(y):
    """Exhaustive nearest grid value, ties to the even code, saturating at 6."""
    out = []
    for v in y.astype(np.float64):
        a = min(abs(v), 6.0)
        d = [abs(a - g) for g in _OCP_E2M1]
        best = min(d)
        cands = [i for i, x in enumerate(d) if x == best]
        code = [c for c in cands if c % 2 == 0][0] if len(cands) > 1 else cands[0]
        out.append(code | (8 if np.signbit(v) else 0))
    return np.array(out, dtype=np.uint8)


def test_e2m1_encode_nearest_even_and_saturating():
    rng = np.random.default_rng(21)
    grid = np.array(_OCP_E2M1)
    mids = (grid[1:] + grid[:-1]) / 2
    y = np.concatenate([rng.uniform(-8, 8, 3000), mids, -mids, grid, -grid, [6.5, 7.0, 100.0, -9.0, 0.1, -0.2]]).astype(np.float32)
    assert np.array_equal(om.e2m1_encode(y), _nearest_e2m1_bruteforce(y))
    assert np.array_equal(om.e2m1_encode(om.e2m1_decode(np.arange(16))), np.arange(16, dtype=np.uint8))
    from flydsl_amd import fp4
    assert np.array_equal(fp4.e2m1_encode(torch.from_numpy(y)).numpy(), om.e2m1_encode(y))


def test_e8m0_encode_closed_form_and_edges():
    import math
    rng = np.random.default_rng(22)
    x = np.concatenate([np.exp2(rng.uniform(-120, 120, 4000)), [1.0, 1.5, 1.4999999, 2.9999, 3.0, 0.75]]).astype(np.float32)
    want = []
    for v in x.astype(np.float64):
        m, e = math.frexp(v)          # v = m * 2**e, m in [0.5, 1)
        sig, ex = 2 * m, e - 1        # v = sig * 2**ex, sig in [1, 2)
        want.append(ex + 127 + (1 if sig >= 1.5 else 0))
    assert np.array_equal(om.e8m0_encode(x).astype(np.int64), np.array(want))
    edge = np.array([0x00000000, 0x00400000, 0x00400001, 0x00200000, 0x7F800000, 0x7FC00000, 0x7F400000],
                    dtype=np.uint32).view(np.float32)
    # 0 -> 0; subnormal with only bit 22 -> 0; bit 22 + lower bit -> 1; bit 21 only -> 0;
    # inf/NaN -> 0xFF; largest finite binade with significand >= 1.5 -> 0xFF
    assert om.e8m0_encode(edge).tolist() == [0, 0, 1, 0, 0xFF, 0xFF, 0xFF]
    from flydsl_amd import fp4
    assert np.array_equal(fp4.e8m0_from_f32(torch.from_numpy(np.concatenate([x, edge]))).numpy(),
                          om.e8m0_encode(np.concatenate([x, edge])))
    d = om.e8m0_decode(np.array([0, 1, 127, 128, 254, 255], dtype=np.uint8))
    assert d[0] == 2.0 ** -127 and d[1] == 2.0 ** -126 and d[2] == 1.0 and d[3] == 2.0 and d[4] == 2.0 ** 127
    assert np.isnan(d[5])
    assert np.array_equal(fp4.e8m0_to_f32(torch.tensor([0, 1, 127, 128, 254], dtype=torch.uint8)).numpy(), d[:5])


def test_quant_1x32_error_bound_and_product_equality():
    from flydsl_amd import fp4
    g = torch.Generator().manual_seed(23)
    x = torch.randn(40, 512, generator=g) * 3
    x[2] = 0.0
    x[3, :32] = 1e-3
    q, s = om.quant_1x32(x.numpy())
    deq = om.dequant(q, s)
    sc = np.repeat(om.e8m0_decode(s).astype(np.float64), 32, axis=1)
    y = np.abs(x.numpy() / sc)
    step = np.where(y < 2, 0.5, np.where(y < 4, 1.0, 2.0))
    sat = y > 6
    err = np.abs(deq - x.numpy())
    assert np.all(err[~sat] <= step[~sat] / 2 * sc[~sat] * (1 + 1e-6))
    assert np.all(deq[2] == 0)
    # the block amax lands in [4/1.5, 6] after scaling (the scale rounds amax/4 to a power of two)
    blk = y.reshape(-1, 32).max(axis=1)
    nz = blk > 0
    assert np.all(blk[nz] >= 4 / 1.5 * (1 - 1e-6)) and np.all(blk[nz] <= 6 * 1.5)
    qt, st, _ = fp4.per_1x32_f4_quant(x)
    assert np.array_equal(qt.numpy(), q) and np.array_equal(st.numpy(), s)


def test_mxfp4_shuffles_elementwise():
    from flydsl_amd import fp4
    rng = np.random.default_rng(24)
    N, K = 64, 512
    b = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    got = om.shuffle_weight_w4(b)
    kb = K // 2
    want = np.empty(N * kb, dtype=np.uint8)
    for n in range(N):
        for k in range(kb):   # reference view (N0, NLane, K0, KLane, KPack) -> (N0, K0, KLane, NLane, KPack)
            n0, nl, k0, kl, kp = n // 16, n % 16, k // 64, (k // 16) % 4, k % 16
            want[(((n0 * (kb // 64) + k0) * 4 + kl) * 16 + nl) * 16 + kp] = b[n, k]
    assert np.array_equal(got, want)
    assert np.array_equal(fp4.shuffle_weight_w4(torch.from_numpy(b)).numpy().reshape(-1), got)
    R, ks = 64, K // 32 * 2     # K = 1024 -> 32 scale blocks per row
    s = rng.integers(0, 256, (R, ks), dtype=np.uint8)
    gs = om.shuffle_scale_w4(s)
    ws = np.empty(R * ks, dtype=np.uint8)
    for r in range(R):
        for k in range(ks):   # (r1, rp, rl) x (k1, kp, kl) -> [r1][k1][kl][rl][kp][rp]
            r1, rp, rl = r // 32, (r // 16) % 2, r % 16
            k1, kp, kl = k // 8, (k // 4) % 2, k % 4
            ws[((((r1 * (ks // 8) + k1) * 4 + kl) * 16 + rl) * 2 + kp) * 2 + rp] = s[r, k]
    assert np.array_equal(gs, ws)
    assert np.array_equal(fp4.shuffle_scale_w4(torch.from_numpy(s)).numpy().reshape(-1), gs)


def test_run_torch_w4_bruteforce():
    rng = np.random.default_rng(25)
    a = rng.integers(0, 256, (3, 32), dtype=np.uint8)     # K = 64
    b = rng.integers(0, 256, (5, 32), dtype=np.uint8)
    sa = rng.integers(120, 135, (32, 2), dtype=np.uint8)  # padded rows like the reference
    sb = rng.integers(120, 135, (5, 2), dtype=np.uint8)
    ref = om.run_torch_w4(a, b, sa, sb, "f64")
    dec = lambda p: [v for byte in p for v in (_OCP_E2M1 + [-x for x in _OCP_E2M1])[byte & 15:(byte & 15) + 1] +
                     (_OCP_E2M1 + [-x for x in _OCP_E2M1])[byte >> 4:(byte >> 4) + 1]]
    for m in range(3):
        for n in range(5):
            av, bv = dec(a[m]), dec(b[n])
            tot = sum(av[k] * 2.0 ** (int(sa[m, k // 32]) - 127) * bv[k] * 2.0 ** (int(sb[n, k // 32]) - 127)
                      for k in range(64))
            assert abs(ref[m, n] - tot) <= 1e-9 * max(1.0, abs(tot))


# ---- MoE 2-stage ------------------------------------------------------------------------
from oracle import moe as omoe  # noqa: E402
from flydsl_amd.moe import moe_sorting as product_moe_sorting  # noqa: E402


def test_moe_sorting_hand_worked_example():
    """topk_ids [[0,2],[2,1],[0,1]], 3 experts, blocks of 2, worked out by hand from the
    reference's loop (test_moe_gemm.py:131-155): expert 0 takes (t0,s0),(t2,s0); expert 1
    (t1,s1),(t2,s1); expert 2 (t0,s1),(t1,s0); buffers sized 3*2 + 3*2 - 2 = 10 entries, 5 blocks."""
    ids = np.array([[0, 2], [2, 1], [0, 1]])
    w = np.array([[.6, .4], [.7, .3], [.5, .5]], np.float32)
    pad = (2 << 24) | 3
    want_ids = [0, 2, (1 << 24) | 1, (1 << 24) | 2, (1 << 24) | 0, 1, pad, pad, pad, pad]
    want_w = [.6, .5, .3, .5, .4, .7, 0, 0, 0, 0]
    for sid, sw, eid, post in (omoe.moe_sorting(ids, w, 3, 2),
                               [t.numpy() for t in product_moe_sorting(torch.tensor(ids), torch.tensor(w), 3, 2)]):
        assert list(sid) == want_ids
        assert np.allclose(sw, want_w)
        assert list(eid) == [0, 1, 2, -1, -1]
        assert list(post) == [6, 3]
    # an expert mask drops expert 1's routes and renumbers expert 2 as 1
    sid, sw, eid, post = omoe.moe_sorting(ids, w, 3, 2, expert_mask=np.array([1, 0, 1]))
    assert list(sid[:4]) == [0, 2, (1 << 24) | 0, 1] and list(eid[:3]) == [0, 1, -1] and list(post) == [4, 3]


@pytest.mark.parametrize("seed", range(12))
def test_moe_sorting_invariants_and_product(seed):
    g = np.random.default_rng(seed)
    T, E = int(g.integers(1, 80)), int(g.integers(1, 12))
    k, bs = int(g.integers(1, min(E, 4) + 1)), int(g.choice([1, 4, 16, 32, 64]))
    ids = np.stack([g.permutation(E)[:k] for _ in range(T)])
    w = g.random((T, k)).astype(np.float32)
    mask = (g.random(E) > 0.3).astype(np.int32) if seed % 3 == 0 else None
    sid, sw, eid, post = omoe.moe_sorting(ids, w, E, bs, mask)
    kept = np.ones(E, bool) if mask is None else mask.astype(bool)
    local = np.cumsum(kept) - 1
    routes = {(t, s) for t in range(T) for s in range(k) if kept[ids[t, s]]}
    seen = set()
    n_valid = int(post[0])
    assert n_valid % bs == 0 and post[1] == T
    assert n_valid == sum(-(-int((ids == e).sum()) // bs) * bs for e in range(E) if kept[e])
    for b in range(len(eid)):
        rows = sid[b * bs:(b + 1) * bs] if (b + 1) * bs <= len(sid) else sid[b * bs:]
        if b * bs >= n_valid:
            assert eid[b] == -1
            continue
        for i, v in enumerate(rows):
            t, s = int(v) & 0xFFFFFF, int(v) >> 24
            if t == T:
                assert s == k          # padding entry
                continue
            assert local[ids[t, s]] == eid[b] and (t, s) not in seen
            assert sw[b * bs + i] == w[t, s]
            seen.add((t, s))
    assert seen == routes
    assert all(int(v) == ((k << 24) | T) for v in sid[n_valid:])
    prod = product_moe_sorting(torch.tensor(ids), torch.tensor(w), E, bs, None if mask is None else torch.tensor(mask))
    for a, b in zip((sid, sw, eid, post), prod):
        assert np.array_equal(a, b.numpy())


def test_silu_closed_forms():
    x = np.array([0.0, 1.0, -1.0, 2.5, -30.0, 30.0, 1e-3])
    y = omoe.silu(x)
    assert y[0] == 0.0
    assert abs(y[1] - 1.0 / (1.0 + np.exp(-1.0))) < 1e-15              # sigmoid(1) = 0.7310585786...
    assert abs(y[1] - 0.7310585786300049) < 1e-15
    assert np.allclose(omoe.silu(x) - omoe.silu(-x), x, rtol=0, atol=1e-12)   # x*s(x) + x*s(-x)... = x
    assert abs(y[4]) < 1e-11 and abs(y[5] - 30.0) < 1e-11


def _moe_case(seed, T=6, D=64, I=32, E=4, k=2, kind="fp8"):
    g = np.random.default_rng(seed)
    ids = np.stack([g.permutation(E)[:k] for _ in range(T)])
    w = g.random((T, k)).astype(np.float32)
    w /= w.sum(1, keepdims=True)
    x = g.standard_normal((T, D)).astype(np.float32)
    w1 = (g.standard_normal((E * 2 * I, D)) * 0.2).astype(np.float32)
    xq, sx = oq.quant_rows(x, kind)
    w1q, sw1 = oq.quant_rows(w1, kind)
    return ids, w, xq, sx.reshape(-1), w1q, sw1.reshape(-1)


@pytest.mark.parametrize("kind", ["fp8", "int8"])
@pytest.mark.parametrize("doweight", [False, True])
def test_moe_gemm1_route_and_sorted_forms_agree(kind, doweight):
    T, D, I, E, k, bs = 7, 64, 32, 5, 3, 4
    ids, w, xq, sx, w1q, sw1 = _moe_case(3, T, D, I, E, k, kind)
    ref = omoe.gemm1(xq, w1q, sx, sw1, ids, w, I, doweight, kind)
    sid, sw, eid, post = omoe.moe_sorting(ids, w, E, bs)
    alt = omoe.gemm1_sorted(xq, w1q, sx, sw1, sid, sw, eid, post[0], bs, T, k, I, doweight, kind)
    assert np.allclose(ref, alt, rtol=1e-12, atol=1e-12)
    # a subset of tokens leaves the other rows at zero and the chosen ones unchanged
    sub = omoe.gemm1(xq, w1q, sx, sw1, ids, w, I, doweight, kind, tokens_subset=[1, 4])
    assert np.allclose(sub[[1, 4]], ref[[1, 4]], rtol=1e-12, atol=1e-12) and not sub[[0, 2, 3, 5, 6]].any()


def test_moe_gemm1_gate_up_order():
    """Zeroing the up rows zeroes the output; zeroing the gate rows gives silu(0) * up = 0 as
    well, but a huge positive gate turns silu(gate) * up into gate * up: the two halves are told
    apart by which one scales linearly."""
    T, D, I, E, k = 3, 64, 16, 2, 1
    ids, w, xq, sx, w1q, sw1 = _moe_case(5, T, D, I, E, k, "int8")
    sw_up0 = sw1.copy().reshape(E, 2, I)
    sw_up0[:, 1] = 0
    assert not omoe.gemm1(xq, w1q, sx, sw_up0.reshape(-1), ids, w, I, False, "int8").any()
    base = omoe.gemm1(xq, w1q, sx, sw1, ids, w, I, False, "int8")
    sw_up2 = sw1.copy().reshape(E, 2, I)
    sw_up2[:, 1] *= 2
    assert np.allclose(omoe.gemm1(xq, w1q, sx, sw_up2.reshape(-1), ids, w, I, False, "int8"), 2 * base, rtol=1e-12)


def test_moe_gemm2_equal_experts_is_one_dense_matmul():
    """Every expert holding the same W2, every slot of a token holding the same a2 row and
    routing weights summing to one: the weighted sum over slots is a2 @ W2^T."""
    T, I, D, E, k = 5, 64, 48, 3, 3
    g = np.random.default_rng(8)
    ids = np.stack([g.permutation(E)[:k] for _ in range(T)])
    w = g.random((T, k))
    w = (w / w.sum(1, keepdims=True)).astype(np.float32)
    a = g.standard_normal((T, I)).astype(np.float32)
    aq, sa = oq.quant_rows(a, "int8")
    a2q = np.repeat(aq, k, axis=0)
    sa2 = np.repeat(sa.reshape(-1), k)
    W = (g.standard_normal((D, I)) * 0.1).astype(np.float32)
    Wq, sW = oq.quant_rows(W, "int8")
    w2q, sw2 = np.tile(Wq, (E, 1)), np.tile(sW.reshape(-1), E)
    got = omoe.gemm2(a2q, w2q, sa2, sw2, ids, w, D, True, "int8")
    dense = og.run_torch(aq, Wq, sa.reshape(-1), sW.reshape(-1), "int8", "f64")
    assert np.allclose(got, dense * w.astype(np.float64).sum(1, keepdims=True), rtol=1e-12, atol=1e-12)
    assert np.allclose(got, dense, rtol=1e-6, atol=1e-6)
    # without the weights the slots add up: k times the dense product
    assert np.allclose(omoe.gemm2(a2q, w2q, sa2, sw2, ids, w, D, False, "int8"), k * dense, rtol=1e-12)
    sid, sw, eid, post = omoe.moe_sorting(ids, w, E, 4)
    alt = omoe.gemm2_sorted(a2q, w2q, sa2, sw2, sid, sw, eid, post[0], 4, T, k, D, True, "int8")
    assert np.allclose(alt, got, rtol=1e-12, atol=1e-12)


def _bs_case(seed, T=5, D=256, I=64, E=3, k=2):
    g = np.random.default_rng(seed)
    ids = np.stack([g.permutation(E)[:k] for _ in range(T)])
    w = g.random((T, k)).astype(np.float32)
    x = g.standard_normal((T, D)).astype(np.float32)
    w1 = (g.standard_normal((E * 2 * I, D)) * 0.3).astype(np.float32)
    xq, xs = oq.quant_blocks(x, 1, 128)
    w1q, w1s = oq.quant_blocks(w1, 128, 128)
    return ids, w, xq, xs, w1q, w1s


def test_moe_blockscale_one_expert_is_the_dense_blockscale_oracle():
    """Every token routed to expert 0 (top-1): gate and up are dense blockscale GEMMs of x with
    the expert's gate / up rows (gemm.run_torch_blockscale, pinned above)."""
    T, D, I, E = 6, 384, 64, 2
    ids, w, xq, xs, w1q, w1s = _bs_case(4, T, D, I, E, 1)
    ids[:] = 0
    got = omoe.gemm1_blockscale(xq, w1q, xs, w1s, ids, w, I, False)
    gate = og.run_torch_blockscale(xq, w1q[:I], xs, w1s[:I // 128 or 1], "f64") if I >= 128 else None
    # I = 64 rows share one 128-row scale block: expand by hand for the gate and up halves
    from oracle.numerics import e4m3fn_decode
    xd = e4m3fn_decode(xq).astype(np.float64) * np.repeat(xs, 128, axis=1)
    wd = e4m3fn_decode(w1q[:2 * I]).astype(np.float64) * np.repeat(np.repeat(w1s[:1], 2 * I, 0), 128, 1)
    y = xd @ wd.T
    assert np.allclose(got[:, 0], omoe.silu(y[:, :I]) * y[:, I:], rtol=1e-12, atol=1e-12)
    assert gate is None
    # with 128-row halves the dense oracle applies directly
    T, D, I, E = 4, 256, 128, 2
    ids, w, xq, xs, w1q, w1s = _bs_case(5, T, D, I, E, 1)
    ids[:] = 1
    got = omoe.gemm1_blockscale(xq, w1q, xs, w1s, ids, w, I, True)
    rows = slice(2 * I, 4 * I)
    g_ = og.run_torch_blockscale(xq, w1q[2 * I:3 * I], xs, w1s[2:3], "f64")
    u_ = og.run_torch_blockscale(xq, w1q[3 * I:4 * I], xs, w1s[3:4], "f64")
    # (the dense oracle rounds the dequantized operands to float32 first)
    assert np.allclose(got[:, 0], omoe.silu(g_) * u_ * w[:, :1], rtol=1e-5, atol=1e-5)
    del rows


def test_moe_blockscale_stage2_one_expert_and_uniform_scales():
    T, I, D, E, k = 5, 256, 128, 2, 2
    g = np.random.default_rng(9)
    ids = np.stack([g.permutation(E)[:k] for _ in range(T)])
    w = g.random((T, k)).astype(np.float32)
    a2 = g.standard_normal((T * k, I)).astype(np.float32)
    w2 = (g.standard_normal((E * D, I)) * 0.1).astype(np.float32)
    a2q, a2s = oq.quant_blocks(a2, 1, 128)
    w2q, w2s = oq.quant_blocks(w2, 128, 128)
    got = omoe.gemm2_blockscale(a2q, w2q, a2s, w2s, ids, w, D, True)
    # route by route through the dense blockscale oracle
    ref = np.zeros((T, D))
    for t in range(T):
        for s in range(k):
            e = ids[t, s]
            r = t * k + s
            ref[t] += w[t, s] * og.run_torch_blockscale(a2q[r:r + 1], w2q[e * D:(e + 1) * D], a2s[r:r + 1],
                                                         w2s[e * D // 128:(e + 1) * D // 128], "f64")[0]
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-6)
    # equal scales across K blocks reduce to the per-row form
    a2s_u = np.repeat(a2s[:, :1], a2s.shape[1], axis=1)
    w2s_u = np.repeat(w2s[:, :1], w2s.shape[1], axis=1)
    got_u = omoe.gemm2_blockscale(a2q, w2q, a2s_u, w2s_u, ids, w, D, True)
    row_u = omoe.gemm2(a2q, w2q, a2s_u[:, 0], np.repeat(w2s_u[:, 0], 128), ids, w, D, True, "fp8")
    assert np.allclose(got_u, row_u, rtol=1e-5, atol=1e-6)   # dequant_rows rounds to float32


# ---- quantizer arguments of the reference's pertoken_quant (smooth quant, given scales) ------
def test_quant_rows_smooth_and_given_scale_known_answers():
    """tests/utils.py:29-73: x_scale multiplies the rows before the scale is taken; a given
    scale replaces amax/qmax; non-finite given scales become 1."""
    x = np.array([[1.0, -2.0, 4.0], [0.5, 0.25, -1.0]], np.float32)
    q, s = oq.quant_rows(x, "int8", x_scale=np.array([4.0, 2.0, 1.0], np.float32))
    assert q[0].tolist() == [127, -127, 127]                 # row 0 becomes [4, -4, 4]
    assert np.float32(s[0]) == np.float32(4.0) / np.float32(127.0)
    # row 1 becomes [2, 0.5, -1]: scale 2/127, codes 127, 31.75 -> 32, -63.5 -> -64 (half to even)
    assert q[1].tolist() == [127, 32, -64]
    q1, s1 = oq.quant_rows(x, "int8", x_scale=np.ones(3, np.float32))
    q0, s0 = oq.quant_rows(x, "int8")
    assert np.array_equal(q1, q0) and np.array_equal(s1, s0)
    # the computed scale given back reproduces the codes; a doubled scale halves them (rounded)
    qg, sg = oq.quant_rows(x, "int8", scale=s0)
    assert np.array_equal(qg, q0) and np.array_equal(sg, s0)
    qd, _ = oq.quant_rows(x, "int8", scale=2 * s0)
    assert np.array_equal(qd, np.rint((x / (2 * s0)[:, None]).astype(np.float32)).astype(np.int8))
    qn, sn = oq.quant_rows(x, "int8", scale=np.array([np.nan, np.inf], np.float32))
    assert sn.tolist() == [1.0, 1.0] and qn[0].tolist() == [1, -2, 4]


@pytest.mark.parametrize("qd,kind", [(torch.int8, "int8"), (torch.float8_e4m3fn, "fp8")])
def test_pertoken_quant_smooth_and_given_scale_match_oracle(qd, kind):
    """The product's pertoken_quant with the reference's x_scale / scale / scale_dtype arguments
    against the oracle's restatement, byte for byte."""
    from flydsl_amd import quant as pq

    g = torch.Generator().manual_seed(17)
    x = torch.randn(33, 200, generator=g) * 3
    xs = 0.5 + torch.rand(1, 200, generator=g)
    q, s = pq.pertoken_quant(x, x_scale=xs, quant_dtype=qd)
    oq_q, oq_s = oq.quant_rows(x.numpy(), kind, x_scale=xs.numpy())
    assert np.array_equal(q.view(torch.uint8).numpy() if kind == "fp8" else q.numpy(), oq_q)
    assert np.array_equal(s.numpy().reshape(-1), oq_s)
    given = torch.rand(33, 1, generator=g) * 0.05 + 0.01
    q2, s2 = pq.pertoken_quant(x, scale=given, quant_dtype=qd)
    o2_q, o2_s = oq.quant_rows(x.numpy(), kind, scale=given.numpy())
    assert np.array_equal(q2.view(torch.uint8).numpy() if kind == "fp8" else q2.numpy(), o2_q)
    assert torch.equal(s2, given)
    _, s3 = pq.pertoken_quant(x, quant_dtype=qd, scale_dtype=torch.bfloat16)
    assert s3.dtype == torch.bfloat16


# ---- MoE oracle: per-route activations, mixed kinds, group-wise weight scales --------------
def test_moe_per_route_activations_reduce_to_per_token():
    """int8smooth gives stage 1 one activation row per route; when every slot of a token holds
    the token's row and scale, the per-route form is the per-token one."""
    T, D, I, E, k = 6, 64, 32, 4, 2
    ids, w, xq, sx, w1q, sw1 = _moe_case(21, T, D, I, E, k, "int8")
    x3 = np.repeat(xq[:, None, :], k, axis=1)
    sx3 = np.repeat(sx[:, None], k, axis=1)
    a = omoe.gemm1(xq, w1q, sx, sw1, ids, w, I, True, "int8")
    b = omoe.gemm1(x3, w1q, sx3, sw1, ids, w, I, True, "int8")
    assert np.allclose(a, b, rtol=1e-12, atol=1e-12)
    # a route's own row is used: doubling one route's scale doubles only its gate and up
    sx4 = sx3.copy()
    sx4[2, 1] *= 2
    c = omoe.gemm1(x3, w1q, sx4, sw1, ids, w, I, False, "int8")
    ref = omoe.gemm1(x3, w1q, sx3, sw1, ids, w, I, False, "int8")
    diff = np.abs(c - ref).sum(axis=-1)
    assert diff[2, 1] > 0 and np.count_nonzero(diff) == 1


def test_moe_gemm2_reduce_mode_rounds_each_route_row():
    """Reduce mode: each route's weighted row is written in the output type and the rows are then
    summed (compile_moe_gemm2(accumulate=False) + compile_moe_reduction).  Checked against a
    brute-force loop over (token, slot) that rounds every row with torch's own conversion; with
    float64 rows (no rounding) it is the atomic-mode sum."""
    rng = np.random.default_rng(5)
    T, k, E, D, I = 7, 3, 4, 32, 64
    a2 = rng.integers(-127, 128, (T * k, I), dtype=np.int8)
    w2 = rng.integers(-127, 128, (E * D, I), dtype=np.int8)
    sa2 = rng.random(T * k).astype(np.float32) * 0.01
    sw2 = rng.random(E * D).astype(np.float32) * 0.01
    ids = np.stack([rng.permutation(E)[:k] for _ in range(T)])
    tw = rng.random((T, k)).astype(np.float32)
    for rr, tdt in (("bf16", torch.bfloat16), ("f16", torch.float16)):
        got = omoe.gemm2(a2, w2, sa2, sw2, ids, tw, D, True, "int8", route_round=rr)
        want = np.zeros((T, D))
        for t in range(T):
            for s_ in range(k):
                e = ids[t, s_]
                row = np.zeros(D)
                for n in range(D):
                    acc = sum(float(a2[t * k + s_, j]) * float(w2[e * D + n, j]) for j in range(I))
                    row[n] = acc * float(sa2[t * k + s_]) * float(sw2[e * D + n]) * float(tw[t, s_])
                want[t] += torch.from_numpy(row.astype(np.float32)).to(tdt).double().numpy()
        assert np.allclose(got, want, rtol=1e-12, atol=0)
    plain = omoe.gemm2(a2, w2, sa2, sw2, ids, tw, D, True, "int8")
    assert not np.array_equal(plain, got) and np.allclose(plain, got, rtol=2e-3, atol=1e-3)


def test_moe_group_scales_brute_force_and_per_row_reduction():
    """W4A16 group scales: w[e,n,k] * G[e, k // 32, n] (tests/kernels/test_ref.py:44-50,117-123),
    checked by an explicit loop over (token, slot, n, k) on a tiny case, and reducing to the
    per-row form when every group of a row has that row's scale.  Activations are bf16 and the
    weights int4 values (w_kind int8)."""
    from oracle import numerics as on

    g = np.random.default_rng(4)
    T, I, D, E, k, grp = 3, 64, 16, 2, 2, 32
    ids = np.stack([g.permutation(E)[:k] for _ in range(T)])
    tw = g.random((T, k)).astype(np.float32)
    a2 = on.bf16_rne(g.standard_normal((T * k, I)).astype(np.float32))
    w2 = g.integers(-7, 8, size=(E * D, I)).astype(np.int8)
    G = (g.random((E, I // grp, D)) * 0.05 + 0.005).astype(np.float32)
    got = omoe.gemm2(a2, w2, None, None, ids, tw, D, True, "bf16", w_kind="int8", w_groups=G)
    af = on.bf16_to_f32(a2).astype(np.float64)
    want = np.zeros((T, D))
    for t in range(T):
        for s in range(k):
            e = ids[t, s]
            for n in range(D):
                acc = 0.0
                for kk in range(I):
                    wv = float(np.float32(np.float32(w2[e * D + n, kk]) * G[e, kk // grp, n]))   # fp32 dequant
                    acc += af[t * k + s, kk] * wv
                want[t, n] += acc * float(tw[t, s])
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)
    # constant over the groups of a row: the per-row scale path
    sw = (g.random(E * D) * 0.05 + 0.005).astype(np.float32)
    Gc = np.repeat(sw.reshape(E, 1, D), I // grp, axis=1)
    a = omoe.gemm2(a2, w2, None, None, ids, tw, D, True, "bf16", w_kind="int8", w_groups=Gc)
    b = omoe.gemm2(a2, w2, None, sw, ids, tw, D, True, "bf16", w_kind="int8")
    assert np.allclose(a, b, rtol=1e-12, atol=1e-12)
    # stage 1 the same way (gate and up rows of one expert; K = model_dim = 64)
    D1 = 64
    x = on.bf16_rne(g.standard_normal((T, D1)).astype(np.float32))
    w1 = g.integers(-7, 8, size=(E * 2 * I, D1)).astype(np.int8)
    sw1 = (g.random(E * 2 * I) * 0.05 + 0.005).astype(np.float32)
    G1 = np.repeat(sw1.reshape(E, 1, 2 * I), D1 // grp, axis=1)
    c = omoe.gemm1(x, w1, None, None, ids, tw, I, False, "bf16", w_kind="int8", w_groups=G1)
    d = omoe.gemm1(x, w1, None, sw1, ids, tw, I, False, "bf16", w_kind="int8")
    assert np.allclose(c, d, rtol=1e-12, atol=1e-12)
