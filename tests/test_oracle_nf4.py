"""Pins of the CPU oracle's NF4 format code (oracle/nf4.py) against facts that do not come from
the oracle's own formula: the normal-quantile construction of the NF4 table, explicit byte-level
known answers of the format (solution/k_nf4.py:16-21), exact rational arithmetic for the
rounding rules, and a quantise/dequantise error bound."""

from fractions import Fraction

import numpy as np
import pytest
import scipy.stats

from oracle import nf4

F32, F16 = np.float32, np.float16


def _tables(absmax_values):
    """code2/qabs/scale2/offset2 such that absmax of block q is exactly absmax_values[q]
    (scale2 = 1, offset2 = 0, code2 holds the values)."""
    a = np.asarray(absmax_values, dtype=F32)
    nq = -(-a.size // 256) * 256
    code2 = np.zeros(256, F32)
    code2[:a.size] = a
    qabs = np.zeros(nq, np.uint8)
    qabs[:a.size] = np.arange(a.size)
    return qabs, np.ones(nq // 256, F32), np.zeros(nq // 256, F32), code2


def test_nf4_table_matches_normal_quantiles():
    # QLoRA's NF4: quantiles of N(0,1) at 8 points of [offset, 1/2) (positive side) and 7 (negative),
    # plus 0, normalised to [-1, 1]; offset = 0.9677083.
    off = 0.9677083
    pos = scipy.stats.norm.ppf(np.linspace(off, 0.5, 9)[:-1])
    neg = -scipy.stats.norm.ppf(np.linspace(off, 0.5, 8)[:-1])
    v = np.sort(np.concatenate([pos, [0.0], neg]))
    v = v / np.abs(v).max()
    t = nf4.nf4_table()
    assert t.shape == (16,)
    assert np.all(np.diff(t) > 0)
    assert t[0] == -1.0 and t[7] == 0.0 and t[15] == 1.0
    np.testing.assert_allclose(t, v, atol=3e-6, rtol=0)


def test_byte_layout_known_answers():
    # element e lives in byte e // 2, the even element in the high nibble
    a = 0.5  # exact in every format
    qabs, s2, o2, code2 = _tables([a])
    packed = np.zeros(32 * 256, np.uint8)
    packed[0] = 0x0F   # e0 <- code 0 (-1.0), e1 <- code 15 (+1.0)
    packed[1] = 0x7A   # e2 <- code 7 (0.0),  e3 <- code 10
    packed[31] = 0xF0  # e62 <- code 15, e63 <- code 0
    out = nf4.dequant(packed, qabs, s2, o2, code2)
    assert out[0] == F16(-0.5) and out[1] == F16(0.5)
    assert out[2] == 0 and out[3] == F16(F32(nf4.NF4_CODE[10]) * F32(a))
    assert out[62] == F16(0.5) and out[63] == F16(-0.5)


def test_sign_of_zero_follows_absmax():
    qabs, s2, o2, code2 = _tables([0.25, -0.25])
    packed = np.full(32 * 256, 0x77, np.uint8)
    out = nf4.dequant(packed, qabs, s2, o2, code2)
    assert np.all(out[:64] == 0) and not np.any(np.signbit(out[:64]))
    assert np.all(out[64:128] == 0) and np.all(np.signbit(out[64:128]))


def test_absmax_rounds_product_and_sum_separately():
    # find (c, s, o) where two roundings differ from one fused rounding, using exact rationals
    rng = np.random.default_rng(1)
    found = None
    for _ in range(20000):
        c, s, o = rng.uniform(-1, 1, 3).astype(F32)
        exact = Fraction(float(c)) * Fraction(float(s)) + Fraction(float(o))
        fused = F32(float(exact))          # one rounding (float64 of the exact value is exact here
        prod = F32(float(Fraction(float(c)) * Fraction(float(s))))   # ... up to 1 ulp of f64)
        twice = F32(float(Fraction(float(prod)) + Fraction(float(o))))
        if fused != twice:
            found = (c, s, o, twice, fused)
            break
    assert found is not None
    c, s, o, twice, fused = found
    got = nf4.absmax_of(np.zeros(256, np.uint8), np.array([s], F32), np.array([o], F32),
                        np.full(256, c, F32))[0]
    assert got == twice and got != fused


def test_fp16_round_to_nearest_even_and_subnormals():
    tie = F32(1.0 + 3 * 2.0 ** -11)      # halfway between fp16 1+2^-10 and 1+2^-9
    tiny = F32(2.0 ** -20)               # an fp16 subnormal
    qabs, s2, o2, code2 = _tables([tie, tiny])
    packed = np.full(32 * 256, 0xFF, np.uint8)   # code 15 = +1.0 everywhere
    out = nf4.dequant(packed, qabs, s2, o2, code2)
    assert np.all(out[:64] == F16(1.0 + 2.0 ** -9))   # even mantissa, not truncation
    assert np.all(out[64:128] == F16(2.0 ** -20)) and out[64] != 0


def test_dequant_matches_scalar_fp64_path_on_all_bytes():
    # every byte value under three absmax values, each element computed alone: the fp32 product
    # is exact in fp64, so one rounding to fp32 then one to fp16
    a_vals = [0.013671875, -0.0625, 1.7e-3]
    qabs, s2, o2, code2 = _tables(a_vals)
    packed = np.zeros(32 * 256, np.uint8)
    for q in range(3):
        packed[q * 32:(q + 1) * 32] = np.arange(q * 32, q * 32 + 32) % 256
    packed[96:96 + 256] = np.arange(256)
    out = nf4.dequant(packed, qabs, s2, o2, code2)
    table = [float(F32(v)) for v in nf4.NF4_CODE]
    for e in range(2 * (96 + 256)):
        q = min(e // 64, 3)
        a = float(F32(a_vals[q])) if q < 3 else 0.0
        if e >= 192:
            q = e // 64
            a = float(code2[qabs[q]])
        byte = int(packed[e // 2])
        nib = byte >> 4 if e % 2 == 0 else byte & 15
        want = F16(F32(table[nib] * a))
        assert out[e] == want or (out[e] == 0 and want == 0), e


def test_range_dequant_is_the_slice_and_rejects_misalignment():
    rng = np.random.default_rng(0)
    nq = 3 * 1024
    packed = rng.integers(0, 256, nq * 32, dtype=np.uint8)
    qabs = rng.integers(0, 256, nq, dtype=np.uint8)
    code2 = np.sort(rng.uniform(-1, 1, 256)).astype(F32)
    s2 = rng.uniform(1e-3, 2e-2, nq // 256).astype(F32)
    o2 = np.full(nq // 256, 0.02, F32)
    whole = nf4.dequant(packed, qabs, s2, o2, code2)
    part = nf4.dequant_range(packed, qabs, s2, o2, code2, 1024, 3072)
    assert np.array_equal(part.view(np.uint16), whole[1024 * 64:].view(np.uint16))
    with pytest.raises(ValueError):
        nf4.dequant_range(packed, qabs, s2, o2, code2, 256, 3072)


def test_dynamic_map_structure():
    c = nf4.dynamic_map_signed()
    assert c.shape == (256,) and c.dtype == F32
    assert np.all(np.diff(c) > 0)
    assert c[-1] == 1.0 and (c == 0).sum() == 1
    assert (c < 0).sum() == 127 and (c > 0).sum() == 128
    # symmetric except for the appended 1.0
    pos = c[(c > 0) & (c < 1)]
    assert np.array_equal(np.sort(-c[c < 0]), pos)
    # decade structure: 2**i values in (10**(i-7), 10**(i-6)] for i = 0..6
    for i in range(7):
        lo, hi = 10.0 ** (i - 7), 10.0 ** (i - 6)
        assert ((pos > lo) & (pos <= hi * 1.0000001)).sum() == 2 ** i


def test_exact_mean():
    rng = np.random.default_rng(3)
    a = np.abs(rng.standard_normal(4096) * 0.05).astype(F16).astype(F32)
    exact = sum(Fraction(float(v)) for v in a) / len(a)
    assert nf4.exact_mean(a) == F32(float(exact))


def test_quantise_dequantise_error_bound():
    rng = np.random.default_rng(0)
    w = (rng.standard_normal(256 * 1536) * 0.02).astype(F16)
    q = nf4.quantize(w)
    deq = nf4.dequant(q["packed"], q["qabs"], q["scale2"], q["offset2"], q["code2"]).astype(np.float64)
    true_amax = np.abs(w.astype(np.float64)).reshape(-1, 64).max(axis=1)
    dq_amax = nf4.absmax_of(q["qabs"], q["scale2"], q["offset2"], q["code2"]).astype(np.float64)
    # second level: the code table's largest half gap times the block scale, plus fp32 rounding
    gap = np.diff(q["code2"].astype(np.float64)).max() / 2
    s2 = np.repeat(q["scale2"].astype(np.float64), 256)
    assert np.all(np.abs(dq_amax - true_amax) <= gap * s2 + 1e-6)
    # first level: the NF4 table's largest half gap times absmax, plus the absmax error
    hg = np.diff(nf4.nf4_table().astype(np.float64)).max() / 2
    bound = np.repeat(hg * true_amax + np.abs(dq_amax - true_amax), 64) + 1e-3 * np.abs(deq) + 1e-7
    assert np.all(np.abs(deq - w.astype(np.float64)) <= bound)
    # and the codes are the nearest NF4 values almost everywhere (ties aside)
    assert np.mean(np.abs(deq - w) <= np.repeat(hg * dq_amax, 64) * 1.01 + 1e-6) > 0.999
