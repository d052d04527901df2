"""Pins of the oracle's int8 restatements (no GPU).

- fma: the C library's fmaf, the numpy round-to-odd emulation (oracle.fma_np) and exact rational
  arithmetic agree bit for bit, including products on an fp32 midpoint and cancellations where an
  unfused multiply-add gives a different answer.
- quantize_embedding_int8 (online_best/infer.py:895-901): C and numpy restatements agree; closed
  forms (zero rows, the row maximum maps to +-127, exact ties round half to even); the division
  part matches torch's own `round().clamp().to(int8)` for the same scales; the scale is within one
  ulp of the true quotient row_max / 127.
- int8 pooling (online_best/infer.py:926-940): C oracle == numpy oracle; closed forms; the test
  data distinguishes the fused accumulation from an unfused one.
The exact device semantics of the scale (multiply by the fp32 reciprocal of 127) are pinned against
torch's own device evaluation of the reference expression in the GPU tests.
"""
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import ebag_oracle as orc


def _rn32(x: Fraction) -> np.float32:
    """Exact round-to-nearest-even of a rational to fp32 (brute force over the neighbours)."""
    f = np.float32(float(x))
    cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
    best = None
    for c in cands:
        if not np.isfinite(c):
            continue
        d = abs(Fraction(float(c)) - x)
        key = (d, int(np.float32(c).view(np.uint32)) & 1)  # ties: even significand first
        if best is None or key < best[0]:
            best = (key, c)
    return np.float32(best[1])


def _exact_fma(a, b, c):
    return np.array([_rn32(Fraction(float(x)) * Fraction(float(y)) + Fraction(float(z)))
                     for x, y, z in zip(a, b, c)], dtype=np.float32)


def _hard_fma_cases():
    one_p = np.float32(1 + 2.0 ** -12)
    a, b, c = [], [], []
    # product exactly on an fp32 midpoint (1 + 2^-11 + 2^-24); a tiny addend decides the direction
    for tiny in (2.0 ** -60, -(2.0 ** -60), 2.0 ** -100, 0.0):
        a.append(one_p), b.append(one_p), c.append(np.float32(tiny))
    # c = -RN(a*b): the fused result is the rounding error of the product, the unfused one is 0
    rng = np.random.default_rng(5)
    for _ in range(16):
        x, y = rng.standard_normal(2).astype(np.float32)
        a.append(x), b.append(y), c.append(-np.float32(x * y))
    # int8 x scale + accumulator, as the pooling forms them
    for _ in range(64):
        a.append(np.float32(rng.integers(-128, 128)))
        b.append(np.float32(rng.random() * 0.02))
        c.append(np.float32(rng.standard_normal()))
    return np.array(a, np.float32), np.array(b, np.float32), np.array(c, np.float32)


def test_fma_three_ways_agree():
    a, b, c = _hard_fma_cases()
    rng = np.random.default_rng(11)
    ra, rb, rc = (rng.standard_normal(200).astype(np.float32) * np.float32(2.0) ** rng.integers(-20, 20, 200)
                  for _ in range(3))
    a, b, c = np.concatenate([a, ra]), np.concatenate([b, rb]), np.concatenate([c, rc])
    exact = _exact_fma(a, b, c)
    assert np.array_equal(orc.c_fmaf(a, b, c).view(np.uint32), exact.view(np.uint32))
    assert np.array_equal(orc.fma_np(a, b, c).view(np.uint32), exact.view(np.uint32))
    # the data can tell a fused multiply-add from an unfused one and from double rounding
    unfused = ((a * b).astype(np.float32) + c).astype(np.float32)
    double_rounded = (a.astype(np.float64) * b + c).astype(np.float32)
    assert (unfused != exact).sum() >= 16
    assert (double_rounded != exact).sum() >= 1


def test_fma_np_large_random():
    rng = np.random.default_rng(3)
    n = 200_000
    a = rng.integers(-128, 128, n).astype(np.float32)
    b = (rng.random(n) * 0.03).astype(np.float32)
    c = rng.standard_normal(n).astype(np.float32)
    assert np.array_equal(orc.fma_np(a, b, c).view(np.uint32), orc.c_fmaf(a, b, c).view(np.uint32))


# ------------------------------------------------------------------------------------------------
# quantiser
# ------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_quantize_c_matches_numpy(dt):
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((300, 72)) * np.float32(2.0) ** rng.integers(-12, 6, (300, 1))).astype(np.float32)
    x[5] = 0.0
    tab = orc.encode(x, dt)
    q1, s1 = orc.quantize_int8_c(tab, dt)
    q2, s2 = orc.quantize_int8_np(orc.decode(tab, dt))
    assert np.array_equal(q1, q2)
    assert np.array_equal(s1.view(np.uint32), s2.view(np.uint32))


def test_quantize_closed_forms():
    # zero row: scale is fp32(1e-8) exactly and every q is 0 (a missing clamp gives NaN / 0-division)
    q, s = orc.quantize_int8_np(np.zeros((1, 32), np.float32))
    assert s[0] == np.float32(1e-8) and not q.any()
    # the row maximum in absolute value maps to +-127
    rng = np.random.default_rng(1)
    x = rng.standard_normal((200, 64)).astype(np.float32)
    q, s = orc.quantize_int8_np(x)
    am = np.abs(x).argmax(axis=1)
    assert np.array_equal(np.abs(q[np.arange(200), am]), np.full(200, 127, np.int8))
    assert q.min() >= -127 and q.max() <= 127


def test_quantize_ties_round_half_to_even():
    # find a row maximum whose scale is exactly 2^-7; then w = (k + 1/2) * 2^-7 divides exactly
    target = np.float32(2.0 ** -7)
    m = np.float32(127 * 2.0 ** -7)
    for _ in range(64):
        s = orc.quantize_int8_np(np.array([[m]], np.float32))[1][0]
        if s == target:
            break
        m = np.nextafter(m, np.float32(np.inf) if s < target else np.float32(-np.inf))
    assert s == target
    ks = np.array([0.5, 1.5, 2.5, 3.5, -0.5, -2.5, -3.5, 125.5, 126.5], np.float32)
    row = np.concatenate([[m], ks * target]).astype(np.float32)[None, :]
    want = np.array([0, 2, 2, 4, 0, -2, -4, 126, 126], np.int8)
    q, s = orc.quantize_int8_np(row)
    assert s[0] == target and np.array_equal(q[0, 1:], want)
    qc, _ = orc.quantize_int8_c(row, "f32")
    assert np.array_equal(qc[0, 1:], want)
    # planted mistakes the tie data exposes: half away from zero, truncation
    away = np.sign(ks) * np.floor(np.abs(ks) + 0.5)
    assert not np.array_equal(away.astype(np.int8), want)
    assert not np.array_equal(np.trunc(ks).astype(np.int8), want)


@pytest.mark.parametrize("dt,torch_dt", [("f32", torch.float32), ("bf16", torch.bfloat16), ("f16", torch.float16)])
def test_quantize_matches_torch_for_given_scales(dt, torch_dt):
    """The division / rounding / clamp half of the quantiser against torch (CPU), and the scale
    half against the true quotient: within one ulp, and equal for most rows."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((2000, 40)).astype(np.float32)
    tab = orc.encode(x, dt)
    q, s = orc.quantize_int8_c(tab, dt)
    w = torch.from_numpy(orc.decode(tab, dt)).to(torch_dt)
    st = torch.from_numpy(s)
    qt = (w.float() / st.unsqueeze(1)).round().clamp(-128, 127).to(torch.int8)
    assert torch.equal(qt, torch.from_numpy(q))
    row_max = w.abs().max(dim=1).values.float()
    true_q = torch.clamp(row_max / 127.0, min=1e-8).numpy()  # torch on the CPU divides exactly
    ulp = np.abs(s.view(np.int32).astype(np.int64) - true_q.view(np.int32).astype(np.int64))
    assert ulp.max() <= 1
    assert (ulp == 0).mean() > 0.8
    # a planted divisor of 128 is far outside that band
    wrong = np.maximum(row_max.numpy() / np.float32(128.0), np.float32(1e-8)).astype(np.float32)
    assert np.abs(wrong.view(np.int32).astype(np.int64) - true_q.view(np.int32).astype(np.int64)).min() > 1000


# ------------------------------------------------------------------------------------------------
# int8 pooling
# ------------------------------------------------------------------------------------------------
def _int8_case(rng, F=5, B=33, V=200, D=32, maxlen=9):
    tables = []
    for _ in range(F):
        q = rng.integers(-128, 128, (V, D)).astype(np.int8)
        sc = (rng.random(V) * 0.02 + 1e-4).astype(np.float32)
        tables.append((q, sc))
    lens = rng.integers(0, maxlen + 1, F * B)
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    values = rng.integers(-5, V + 5, int(offsets[-1])).astype(np.int64)  # some out of range: clamped
    return values, offsets, tables


@pytest.mark.parametrize("pooling", ["sum", "mean"])
@pytest.mark.parametrize("odt", ["f32", "bf16", "f16"])
def test_int8_pool_c_matches_numpy(pooling, odt):
    rng = np.random.default_rng(21)
    values, offsets, tables = _int8_case(rng)
    a = orc.pool_c(values, offsets, tables, "i8", pooling, odt)
    b = orc.pool_np(values, offsets, tables, "i8", pooling, odt)
    assert np.array_equal(a, b)


def test_int8_pool_closed_forms():
    rng = np.random.default_rng(2)
    V, D = 50, 16
    q = rng.integers(-128, 128, (V, D)).astype(np.int8)
    # power-of-two scales: every product and every partial sum of <= 4 rows is exact
    sc = (np.float32(2.0) ** rng.integers(-10, -2, V)).astype(np.float32)
    values = rng.integers(0, V, 4 * 8).astype(np.int64)
    offsets = np.arange(0, 33, 4, dtype=np.int64)
    out = orc.pool_c(values, offsets, [(q, sc)], "i8", "sum", "f32")
    want = (q[values].astype(np.float64) * sc[values][:, None]).reshape(8, 4, D).sum(axis=1)
    assert np.array_equal(out, want.astype(np.float32))
    # single-row bags are the correctly rounded product
    sc2 = rng.random(V).astype(np.float32)
    out1 = orc.pool_c(values[:8], np.arange(9, dtype=np.int64), [(q, sc2)], "i8", "sum", "f32")
    want1 = (q[values[:8]].astype(np.float64) * sc2[values[:8]][:, None]).astype(np.float32)
    assert np.array_equal(out1, want1)


def test_int8_pool_data_separates_fused_from_unfused():
    rng = np.random.default_rng(21)
    values, offsets, tables = _int8_case(rng)
    fused = orc.pool_c(values, offsets, tables, "i8", "sum", "f32")
    # planted mistake: dequantise first (round q*s), then add
    deq = [(q.astype(np.float32) * s[:, None]).astype(np.float32) for q, s in tables]
    unfused = orc.pool_c(values, offsets, deq, "f32", "sum", "f32")
    assert (fused != unfused).sum() > 100
