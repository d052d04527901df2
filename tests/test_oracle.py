"""Pins of the CPU oracle (no GPU): against library routines, closed forms, brute force and the
committed golden fixtures, plus planted mistakes that those pins must catch."""
import glob
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as Fn

from _cases import I64_MAX, I64_MIN, random_case
from oracle import ebag_oracle as orc

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def torch_segment_loop(case, pooling="sum"):
    """baseline/infer.py:256-263 with torch's library routines (fp32 accumulation)."""
    pooled = []
    for f in range(case.F):
        s, e = int(case.offsets[f * case.B]), int(case.offsets[(f + 1) * case.B])
        vals = torch.from_numpy(case.values[s:e])
        local = torch.from_numpy(case.offsets[f * case.B:(f + 1) * case.B + 1] - s)
        w = torch.from_numpy(orc.decode(case.tables[f], case.tdt).copy())
        vals = vals.clamp(0, w.shape[0] - 1)
        emb = Fn.embedding(vals, w)
        res = torch.segment_reduce(emb, reduce="sum", offsets=local, initial=0)
        if pooling == "mean":
            L = (local[1:] - local[:-1]).to(torch.float32)
            res = torch.where(L[:, None] > 0, res / L.clamp(min=1)[:, None], torch.zeros_like(res))
        pooled.append(res)
    return torch.cat(pooled, dim=1).numpy()


def torch_embedding_bag_loop(case, pooling="sum"):
    pooled = []
    for f in range(case.F):
        s, e = int(case.offsets[f * case.B]), int(case.offsets[(f + 1) * case.B])
        w = torch.from_numpy(orc.decode(case.tables[f], case.tdt).copy())
        vals = torch.from_numpy(case.values[s:e]).clamp(0, w.shape[0] - 1)
        local = torch.from_numpy(case.offsets[f * case.B:(f + 1) * case.B + 1] - s)
        pooled.append(Fn.embedding_bag(vals, w, local, mode=pooling, include_last_offset=True))
    return torch.cat(pooled, dim=1).numpy()


def f64_reference(case, pooling="sum"):
    """fp64 pooling of the decoded rows and the fp32 reassociation bound sum_i |x_i| * L * 2^-24."""
    cols = []
    bounds = []
    for f in range(case.F):
        w = orc.decode(case.tables[f], case.tdt).astype(np.float64)
        D = w.shape[1]
        acc = np.zeros((case.B, D))
        absacc = np.zeros((case.B, D))
        for b in range(case.B):
            s, e = case.offsets[f * case.B + b], case.offsets[f * case.B + b + 1]
            rows = np.clip(case.values[s:e], 0, w.shape[0] - 1)
            if e > s:
                acc[b] = w[rows].sum(axis=0)
                absacc[b] = np.abs(w[rows]).sum(axis=0) * (e - s) * 2.0 ** -24
                if pooling == "mean":
                    acc[b] /= (e - s)
                    absacc[b] /= (e - s)
        cols.append(acc)
        bounds.append(absacc)
    return np.concatenate(cols, axis=1), np.concatenate(bounds, axis=1)


CONFIGS = [
    dict(F=3, B=17, dims=(64,), V=(300,), tdt="f32"),
    dict(F=5, B=40, dims=(32, 128, 8), V=(50, 1000), tdt="f32", max_len=40),
    dict(F=2, B=9, dims=(128,), V=(64,), tdt="bf16"),
    dict(F=4, B=25, dims=(16, 100), V=(70,), tdt="f16"),
    dict(F=3, B=12, dims=(512,), V=(20,), tdt="bf16", long_every=5, long_len=300),
]


@pytest.mark.parametrize("cfg", range(len(CONFIGS)))
@pytest.mark.parametrize("pooling", ["sum", "mean"])
def test_c_and_numpy_restatements_agree_bitwise(cfg, pooling):
    case = random_case(100 + cfg, **CONFIGS[cfg])
    for odt in ("f32", "bf16", "f16"):
        a = orc.pool_c(case.values, case.offsets, case.tables, case.tdt, pooling, odt)
        b = orc.pool_np(case.values, case.offsets, case.tables, case.tdt, pooling, odt)
        assert np.array_equal(a, b), (cfg, pooling, odt)


@pytest.mark.parametrize("cfg", range(len(CONFIGS)))
@pytest.mark.parametrize("pooling", ["sum", "mean"])
def test_against_torch_library_routines(cfg, pooling):
    case = random_case(200 + cfg, **CONFIGS[cfg])
    got = orc.pool_c(case.values, case.offsets, case.tables, case.tdt, pooling, "f32")
    ref64, bound = f64_reference(case, pooling)
    assert np.all(np.abs(got - ref64) <= bound + 1e-30)
    if pooling == "sum":
        seg = torch_segment_loop(case, pooling)
        np.testing.assert_allclose(got, seg, rtol=0, atol=5e-5)
    eb = torch_embedding_bag_loop(case, pooling)
    np.testing.assert_allclose(got, eb, rtol=0, atol=5e-5)


@pytest.mark.parametrize("pooling", ["sum", "mean"])
@pytest.mark.parametrize("kind", ["normal", "int"])
def test_cpu_loops_match_the_c_oracle(pooling, kind):
    """oracle/cpu_loops.py (the CPU baseline's loops) against pool_c: exact on integer rows,
    within the fp32 reassociation bound otherwise; clamp cases and empty bags included."""
    from oracle import cpu_loops

    case = random_case(300, F=4, B=33, dims=(64, 128), V=(500,), tdt="f32", kind=kind, max_len=40,
                       long_every=7, long_len=200)
    got = orc.pool_c(case.values, case.offsets, case.tables, "f32", pooling, "f32")
    vals = torch.from_numpy(case.values)
    offs = torch.from_numpy(case.offsets)
    tables = [torch.from_numpy(orc.decode(t, "f32").copy()) for t in case.tables]
    _, bound = f64_reference(case, pooling)
    for loop in (cpu_loops.baseline_loop, cpu_loops.embedding_bag_loop):
        ref = loop(vals, offs, tables, pooling, case.B).numpy()
        assert ref.shape == got.shape
        if kind == "int" and pooling == "sum":
            assert np.array_equal(ref, got), loop.__name__
        else:
            assert np.all(np.abs(ref - got) <= 2 * bound + 1e-30), loop.__name__


def test_reference_layout_equals_global_layout():
    case = random_case(7, F=6, B=31, dims=(64,), V=(400,), tdt="bf16")
    ro, vo = case.reference_layout()
    shared = [case.tables[0]] * case.F
    a = orc.pool_c(case.values, ro, shared, "bf16", "sum", batch=case.B, val_base=vo)
    b = orc.pool_c(case.values, case.offsets, shared, "bf16", "sum")
    assert np.array_equal(a, b)
    g = orc.to_global_offsets(vo, ro, case.B, len(case.values))
    assert np.array_equal(g, case.offsets)


@pytest.mark.parametrize("pooling", ["sum", "mean"])
def test_integer_tables_are_exact(pooling):
    # integer rows in [-32, 32], bags up to 2048 long: every fp32 partial sum is an exact integer
    case = random_case(11, F=3, B=20, dims=(64, 128), V=(1000,), tdt="f32", kind="int", max_len=64,
                       long_every=4, long_len=2048)
    got = orc.pool_c(case.values, case.offsets, case.tables, "f32", pooling, "f32")
    for f in range(case.F):
        w = case.tables[f].astype(np.int64)
        D = w.shape[1]
        col = sum(case.tables[g].shape[1] for g in range(f))
        for b in range(case.B):
            s, e = case.offsets[f * case.B + b], case.offsets[f * case.B + b + 1]
            exact = w[np.clip(case.values[s:e], 0, w.shape[0] - 1)].sum(axis=0) if e > s else np.zeros(D, np.int64)
            want = exact.astype(np.float32)
            if pooling == "mean" and e > s:
                want = want / np.float32(e - s)
            assert np.array_equal(got[b, col:col + D], want), (f, b)


def test_rowid_tables_identify_every_row():
    # table[r, j] = bit j of r: a length-1 bag returns the bits of the row actually read
    V, D = 5000, 16
    r = np.arange(V, dtype=np.int64)
    table = ((r[:, None] >> np.arange(D)) & 1).astype(np.float32)
    ids = np.array([0, 1, V - 1, V, -1, I64_MAX, I64_MIN, 1234, -(2 ** 40), V + 99], dtype=np.int64)
    offsets = np.arange(len(ids) + 1, dtype=np.int64)
    got = orc.pool_c(ids, offsets, [table], "f32", "sum", "f32")
    rows = np.clip(ids, 0, V - 1)
    want = ((rows[:, None] >> np.arange(D)) & 1).astype(np.float32)
    assert np.array_equal(got, want)
    assert list(rows[3:7]) == [V - 1, 0, V - 1, 0]


def test_empty_bags_pool_to_positive_zero():
    V, D = 10, 8
    table = np.full((V, D), -3.5, dtype=np.float32)
    offsets = np.array([0, 0, 2, 2, 2], dtype=np.int64)  # bags: empty, 2 rows, empty, empty
    ids = np.array([1, 2], dtype=np.int64)
    for pooling in ("sum", "mean"):
        for odt in ("f32", "bf16", "f16"):
            got = orc.pool_c(ids, offsets, [table], "f32", pooling, odt)
            raw = got.view(np.uint32) if odt == "f32" else got
            assert np.all(raw[[0, 2, 3]] == 0), (pooling, odt)  # +0 bit pattern
    got = orc.pool_c(ids, offsets, [table], "f32", "mean", "f32")
    assert np.all(got[1] == -3.5)


def test_brute_force_tiny():
    # pure-Python scalar loop, fp32 at every step, on tiny inputs
    for seed in range(5):
        case = random_case(300 + seed, F=2, B=5, dims=(3, 5), V=(9,), tdt="f32", max_len=6)
        for pooling in ("sum", "mean"):
            got = orc.pool_c(case.values, case.offsets, case.tables, "f32", pooling, "f32")
            col = 0
            for f in range(case.F):
                t = case.tables[f]
                for b in range(case.B):
                    s, e = int(case.offsets[f * case.B + b]), int(case.offsets[f * case.B + b + 1])
                    for d in range(t.shape[1]):
                        acc = np.float32(0.0)
                        for i in range(s, e):
                            row = min(max(int(case.values[i]), 0), t.shape[0] - 1)
                            acc = np.float32(acc + t[row, d])
                        if pooling == "mean" and e > s:
                            acc = np.float32(acc / np.float32(e - s))
                        assert got[b, col + d] == acc
                col += t.shape[1]


def test_bf16_encoder_matches_torch():
    rng = np.random.default_rng(5)
    x = np.concatenate([
        rng.normal(0, 1, 20000).astype(np.float32),
        rng.normal(0, 1e-38, 2000).astype(np.float32),                       # subnormals
        (rng.integers(0, 2 ** 16, 4000, dtype=np.uint32) << 16 | 0x8000).view(np.float32),  # exact ties
        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 3.4028235e38, -3.4028235e38, 3.3961776e38], np.float32),
    ])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    for got in (orc.f32_to_bf16(x), orc.c_f32_to_bf16(x)):
        fin = ~np.isnan(x)
        assert np.array_equal(got[fin], want[fin])
        assert np.all(np.isnan(orc.bf16_to_f32(got[~fin])))
    # decode is exact: bf16 -> fp32 -> bf16 is the identity on every non-NaN pattern
    pats = np.arange(2 ** 16, dtype=np.uint32).astype(np.uint16)
    dec = orc.bf16_to_f32(pats)
    keep = ~np.isnan(dec)
    assert np.array_equal(orc.f32_to_bf16(dec)[keep], pats[keep])
    assert np.array_equal(dec, torch.from_numpy(pats.view(np.int16)).view(torch.bfloat16).float().numpy(),
                          equal_nan=True)


def test_f16_encoder_matches_numpy():
    rng = np.random.default_rng(6)
    x = np.concatenate([
        rng.normal(0, 1, 20000).astype(np.float32),
        rng.normal(0, 1e-5, 5000).astype(np.float32),       # fp16 subnormal range
        rng.normal(0, 1e5, 2000).astype(np.float32),        # overflow range
        (np.arange(-30, 17, dtype=np.float32)[:, None] * 0 + 2.0 ** np.arange(-30, 17)[:, None]
         * (1 + np.array([2 ** -11, 3 * 2 ** -11], np.float32))).reshape(-1).astype(np.float32),  # ties
        np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 65519.996, 65520.0, 2.0 ** -25, 2.0 ** -24], np.float32),
    ])
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(orc.c_f32_to_f16(x), want)
    pats = np.arange(2 ** 16, dtype=np.uint32).astype(np.uint16)
    a = orc.c_f16_to_f32(pats)
    b = pats.view(np.float16).astype(np.float32)
    assert np.array_equal(a, b, equal_nan=True)


# ---- planted mistakes: each plausible bug in a restatement must fail one of the pins ----------
def _mutant_no_clamp(values, offsets, tables, tdt, pooling, odt):
    V = tables[0].shape[0]
    return orc.pool_c(np.mod(values, V), offsets, tables, tdt, pooling, odt)  # wraps instead of clamps


def _mutant_off_by_one(values, offsets, tables, tdt, pooling, odt):
    o = offsets.copy()
    o[1:-1] += 1  # bag boundaries shifted by one element
    return orc.pool_c(values, o, tables, tdt, pooling, odt)


def _mutant_swapped_fields(values, offsets, tables, tdt, pooling, odt):
    t = list(tables)
    t[0], t[1] = t[1], t[0]
    return orc.pool_c(values, offsets, t, tdt, pooling, odt)


def _mutant_mean_for_sum(values, offsets, tables, tdt, pooling, odt):
    return orc.pool_c(values, offsets, tables, tdt, "mean" if pooling == "sum" else "sum", odt)


@pytest.mark.parametrize("mutant", [_mutant_no_clamp, _mutant_off_by_one, _mutant_swapped_fields, _mutant_mean_for_sum])
def test_pins_catch_planted_mistakes(mutant):
    # the integer-table pin (exact closed form) must reject each mutant
    case = random_case(13, F=2, B=30, dims=(16,), V=(200,), tdt="f32", kind="int", max_len=8, clamp_frac=0.3)
    good = orc.pool_c(case.values, case.offsets, case.tables, "f32", "sum", "f32")
    bad = mutant(case.values, case.offsets, case.tables, "f32", "sum", "f32")
    want = torch_segment_loop(case, "sum")
    assert np.array_equal(good, want)
    assert not np.array_equal(bad, want)


# ---- golden fixtures --------------------------------------------------------------------------
def _fixtures():
    return sorted(glob.glob(os.path.join(GOLDEN, "*.npz")))


def test_golden_fixtures_exist():
    assert len(_fixtures()) >= 5


@pytest.mark.parametrize("path", _fixtures(), ids=lambda p: os.path.basename(p))
def test_oracle_reproduces_golden_fixtures(path):
    from golden import fixture_io

    fx = fixture_io.load(path)
    got = orc.pool_c(fx["values"], fx["offsets"], fx["tables"], fx["table_dtype"], fx["pooling"],
                     fx["out_dtype"], batch=fx["batch"], val_base=fx.get("val_base"))
    assert np.array_equal(got, fx["expected"])


# ---- input LayerNorm (online_best/infer.py:829-858) ----------------------------------------------
def _ln_case(seed, rows=16, cols=448, offset=0.0, scale=1.0):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, cols)) * scale + offset).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    b = (0.1 * rng.standard_normal(cols)).astype(np.float32)
    return x, g, b


@pytest.mark.parametrize("cols", [7, 448, 3584])
def test_layer_norm_matches_torch(cols):
    x, g, b = _ln_case(cols, cols=cols)
    y, mean, rstd = orc.layer_norm_np(x, g, b, 1e-5)
    ref = Fn.layer_norm(torch.from_numpy(x).double(), (cols,), torch.from_numpy(g).double(),
                        torch.from_numpy(b).double(), 1e-5).numpy()
    np.testing.assert_allclose(y, ref, rtol=2e-5, atol=2e-5)
    np.testing.assert_allclose(mean, x.astype(np.float64).mean(axis=1), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(rstd, 1 / np.sqrt(x.astype(np.float64).var(axis=1) + 1e-5), rtol=1e-5)


def test_layer_norm_closed_forms():
    # constant rows of exactly representable values: mean exact, deviations exactly 0, y == beta
    cols = 256
    x = np.repeat(np.array([[1.0], [-3.5], [0.0], [1024.0]], np.float32), cols, axis=1)
    g = np.linspace(0.5, 2, cols).astype(np.float32)
    b = np.linspace(-1, 1, cols).astype(np.float32)
    y, mean, rstd = orc.layer_norm_np(x, g, b, 1e-5)
    assert np.array_equal(mean, x[:, 0])
    assert np.array_equal(y, np.broadcast_to(b, y.shape))
    assert np.all(rstd == np.float32(1) / np.sqrt(np.float32(1e-5)))
    # gamma = 1, beta = 0: every row has mean ~0 and variance var / (var + eps)
    x, _, _ = _ln_case(3, rows=8, cols=1024, scale=3.0)
    y, _, _ = orc.layer_norm_np(x, np.ones(1024, np.float32), np.zeros(1024, np.float32), 1e-5)
    v = x.astype(np.float64).var(axis=1)
    np.testing.assert_allclose(y.astype(np.float64).mean(axis=1), 0, atol=1e-6)
    np.testing.assert_allclose(y.astype(np.float64).var(axis=1), v / (v + 1e-5), rtol=1e-5)


def test_layer_norm_planted_mistakes_are_caught():
    def torch_ref(x, g, b):
        return Fn.layer_norm(torch.from_numpy(x).double(), (x.shape[1],), torch.from_numpy(g).double(),
                             torch.from_numpy(b).double(), 1e-5).numpy()

    # well-conditioned rows: unbiased variance (N-1) and a wrong eps are visible at 1e-4
    x, g, b = _ln_case(8, rows=8, cols=64)
    ref = torch_ref(x, g, b)
    assert np.allclose(orc.layer_norm_np(x, g, b, 1e-5)[0], ref, rtol=1e-4, atol=1e-4)
    mean = x.mean(axis=1, dtype=np.float64)[:, None]
    v = x.var(axis=1, dtype=np.float64)[:, None]
    unbiased = (x - mean) / np.sqrt(x.var(axis=1, ddof=1, dtype=np.float64)[:, None] + 1e-5) * g + b
    wrong_eps = (x - mean) / np.sqrt(v + 1e-2) * g + b
    for wrong in (unbiased, wrong_eps):
        assert not np.allclose(wrong, ref, rtol=1e-4, atol=1e-4)

    # large mean, small spread: the two-pass variance survives, a one-pass E[x^2] - E[x]^2 in fp32
    # or skipping the centring does not (fp32 rounding of the mean alone costs ~3e-3 here)
    x, g, b = _ln_case(9, rows=8, cols=512, offset=3000.0, scale=0.05)
    ref = torch_ref(x, g, b)
    assert np.allclose(orc.layer_norm_np(x, g, b, 1e-5)[0], ref, rtol=1e-2, atol=1e-2)
    n = x.shape[1]
    m32 = (x.sum(axis=1, dtype=np.float32) / np.float32(n)).astype(np.float32)[:, None]
    one_pass_var = np.maximum((x * x).sum(axis=1, dtype=np.float32)[:, None] / np.float32(n) - m32 * m32, 0)
    one_pass = (x - m32) / np.sqrt(one_pass_var + np.float32(1e-5)) * g + b
    no_centre = x / np.sqrt(x.var(axis=1, dtype=np.float64)[:, None] + 1e-5) * g + b
    for wrong in (one_pass, no_centre):
        assert not np.allclose(wrong, ref, rtol=1e-2, atol=1e-2)


# ---- input LayerNorm, then the encoder's Linear (online_best/infer.py:1061-1085) ----------------
def _lin_case(seed, rows=12, cols=448, n=40):
    x, g, b = _ln_case(seed, rows=rows, cols=cols)
    rng = np.random.default_rng(seed + 100)
    w = orc.decode(orc.encode((0.05 * rng.standard_normal((n, cols))).astype(np.float32), "bf16"), "bf16")
    bias = (0.1 * rng.standard_normal(n)).astype(np.float32)
    return x, g, b, w, bias


def test_layer_norm_linear_matches_torch():
    """Against torch's own layer_norm and linear in float64 on the same bf16-rounded operands:
    the oracle's normalised rows are layer_norm_np's, rounded to bf16 (as the reference stores
    them), and its product is exact up to float64 rounding."""
    x, g, b, w, bias = _lin_case(1)
    y, a, absum = orc.layer_norm_linear_np(x, g, b, 1e-5, w, bias)
    ln = Fn.layer_norm(torch.from_numpy(x).double(), (x.shape[1],), torch.from_numpy(g).double(),
                       torch.from_numpy(b).double(), 1e-5)
    a_t = ln.float().to(torch.bfloat16).double()
    # the fp32 LayerNorm and torch's fp64 one round to the same bf16 value except near a midpoint
    assert (a_t.numpy() == a).mean() > 0.99
    ref = Fn.linear(torch.from_numpy(a).double(), torch.from_numpy(w).double(), torch.from_numpy(bias).double())
    np.testing.assert_allclose(y, ref.numpy(), rtol=1e-12, atol=1e-12)
    ref_t = Fn.linear(a_t, torch.from_numpy(w).double(), torch.from_numpy(bias).double()).numpy()
    assert np.all(np.abs(y - ref_t) <= 2.0 ** -8 * absum + 1e-12)  # one bf16 ulp per operand at most
    assert np.all(absum >= np.abs(y - bias[None, :]) - 1e-12)


def test_layer_norm_linear_closed_forms():
    # weight = the first n rows of the identity: y is the normalised block's first n columns plus
    # the bias, exactly; a given mean / rstd is used as given
    x, g, b, _, bias = _lin_case(2, cols=64, n=16)
    eye = np.eye(16, 64, dtype=np.float32)
    y, a, _ = orc.layer_norm_linear_np(x, g, b, 1e-5, eye, bias)
    assert np.array_equal(y, a[:, :16].astype(np.float64) + bias.astype(np.float64))
    ln, _, _ = orc.layer_norm_np(x, g, b, 1e-5)
    assert np.array_equal(a, orc.decode(orc.encode(ln, "bf16"), "bf16"))
    mean = np.full(x.shape[0], 0.5, np.float32)
    rstd = np.full(x.shape[0], 2.0, np.float32)
    y2, a2, _ = orc.layer_norm_linear_np(x, g, b, 1e-5, eye, None, mean=mean, rstd=rstd)
    want = ((x - np.float32(0.5)) * np.float32(2.0)).astype(np.float32) * g + b
    assert np.array_equal(a2, orc.decode(orc.encode(want.astype(np.float32), "bf16"), "bf16"))
    assert np.array_equal(y2, a2[:, :16].astype(np.float64))


def test_layer_norm_linear_planted_mistakes_are_caught():
    """The bound the GPU test uses (one bf16 ulp per operand plus fp32 accumulation) rejects a
    transposed weight, a missing bias, a skipped LayerNorm and gamma / beta swapped."""
    x, g, b, w, bias = _lin_case(3, cols=64, n=64)
    y, a, absum = orc.layer_norm_linear_np(x, g, b, 1e-5, w, bias)
    tol = 2.0 ** -8 * np.abs(y) + (2.0 ** -8 + 64 * 2.0 ** -24) * absum + 1e-12

    def ok(got):
        return np.all(np.abs(got - y) <= tol)

    assert ok(a.astype(np.float64) @ w.T.astype(np.float64) + bias)
    assert not ok(a.astype(np.float64) @ w.astype(np.float64) + bias)  # transposed weight
    assert not ok(a.astype(np.float64) @ w.T.astype(np.float64))  # no bias
    assert not ok(x.astype(np.float64) @ w.T.astype(np.float64) + bias)  # no LayerNorm
    assert not ok(orc.layer_norm_linear_np(x, b, g, 1e-5, w, bias)[0])  # gamma / beta swapped
