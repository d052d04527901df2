"""The input LayerNorm and the encoder's Linear in one matrix-core kernel (online_best/infer.py:
1061-1085), through the C ABI, on the GPU.

Bar:
- integer-valued operands (every product and partial sum exact in fp32): the output equals the
  exactly computed result rounded once, bit for bit, for the plain Linear and for the LayerNorm
  path with power-of-two statistics, over tile edges (rows, outputs and K not multiples of the
  tiles) and both tile shapes;
- realistic operands: with the kernel's own statistics (cti_ebag_layernorm with no output), the
  normalised operand is the LayerNorm kernel's bit for bit, so the output must meet the fp32
  accumulation bound K * 2^-23 * sum|a w| plus the output rounding; against the oracle's own
  statistics (layer_norm_np, then bf16, then a float64 product) one bf16 ulp per operand more;
- the statistics match layer_norm_np's; RepEncoder.forward, with this kernel or with the
  LayerNorm kernel and torch's Linear, matches the oracle's chain pool_c -> layer_norm_np -> bf16
  -> Linear.
"""
import numpy as np
import pytest
import torch

from oracle import ebag_oracle as orc

pytestmark = pytest.mark.gpu


def _bf16(x, dev):
    return torch.from_numpy(orc.encode(np.asarray(x, np.float32), "bf16")).view(torch.int16).view(torch.bfloat16).to(dev)


def _np(t):
    t = t.detach().cpu()
    return t.float().numpy() if t.dtype == torch.bfloat16 else t.numpy()


def _exact_round(y64, odt):
    """The exactly computed result rounded once to the output type (RNE)."""
    y32 = y64.astype(np.float32)  # exact: integer sums below 2^24
    assert np.array_equal(y32.astype(np.float64), y64)
    return y32 if odt == torch.float32 else orc.decode(orc.encode(y32, "bf16"), "bf16")


SHAPES = [  # (rows, cols, out_features): tile edges in every dimension, every kernel form
    # K not a multiple of 128: the general form (64 x 256 tiles)
    (1, 8, 1), (5, 72, 33), (300, 136, 512), (77, 200, 300),
    # K a multiple of 128: 128 x 128 tiles, and 128 x 256 tiles from two per CU on
    (64, 640, 128), (100, 3584, 200), (4096, 3584, 512), (8192, 896, 512), (129, 14336, 96),
    (32768, 256, 512), (40000, 128, 300)]


@pytest.mark.parametrize("rows,cols,n", SHAPES)
@pytest.mark.parametrize("odt", [torch.bfloat16, torch.float32])
def test_integer_operands_exact(pkg, dev, rows, cols, n, odt):
    print(f"linear exact rows={rows} cols={cols} n={n} out={odt}", flush=True)
    rng = np.random.default_rng(rows + cols + n)
    x = rng.integers(-1, 2, (rows, cols)).astype(np.float32)
    w = rng.integers(-1, 2, (n, cols)).astype(np.float32)
    bias = rng.integers(-8, 9, n).astype(np.float32)
    got = pkg.layer_norm_linear(_bf16(x, dev), _bf16(w, dev), torch.from_numpy(bias).to(dev), out_dtype=odt)
    torch.cuda.synchronize()
    want = _exact_round(x.astype(np.float64) @ w.T.astype(np.float64) + bias, odt)
    assert np.array_equal(_np(got), want)


@pytest.mark.parametrize("rows,cols,n", [(7, 72, 40), (100, 3584, 200), (4096, 3584, 512), (300, 640, 512),
                                         (33000, 256, 512)])
@pytest.mark.parametrize("pdt", [torch.bfloat16, torch.float32])
def test_layer_norm_operands_exact(pkg, dev, rows, cols, n, pdt):
    """Statistics and parameters that keep the normalised operand exact: x and mean small
    integers, rstd a power of two, gamma in {1, 2}, beta an integer, so a = ((x - mean) * rstd) *
    gamma + beta is an integer below 2^8 (exact in bf16) and must land in the right row and
    column; swapping gamma and beta, or mean and rstd, changes the result."""
    print(f"ln-linear exact rows={rows} cols={cols} n={n} params={pdt}", flush=True)
    rng = np.random.default_rng(rows * 7 + cols)
    x = rng.integers(-3, 4, (rows, cols)).astype(np.float32)
    mean = rng.integers(-2, 3, rows).astype(np.float32)
    rstd = np.where(rng.random(rows) < 0.5, 1.0, 2.0).astype(np.float32)
    gamma = rng.integers(1, 3, cols).astype(np.float32)
    beta = rng.integers(-4, 5, cols).astype(np.float32)
    w = rng.integers(-1, 2, (n, cols)).astype(np.float32)
    bias = rng.integers(-8, 9, n).astype(np.float32)
    a = ((x - mean[:, None]) * rstd[:, None]) * gamma + beta
    assert np.abs(a).max() < 256
    to_p = (lambda v: _bf16(v, dev)) if pdt == torch.bfloat16 else (lambda v: torch.from_numpy(v).to(dev))
    got = pkg.layer_norm_linear(_bf16(x, dev), _bf16(w, dev), _bf16(bias, dev), mean=torch.from_numpy(mean).to(dev),
                                rstd=torch.from_numpy(rstd).to(dev), norm_weight=to_p(gamma), norm_bias=to_p(beta),
                                out_dtype=torch.float32)
    torch.cuda.synchronize()
    want = a.astype(np.float64) @ w.T.astype(np.float64) + bias
    assert np.array_equal(_np(got).astype(np.float64), want)


def _realistic(rows, cols, n, seed, dev):
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = (0.02 * torch.randn(rows, cols, generator=g) + 0.003).to(torch.bfloat16)
    gamma = (1 + 0.1 * torch.randn(cols, generator=g)).to(torch.bfloat16)
    beta = (0.1 * torch.randn(cols, generator=g)).to(torch.bfloat16)
    w = (torch.randn(n, cols, generator=g) / cols ** 0.5).to(torch.bfloat16)
    bias = (0.1 * torch.randn(n, generator=g)).to(torch.bfloat16)
    return [t.to(dev) for t in (x, gamma, beta, w, bias)]


@pytest.mark.parametrize("rows,cols,n", [(4096, 3584, 512), (33, 14336, 512), (777, 896, 256), (32768, 1024, 512),
                                         (50, 200, 64)])
def test_realistic_operands_against_the_oracle(pkg, dev, rows, cols, n):
    print(f"ln-linear realistic rows={rows} cols={cols} n={n}", flush=True)
    x, gamma, beta, w, bias = _realistic(rows, cols, n, rows + cols, dev)
    mean, rstd = pkg.layer_norm_stats(x, 1e-5)
    y = pkg.layer_norm_linear(x, w, bias, mean=mean, rstd=rstd, norm_weight=gamma, norm_bias=beta)
    y32 = pkg.layer_norm_linear(x, w, bias, mean=mean, rstd=rstd, norm_weight=gamma, norm_bias=beta,
                                out_dtype=torch.float32)
    torch.cuda.synchronize()
    xn, gn, bn, wn, biasn = (_np(t) for t in (x, gamma, beta, w, bias))
    # statistics: layer_norm_np's within fp32 summation-order differences
    _, m_ref, r_ref = orc.layer_norm_np(xn, gn, bn, 1e-5)
    np.testing.assert_allclose(_np(mean), m_ref, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(_np(rstd), r_ref, rtol=1e-5)
    # with the kernel's statistics the operand is exact: accumulation and output rounding only
    ref, a, absum = orc.layer_norm_linear_np(xn, gn, bn, 1e-5, wn, biasn, mean=_np(mean), rstd=_np(rstd))
    # fp32 accumulation: K additions, each within one fp32 ulp of its partial sum (2^-23 relative,
    # whatever rounding the matrix cores apply inside an instruction)
    acc_bound = cols * 2.0 ** -23 * absum
    assert np.all(np.abs(_np(y32) - ref) <= acc_bound * (1 + 2.0 ** -23) + np.abs(ref) * 2.0 ** -24 + 1e-30)
    assert np.all(np.abs(_np(y) - ref) <= acc_bound * (1 + 2.0 ** -8) + np.abs(ref) * 2.0 ** -8 + 1e-30)
    # the bf16 output is the fp32 output rounded once (same accumulation)
    assert np.array_equal(_np(y), orc.decode(orc.encode(_np(y32), "bf16"), "bf16"))
    # against the oracle's own statistics: one bf16 ulp per operand more
    ref2, _, absum2 = orc.layer_norm_linear_np(xn, gn, bn, 1e-5, wn, biasn)
    tol = np.abs(ref2) * 2.0 ** -8 + (2.0 ** -8 + cols * 2.0 ** -23) * absum2 + 1e-30
    assert np.all(np.abs(_np(y) - ref2) <= tol)
    # determinism
    y_again = pkg.layer_norm_linear(x, w, bias, mean=mean, rstd=rstd, norm_weight=gamma, norm_bias=beta)
    assert torch.equal(y.view(torch.int16), y_again.view(torch.int16))


def test_rep_encoder_forward_against_the_oracle_chain(pkg, dev):
    """RepEncoder.forward on a bf16 model, in both orders (pooling, the LayerNorm kernel and
    torch's Linear; pooling, statistics and the fused LayerNorm-Linear), against pool_c ->
    layer_norm_np -> bf16 -> Linear (float64)."""
    S, B, D, V, d_model = 28, 200, 128, 5000, 512
    torch.manual_seed(0)
    enc = pkg.RepEncoder(V, D, slot_num=S, d_model=d_model).to(dev).to(torch.bfloat16)
    with torch.no_grad():
        enc.emb.weight.normal_(0, 0.02)
        enc.input_norm.weight.normal_(1, 0.1)
        enc.input_norm.bias.normal_(0, 0.1)
    rng = np.random.default_rng(3)
    lens = rng.integers(0, 14, (S, B))
    ids = rng.integers(-2, V + 2, int(lens.sum()))
    ro = np.concatenate([np.concatenate([[0], np.cumsum(l)]) for l in lens]).astype(np.int64)
    vo = np.concatenate([[0], np.cumsum(lens.sum(axis=1))[:-1]]).astype(np.int64)
    batch = {"_flat_values": torch.from_numpy(ids).to(dev), "_flat_row_offsets": torch.from_numpy(ro).to(dev),
             "_val_offsets": torch.from_numpy(vo).to(dev)}
    wbits = enc.emb.weight.detach().cpu().view(torch.int16).numpy().view(np.uint16)
    pooled = orc.decode(orc.pool_c(ids, ro, [wbits] * S, "bf16", "sum", batch=B, val_base=vo), "bf16")
    ref, _, absum = orc.layer_norm_linear_np(pooled, _np(enc.input_norm.weight), _np(enc.input_norm.bias),
                                             enc.input_norm.eps, _np(enc.linear.weight), _np(enc.linear.bias))
    # one bf16 ulp per operand and of the output, plus fp32 accumulation over K
    tol = np.abs(ref) * 2.0 ** -8 + (2.0 ** -8 + S * D * 2.0 ** -23) * absum + 1e-30
    for fused_linear in (False, True):
        y = enc(batch, fused_linear=fused_linear)
        torch.cuda.synchronize()
        assert y.shape == (B, d_model) and y.dtype == torch.bfloat16
        assert np.all(np.abs(_np(y) - ref) <= tol), fused_linear
    enc.float()
    with pytest.raises(ValueError, match="fused_linear"):
        enc(batch, fused_linear=True)


@pytest.mark.parametrize("rows,cols,n", [(129, 14336, 96), (4096, 3584, 512), (700, 1792, 512), (129, 1792, 63)])
def test_split_k_against_the_unsplit_kernel(pkg, dev, rows, cols, n):
    """K split over workgroups (fp32 partials added in split order) against one pass over K: bit
    for bit on integer operands (every partial sum exact), within twice the fp32 accumulation
    bound on realistic ones; the workspace the library asks for is what the wrapper uses."""
    print(f"split-K rows={rows} cols={cols} n={n}", flush=True)
    assert pkg._capi.lib().cti_ebag_layernorm_linear_workspace_bytes(rows, cols, n) > 0
    rng = np.random.default_rng(rows)
    xi = rng.integers(-1, 2, (rows, cols)).astype(np.float32)
    wi = rng.integers(-1, 2, (n, cols)).astype(np.float32)
    a = pkg.layer_norm_linear(_bf16(xi, dev), _bf16(wi, dev), out_dtype=torch.float32)
    b = pkg.layer_norm_linear(_bf16(xi, dev), _bf16(wi, dev), out_dtype=torch.float32, split_k=False)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    x, gamma, beta, w, bias = _realistic(rows, cols, n, rows, dev)
    mean, rstd = pkg.layer_norm_stats(x, 1e-5)
    kw = dict(mean=mean, rstd=rstd, norm_weight=gamma, norm_bias=beta, out_dtype=torch.float32)
    ys = pkg.layer_norm_linear(x, w, bias, **kw)
    yu = pkg.layer_norm_linear(x, w, bias, split_k=False, **kw)
    torch.cuda.synchronize()
    _, a_op, absum = orc.layer_norm_linear_np(_np(x), _np(gamma), _np(beta), 1e-5, _np(w), _np(bias), mean=_np(mean),
                                              rstd=_np(rstd))
    bound = 2 * cols * 2.0 ** -23 * absum + 1e-30
    assert np.all(np.abs(_np(ys).astype(np.float64) - _np(yu)) <= bound)


def test_split_k_uses_as_many_splits_as_the_workspace_holds(pkg, dev):
    """The C ABI with workspaces smaller than the queried size: fewer splits (one split's worth or
    less: none), integer operands bit for bit against the unsplit call each time."""
    c = pkg._capi
    lib = c.lib()
    rows, cols, n = 300, 3584, 512
    full = lib.cti_ebag_layernorm_linear_workspace_bytes(rows, cols, n)
    one = rows * n * 4  # one split's partials
    assert full >= 4 * one
    rng = np.random.default_rng(7)
    x = _bf16(rng.integers(-1, 2, (rows, cols)).astype(np.float32), dev)
    w = _bf16(rng.integers(-1, 2, (n, cols)).astype(np.float32), dev)
    want = pkg.layer_norm_linear(x, w, out_dtype=torch.float32, split_k=False)
    stream = c.current_stream_handle(dev)
    for ws_bytes in (full, full // 2, 3 * one + 4096, 2 * one, one + 16, one, 16):
        print(f"workspace {ws_bytes} bytes", flush=True)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        y = torch.full((rows, n), float("nan"), dtype=torch.float32, device=dev)
        c.check(lib.cti_ebag_layernorm_linear(x.data_ptr(), rows, cols, None, None, None, None, c.F32, w.data_ptr(), n,
                                              None, c.F32, y.data_ptr(), c.F32, ws.data_ptr(), ws_bytes, stream))
        torch.cuda.synchronize()
        assert torch.equal(y, want), ws_bytes
