"""The input LayerNorm (cti_ebag_layernorm) on the GPU against a torch fp32 LayerNorm of the same
rows and against the oracle's restatement of online_best/infer.py:829-858.

Bar (floating point): fp32 output within 1e-4 (absolute and relative) of the fp64 LayerNorm of
the decoded input; bf16 / fp16 output within one rounding of the output type (2^-7 / 2^-10
relative) plus 1e-4; per-row mean and rstd within 1e-5 relative. Constant rows of exactly
representable values give mean == value and y == beta exactly (every deviation is 0).
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as Fn

from oracle import ebag_oracle as orc

pytestmark = pytest.mark.gpu

TORCH_DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
RND = {"f32": 0.0, "bf16": 2.0 ** -7, "f16": 2.0 ** -10}


def _inputs(seed, rows, cols, dt, pdt, dev, offset=0.5, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(rows, cols, generator=g) * scale + offset).to(TORCH_DT[dt])
    w = (1 + 0.2 * torch.randn(cols, generator=g)).to(TORCH_DT[pdt])
    b = (0.3 * torch.randn(cols, generator=g)).to(TORCH_DT[pdt])
    return x.to(dev), w.to(dev), b.to(dev)


def _check(got, x, w, b, eps, dt):
    ref = Fn.layer_norm(x.double().cpu(), (x.shape[1],), w.double().cpu(), b.double().cpu(), eps)
    err = (got.double().cpu() - ref).abs()
    tol = 1e-4 + (RND[dt] + 1e-4) * ref.abs()
    assert bool((err <= tol).all()), f"max err {err.max().item():.3e}"


@pytest.mark.parametrize("cols", [7, 100, 448, 2048, 3584, 14336, 16392])
@pytest.mark.parametrize("dt,pdt", [("f32", "f32"), ("f32", "bf16"), ("bf16", "f32"), ("bf16", "bf16"), ("f16", "f32")])
def test_layer_norm_matches_torch(pkg, dev, cols, dt, pdt):
    x, w, b = _inputs(cols, 33, cols, dt, pdt, dev)
    mean = torch.empty(33, dtype=torch.float32, device=dev)
    rstd = torch.empty(33, dtype=torch.float32, device=dev)
    y = pkg.layer_norm(x, w, b, 1e-5, mean=mean, rstd=rstd)
    torch.cuda.synchronize()
    _check(y, x, w, b, 1e-5, dt)
    xr = x.float().cpu().numpy()
    _, m_ref, r_ref = orc.layer_norm_np(xr, w.float().cpu().numpy(), b.float().cpu().numpy(), 1e-5)
    np.testing.assert_allclose(mean.cpu().numpy(), m_ref, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(rstd.cpu().numpy(), r_ref, rtol=1e-5)


def test_layer_norm_encoder_shape(pkg, dev):
    # the pooled block of the bf16-2m configuration: 4096 rows of 28 * 128 bf16 columns
    x, w, b = _inputs(7, 4096, 3584, "bf16", "f32", dev, offset=0.0, scale=0.05)
    y = pkg.layer_norm(x, w, b, 1e-5)
    torch.cuda.synchronize()
    _check(y, x, w, b, 1e-5, "bf16")
    y2 = pkg.layer_norm(x, w, b, 1e-5)
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))  # deterministic


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_layer_norm_constant_rows_are_exact(pkg, dev, dt):
    cols = 3584
    vals = torch.tensor([1.0, -3.5, 0.0, 1024.0, 0.25])
    x = vals[:, None].repeat(1, cols).to(TORCH_DT[dt]).to(dev)
    w = torch.linspace(0.5, 2.0, cols).to(dev)
    b = torch.linspace(-1.0, 1.0, cols).to(dev)
    mean = torch.empty(len(vals), dtype=torch.float32, device=dev)
    y = pkg.layer_norm(x, w, b, 1e-5, mean=mean)
    torch.cuda.synchronize()
    assert torch.equal(mean.cpu(), vals)
    assert torch.equal(y.cpu(), b.to(TORCH_DT[dt]).cpu()[None, :].expand(len(vals), cols))


def test_layer_norm_in_place(pkg, dev):
    x, w, b = _inputs(3, 64, 3584, "bf16", "bf16", dev)
    want = pkg.layer_norm(x, w, b, 1e-5)
    out = pkg.layer_norm(x, w, b, 1e-5, out=x)
    torch.cuda.synchronize()
    assert out.data_ptr() == x.data_ptr()
    assert torch.equal(x.view(torch.int16), want.view(torch.int16))


def test_layer_norm_rejects_bad_arguments(pkg, dev):
    x, w, b = _inputs(1, 4, 64, "f32", "f32", dev)
    with pytest.raises(ValueError):
        pkg.layer_norm(x, w[:63], b, 1e-5)
    with pytest.raises(ValueError):
        pkg.layer_norm(x[:, :32].t(), w[:4], b[:4], 1e-5)  # not contiguous
    with pytest.raises(TypeError):
        pkg.layer_norm(x, w, b.to(torch.bfloat16), 1e-5)
    c = pkg._capi
    assert c.lib().cti_ebag_layernorm(x.data_ptr(), x.data_ptr(), 4, 0, c.F32, w.data_ptr(), b.data_ptr(), c.F32,
                                      1e-5, None, None, None) == c.EINVAL
    assert "cols" in c.last_error()
