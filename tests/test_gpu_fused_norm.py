"""Pooling with the input LayerNorm fused into the writer, on the GPU.

Bar: the fused kernel's output equals LayerNorm(pooled row) where the pooled row is the oracle's
(bit-exact for bags pooled by one lane group, rounded to the table dtype) and the LayerNorm is
the oracle's fp32 restatement (online_best/infer.py:829-858): within 2e-5 absolute before the
final rounding (fp32 output) or half an output ulp plus 2e-5 (bf16 output). It also agrees with
running the pooling kernel and the LayerNorm kernel one after the other, and is deterministic.
"""
import numpy as np
import pytest
import torch

from oracle import ebag_oracle as orc

pytestmark = pytest.mark.gpu

TORCH_DT = {"f32": torch.float32, "bf16": torch.bfloat16}


def ref_layout(rng, S, B, V, max_len, long_every=0, long_len=0):
    L = rng.integers(0, max_len + 1, (S, B))
    L[:, rng.random(B) < 0.1] = 0
    if long_every:
        L[:, ::long_every] = long_len
    ro = np.zeros((S, B + 1), np.int64)
    np.cumsum(L, axis=1, out=ro[:, 1:])
    vo = np.concatenate([[0], np.cumsum(L.sum(axis=1))[:-1]]).astype(np.int64)
    v = rng.integers(-3, V + 3, int(L.sum())).astype(np.int64)
    return v, ro.reshape(-1), vo


def run_fused(pkg, dev, v, ro, vo, w, g, bb, B, pooling="sum", eps=1e-5):
    S = vo.size
    D = w.shape[1]
    out = torch.empty((B, S * D), dtype=w.dtype, device=dev)
    pkg.fused_all_slots_embedding_layernorm(torch.from_numpy(v).to(dev), torch.from_numpy(vo).to(dev),
                                            torch.from_numpy(ro).to(dev), w, out, B, D, w.shape[0] - 1, g, bb, eps,
                                            pooling=pooling)
    torch.cuda.synchronize()
    return out


def expected(v, ro, vo, w, g, bb, B, pooling, dt, eps=1e-5):
    """Oracle pooling (rounded to the table dtype) then the oracle LayerNorm, fp32."""
    S = vo.size
    wn = w.cpu()
    tab = wn.numpy() if dt == "f32" else wn.view(torch.int16).numpy().view(np.uint16)
    pooled = orc.pool_c(v, ro, [tab] * S, dt, pooling, dt, batch=B, val_base=vo)
    x = orc.decode(pooled, dt)
    y, _, _ = orc.layer_norm_np(x, g.float().cpu().numpy(), bb.float().cpu().numpy(), eps)
    return y


def check(out, y, dt):
    got = out.float().cpu().numpy()
    if dt == "f32":
        tol = 2e-5 + 1e-5 * np.abs(y)
    else:
        tol = 2e-5 + np.abs(y) * 2.0 ** -8
    assert (np.abs(got - y) <= tol).all(), np.abs(got - y).max()


@pytest.mark.parametrize("dt", ["bf16", "f32"])
@pytest.mark.parametrize("pdt", ["f32", "bf16"])
@pytest.mark.parametrize("D", [32, 64, 128, 256, 512])
@pytest.mark.parametrize("pooling", ["sum", "mean"])
def test_fused_matches_oracle(pkg, dev, dt, pdt, D, pooling):
    print(f"fused dt={dt} pdt={pdt} D={D} pooling={pooling}", flush=True)
    rng = np.random.default_rng(D + len(dt) * 7 + len(pdt) + len(pooling))
    S, B, V = 28 if D <= 128 else 12, 37, 700
    v, ro, vo = ref_layout(rng, S, B, V, 20)
    w = torch.from_numpy(rng.standard_normal((V, D)).astype(np.float32)).to(TORCH_DT[dt]).to(dev)
    g = torch.from_numpy((1 + 0.1 * rng.standard_normal(S * D)).astype(np.float32)).to(TORCH_DT[pdt]).to(dev)
    bb = torch.from_numpy((0.1 * rng.standard_normal(S * D)).astype(np.float32)).to(TORCH_DT[pdt]).to(dev)
    if dt == "f32" and D == 512 and pooling == "mean":
        # 2 KiB rows are outside the fused kernel and the unfused fallback pools by sum only
        with pytest.raises(pkg.EbagError, match="fused LayerNorm"):
            run_fused(pkg, dev, v, ro, vo, w, g, bb, B, pooling)
        return
    out = run_fused(pkg, dev, v, ro, vo, w, g, bb, B, pooling)
    check(out, expected(v, ro, vo, w, g, bb, B, pooling, dt), dt)


@pytest.mark.parametrize("S", [1, 5, 64])
@pytest.mark.parametrize("B", [1, 2, 3])
def test_fused_slot_counts_and_small_batches(pkg, dev, S, B):
    """Workgroups pool two samples when the slots allow it; odd batches leave the last one half
    full, and 64 slots (16 bags per wavefront per sample) is the largest fused shape."""
    print(f"fused S={S} B={B}", flush=True)
    rng = np.random.default_rng(S * 10 + B)
    V, D = 400, 32
    v, ro, vo = ref_layout(rng, S, B, V, 24, long_every=2, long_len=70)
    # integer rows: the split sums of the 70-id bags are exact, so the pooled rows equal the oracle's
    w = torch.from_numpy(rng.integers(-8, 9, (V, D)).astype(np.float32)).to(torch.bfloat16).to(dev)
    g = torch.from_numpy((1 + 0.1 * rng.standard_normal(S * D)).astype(np.float32)).to(dev)
    bb = torch.from_numpy((0.1 * rng.standard_normal(S * D)).astype(np.float32)).to(dev)
    for pooling in ("sum", "mean"):
        out = run_fused(pkg, dev, v, ro, vo, w, g, bb, B, pooling)
        check(out, expected(v, ro, vo, w, g, bb, B, pooling, "bf16"), "bf16")


def test_fused_long_bags_and_int32_inputs(pkg, dev):
    """Bags longer than the short-bag limit are pooled by the whole wavefront (split sums: the
    pooled row is within the reassociation bound, the LayerNorm tolerance covers it)."""
    rng = np.random.default_rng(5)
    S, B, V, D = 28, 20, 900, 128
    v, ro, vo = ref_layout(rng, S, B, V, 30, long_every=3, long_len=300)
    w = torch.from_numpy((rng.integers(-8, 9, (V, D))).astype(np.float32)).to(torch.bfloat16).to(dev)  # exact sums
    g = torch.ones(S * D, dtype=torch.float32, device=dev)
    bb = torch.zeros(S * D, dtype=torch.float32, device=dev)
    a = run_fused(pkg, dev, v, ro, vo, w, g, bb, B)
    check(a, expected(v, ro, vo, w, g, bb, B, "sum", "bf16"), "bf16")
    b = run_fused(pkg, dev, v.astype(np.int32), ro.astype(np.int32), vo.astype(np.int32), w, g, bb, B)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_fused_agrees_with_separate_kernels_and_is_deterministic(pkg, dev):
    rng = np.random.default_rng(9)
    S, B, V, D = 28, 300, 5000, 128
    v, ro, vo = ref_layout(rng, S, B, V, 16)
    w = torch.from_numpy((0.01 * rng.standard_normal((V, D))).astype(np.float32)).to(torch.bfloat16).to(dev)
    g = torch.from_numpy((1 + 0.1 * rng.standard_normal(S * D)).astype(np.float32)).to(torch.bfloat16).to(dev)
    bb = torch.from_numpy((0.1 * rng.standard_normal(S * D)).astype(np.float32)).to(torch.bfloat16).to(dev)
    fused = run_fused(pkg, dev, v, ro, vo, w, g, bb, B)
    again = run_fused(pkg, dev, v, ro, vo, w, g, bb, B)
    assert torch.equal(fused.view(torch.int16), again.view(torch.int16))
    pooled = torch.empty((B, S * D), dtype=torch.bfloat16, device=dev)
    pkg.fused_all_slots_embedding(torch.from_numpy(v).to(dev), torch.from_numpy(vo).to(dev),
                                  torch.from_numpy(ro).to(dev), w, pooled, B, D, V - 1)
    sep = pkg.layer_norm(pooled, g, bb, 1e-5)
    torch.cuda.synchronize()
    # the pooled rows are the same bits; the two LayerNorms reduce in different orders, so their
    # fp32 results differ in the last bits and a bf16 rounding may land one ulp apart
    # (one ulp <= 2^-7 of the value)
    diff = (fused.float() - sep.float()).abs()
    big = torch.maximum(fused.float().abs(), sep.float().abs())
    assert (diff <= big * 2.0 ** -7 + 1e-5).all(), (diff - big * 2.0 ** -7).max().item()
    assert (diff == 0).float().mean().item() > 0.95


def test_unfused_shapes_fall_back(pkg, dev):
    """16-byte rows (bf16 D=8) are outside the fused kernel: the wrapper runs the pooling and
    LayerNorm kernels instead and the result is the same within the LayerNorm tolerance."""
    rng = np.random.default_rng(3)
    S, B, V, D = 28, 25, 300, 8
    v, ro, vo = ref_layout(rng, S, B, V, 10)
    w = torch.from_numpy(rng.standard_normal((V, D)).astype(np.float32)).to(torch.bfloat16).to(dev)
    g = torch.ones(S * D, device=dev)
    bb = torch.zeros(S * D, device=dev)
    out = run_fused(pkg, dev, v, ro, vo, w, g, bb, B)
    check(out, expected(v, ro, vo, w, g, bb, B, "sum", "bf16"), "bf16")
    with pytest.raises(pkg.EbagError, match="fused LayerNorm"):
        run_fused(pkg, dev, v, ro, vo, w, g, bb, B, pooling="mean")


def test_encoder_normalized_uses_fused_path(pkg, dev):
    torch.manual_seed(0)
    S, D = 28, 128
    enc = pkg.RepEncoder(vocab_size=4000, emb_dim=D, padding_idx=0, slot_num=S, d_model=32).to(dev).to(torch.bfloat16)
    with torch.no_grad():
        enc.input_norm.weight.copy_(1 + 0.1 * torch.randn(S * D))
        enc.input_norm.bias.copy_(0.1 * torch.randn(S * D))
    rng = np.random.default_rng(1)
    B = 64
    v, ro, vo = ref_layout(rng, S, B, 4000, 12)
    batch = {"_flat_values": torch.from_numpy(v).to(dev), "_flat_row_offsets": torch.from_numpy(ro).to(dev),
             "_val_offsets": torch.from_numpy(vo).to(dev)}
    y = enc.normalized(batch)
    torch.cuda.synchronize()
    check(y, expected(v, ro, vo, enc.emb.weight.detach(), enc.input_norm.weight.detach(),
                      enc.input_norm.bias.detach(), B, "sum", "bf16"), "bf16")
