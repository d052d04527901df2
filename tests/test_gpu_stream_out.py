"""Output blocks of 128 MiB and more are stored non-temporally (a launch-wide flag the host sets
from the block's size); smaller ones take plain stores. Every kernel form's large-block launch is
checked here: pooled blocks bit for bit against the oracle (short bags, or integer tables where
bags are split), the LayerNorm and the fused pooling + LayerNorm bit for bit against the same rows
computed in launches whose blocks are below the threshold.
"""
import numpy as np
import pytest
import torch

from _cases import make_ids, make_table
from oracle import ebag_oracle as orc

pytestmark = pytest.mark.gpu

STREAM_OUT_BYTES = 128 << 20
TORCH_DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
OUT_BYTES = {"f32": 4, "bf16": 2, "f16": 2}


def to_dev(arr, tdt, dev):
    t = torch.from_numpy(np.ascontiguousarray(arr))
    if tdt != "f32":
        t = t.view(torch.int16).view(TORCH_DT[tdt])
    return t.to(dev)


def to_np(t, odt):
    t = t.cpu()
    return t.numpy() if odt == "f32" else t.view(torch.int16).numpy().view(np.uint16)


# (table dtype, width, fields, output dtype, table values, binning): 256-byte rows take the
# streamed tiles, 128-byte rows the ranked tiles, 33 columns the generic kernel, and the binned
# launch the list kernels (bags of 100 rows on one wavefront, 400 rows split over a workgroup).
CASES = [
    ("bf16", 128, 4, "f32", "normal", False),
    ("bf16", 128, 8, "bf16", "normal", False),
    ("f32", 64, 8, "f16", "normal", False),
    ("bf16", 64, 16, "bf16", "normal", False),
    ("f32", 33, 16, "f32", "normal", False),
    ("bf16", 128, 8, "bf16", "int", True),
]


@pytest.mark.parametrize("tdt,D,F,odt,kind,bins", CASES)
def test_large_pooled_block_matches_oracle(pkg, dev, tdt, D, F, odt, kind, bins):
    rng = np.random.default_rng(D + F)
    B = -(-STREAM_OUT_BYTES // (F * D * OUT_BYTES[odt])) + 64  # just above the threshold
    print(f"large block {tdt} D={D} F={F} out={odt} bins={bins} B={B}", flush=True)
    V = 1500
    L = rng.integers(0, 7, size=(F, B))
    if bins:
        L[:, ::97] = 100
        L[:, 5::1009] = 400
    ids = make_ids(rng, int(L.sum()), V)
    offsets = np.concatenate([[0], np.cumsum(L.reshape(-1))]).astype(np.int64)
    tables = [make_table(rng, V, D, tdt, kind) for _ in range(F)]
    kw = dict(use_bins=True, block_threshold=32, split_threshold=192) if bins else {}
    out = pkg.embedding_bag_pooled(torch.from_numpy(ids).to(dev), torch.from_numpy(offsets).to(dev),
                                   [to_dev(t, tdt, dev) for t in tables], pooling="sum",
                                   out_dtype=TORCH_DT[odt], **kw)
    torch.cuda.synchronize()
    assert out.numel() * out.element_size() >= STREAM_OUT_BYTES
    want = orc.pool_c(ids, offsets, tables, tdt, "sum", odt)
    assert np.array_equal(to_np(out, odt), want)


def test_large_layernorm_block_matches_smaller_launches(pkg, dev):
    rows, cols = 70_000, 1024
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    x = torch.randn((rows, cols), generator=g, device=dev).to(torch.bfloat16)
    gamma = torch.randn(cols, generator=g, device=dev).to(torch.bfloat16)
    beta = torch.randn(cols, generator=g, device=dev).to(torch.bfloat16)
    assert x.numel() * 2 >= STREAM_OUT_BYTES
    full = pkg.layer_norm(x, gamma, beta, 1e-5)
    half = rows // 2
    parts = torch.cat([pkg.layer_norm(x[:half].contiguous(), gamma, beta, 1e-5),
                       pkg.layer_norm(x[half:].contiguous(), gamma, beta, 1e-5)])
    torch.cuda.synchronize()
    assert torch.equal(full.view(torch.int16), parts.view(torch.int16))


def test_large_fused_block_matches_a_smaller_launch(pkg, dev):
    """The reference layout's fused pooling + LayerNorm over 28 slots: a batch whose normalised
    block passes the threshold, against the first samples of it in a launch below it (slot-local
    row offsets of a batch's first samples are a prefix of each slot's offsets)."""
    rng = np.random.default_rng(12)
    S, D, V = 28, 128, 3000
    B = -(-STREAM_OUT_BYTES // (S * D * 2)) + 64
    Bp = 8000
    L = rng.integers(0, 9, (S, B))
    ro = np.zeros((S, B + 1), np.int64)
    np.cumsum(L, axis=1, out=ro[:, 1:])
    vo = np.concatenate([[0], np.cumsum(L.sum(axis=1))[:-1]]).astype(np.int64)
    v = rng.integers(0, V, int(L.sum())).astype(np.int64)
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    w = (torch.randn((V, D), generator=g, device=dev) * 0.1).to(torch.bfloat16)
    gamma = torch.randn(S * D, generator=g, device=dev).to(torch.bfloat16)
    beta = torch.randn(S * D, generator=g, device=dev).to(torch.bfloat16)
    dv, dvo = torch.from_numpy(v).to(dev), torch.from_numpy(vo).to(dev)

    def fused(row_offsets, batch):
        out = torch.empty((batch, S * D), dtype=torch.bfloat16, device=dev)
        pkg.fused_all_slots_embedding_layernorm(dv, dvo, torch.from_numpy(np.ascontiguousarray(row_offsets)).to(dev),
                                                w, out, batch, D, V - 1, gamma, beta, 1e-5)
        return out

    full = fused(ro.reshape(-1), B)
    assert full.numel() * 2 >= STREAM_OUT_BYTES
    part = fused(ro[:, :Bp + 1].reshape(-1), Bp)
    torch.cuda.synchronize()
    assert torch.equal(full[:Bp].view(torch.int16), part.view(torch.int16))
