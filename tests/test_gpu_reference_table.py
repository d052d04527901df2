"""The drop-in entry points on the reference's own table shape: one shared nn.Embedding of
5,000,000 x 512 bf16 rows (online_best/infer.py:948, 5.12 GB), 28 slots (online_best/infer.py:
1050-1059 launch, kernel :805-827; input LayerNorm :1061-1076).

At 1 KiB per row the table spans more than 4 GiB, so the kernels address rows with 64-bit
offsets instead of buffer loads; ids are drawn over the whole table and some are forced into
the rows above the 4 GiB mark and onto the clamp bounds. The oracle pools a compact copy of the
rows the batch touches (gathered on the device), with the ids renumbered to it. Bags are kept
to at most 48 rows so that each is pooled by one lane group in element order: the pooled block
must equal the oracle bit for bit, and the fused LayerNorm must match the oracle's LayerNorm of
it within the LayerNorm tolerance.
"""
import numpy as np
import pytest
import torch

from oracle import ebag_oracle as orc

pytestmark = pytest.mark.gpu

V, D, S, B = 5_000_000, 512, 28, 96


@pytest.fixture(scope="module")
def weight(dev):
    w = torch.empty((V, D), dtype=torch.bfloat16, device=dev)
    w.normal_(0.0, 0.01, generator=torch.Generator(device=dev).manual_seed(11))
    yield w
    del w
    torch.cuda.empty_cache()


def _batch(seed):
    rng = np.random.default_rng(seed)
    lens = np.clip(rng.geometric(1 / 9, (S, B)) - 1, 0, 48)
    ids = rng.integers(0, V, int(lens.sum())).astype(np.int64)
    high = rng.random(ids.size) < 0.2
    ids[high] = rng.integers((1 << 32) // (D * 2), V, int(high.sum()))  # rows past the 4 GiB mark
    for k, v in enumerate((-1, V - 1, V, V + 12345, 2 ** 40)):             # clamp bounds
        if ids.size > k:
            ids[k * 7 % ids.size] = v
    row_offsets = np.concatenate([np.concatenate([[0], np.cumsum(l)]) for l in lens]).astype(np.int64)
    val_offsets = np.concatenate([[0], np.cumsum(lens.sum(axis=1))[:-1]]).astype(np.int64)
    return ids, row_offsets, val_offsets


def _oracle_pooled(weight, ids, row_offsets, val_offsets):
    rows = np.clip(ids, 0, V - 1)
    uniq, compact = np.unique(rows, return_inverse=True)
    sub = weight.index_select(0, torch.from_numpy(uniq).to(weight.device)).cpu()
    sub_bits = sub.view(torch.int16).numpy().view(np.uint16)
    return orc.pool_c(compact.astype(np.int64), row_offsets, [sub_bits] * S, "bf16", "sum", batch=B,
                      val_base=val_offsets)


def test_reference_table_pooling_bitwise(pkg, dev, weight):
    ids, ro, vo = _batch(31)
    want = _oracle_pooled(weight, ids, ro, vo)
    out = torch.empty((B, S * D), dtype=torch.bfloat16, device=dev)
    pkg.fused_all_slots_embedding(torch.from_numpy(ids).to(dev), torch.from_numpy(vo).to(dev),
                                  torch.from_numpy(ro).to(dev), weight, out, B, D, V - 1)
    torch.cuda.synchronize()
    got = out.cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


def test_reference_table_fused_layernorm(pkg, dev, weight):
    ids, ro, vo = _batch(32)
    pooled = orc.decode(_oracle_pooled(weight, ids, ro, vo), "bf16")
    g = torch.Generator().manual_seed(5)
    gamma = (1 + 0.1 * torch.randn(S * D, generator=g)).to(dev)
    beta = (0.1 * torch.randn(S * D, generator=g)).to(dev)
    out = torch.empty((B, S * D), dtype=torch.bfloat16, device=dev)
    pkg.fused_all_slots_embedding_layernorm(torch.from_numpy(ids).to(dev), torch.from_numpy(vo).to(dev),
                                            torch.from_numpy(ro).to(dev), weight, out, B, D, V - 1, gamma, beta,
                                            1e-5)
    torch.cuda.synchronize()
    y, _, _ = orc.layer_norm_np(pooled, gamma.cpu().numpy(), beta.cpu().numpy(), 1e-5)
    err = np.abs(out.float().cpu().numpy() - y)
    assert (err <= 2e-5 + np.abs(y) * 2.0 ** -8).all(), err.max()  # half a bf16 ulp of the output
