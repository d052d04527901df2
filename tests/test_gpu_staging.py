"""int32 inputs and the host -> device staging path on the GPU.

Bar: the pooled output from int32 ids / offsets, and from batches moved by InputStager (pinned,
int32-compacted, double-buffered), equals the oracle's pooling of the host batch bit for bit
(bags of at most 12 rows: one lane group each, element order), including ids outside the int32
range (saturated on the host, clamped on the device), and equals the int64 path's.
"""
import numpy as np
import pytest
import torch

from oracle import ebag_oracle as orc

pytestmark = pytest.mark.gpu

S, V, D = 28, 3000, 128


def host_batch(rng, B, max_len=12, wide_ids=True):
    L = rng.integers(0, max_len + 1, (S, B))
    L[:, min(1, B - 1)] = 0
    ro = np.zeros((S, B + 1), np.int64)
    np.cumsum(L, axis=1, out=ro[:, 1:])
    vo = np.concatenate([[0], np.cumsum(L.sum(axis=1))[:-1]]).astype(np.int64)
    v = rng.integers(0, V, int(L.sum())).astype(np.int64)
    if wide_ids and v.size >= 6:
        v[:6] = [2 ** 31, -(2 ** 31) - 5, np.iinfo(np.int64).max, np.iinfo(np.int64).min, 2 ** 40 + 3, -1]
    return {"_flat_values": torch.from_numpy(v), "_flat_row_offsets": torch.from_numpy(ro.reshape(-1)),
            "_val_offsets": torch.from_numpy(vo)}, B


def oracle_pool(hb, weight, B):
    """The oracle's pooling of a host batch (int64 ids as the collate leaves them) as bf16 bits."""
    wbits = weight.cpu().view(torch.int16).numpy().view(np.uint16)
    return orc.pool_c(hb["_flat_values"].numpy(), hb["_flat_row_offsets"].numpy(), [wbits] * S, "bf16", "sum",
                      batch=B, val_base=hb["_val_offsets"].numpy())


def pool(pkg, dev_batch, weight, B):
    out = torch.empty((B, S * D), dtype=weight.dtype, device=weight.device)
    return pkg.fused_all_slots_embedding(dev_batch["_flat_values"], dev_batch["_val_offsets"],
                                         dev_batch["_flat_row_offsets"], weight, out, B, D, V - 1)


def weight_of(dev):
    g = torch.Generator(device="cpu").manual_seed(1)
    return torch.randn(V, D, generator=g).to(torch.bfloat16).to(dev)


@pytest.fixture(scope="module")
def weight(dev):
    return weight_of(dev)


@pytest.mark.parametrize("vt,ot", [(torch.int32, torch.int32), (torch.int32, torch.int64), (torch.int64, torch.int32)])
def test_int32_layouts_match_int64(pkg, dev, weight, vt, ot):
    rng = np.random.default_rng(3)
    hb, B = host_batch(rng, 77, wide_ids=False)
    ref = pool(pkg, {k: t.to(dev) for k, t in hb.items()}, weight, B)
    narrow = {"_flat_values": hb["_flat_values"].to(vt).to(dev), "_flat_row_offsets": hb["_flat_row_offsets"].to(ot).to(dev),
              "_val_offsets": hb["_val_offsets"].to(ot).to(dev)}
    got = pool(pkg, narrow, weight, B)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    assert np.array_equal(got.cpu().view(torch.int16).numpy().view(np.uint16), oracle_pool(hb, weight, B))


def test_int32_mixed_offset_types_and_int8(pkg, dev, weight):
    rng = np.random.default_rng(4)
    hb, B = host_batch(rng, 50, wide_ids=False)
    q, s = pkg.quantize_embedding_int8(weight)
    outs = []
    for vt, rt, bt in ((torch.int64, torch.int64, torch.int64), (torch.int32, torch.int32, torch.int64)):
        out = torch.empty((B, S * D), dtype=torch.bfloat16, device=dev)
        pkg.fused_all_slots_embedding_int8(hb["_flat_values"].to(vt).to(dev), hb["_val_offsets"].to(bt).to(dev),
                                           hb["_flat_row_offsets"].to(rt).to(dev), q, s, out, B, D, V - 1)
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))


@pytest.mark.parametrize("compact", [True, False])
@pytest.mark.parametrize("depth", [1, 2, 3])
def test_stager_pipeline_matches_direct_transfer(pkg, dev, weight, compact, depth):
    print(f"stager compact={compact} depth={depth}", flush=True)
    rng = np.random.default_rng(depth * 2 + compact)
    batches = [host_batch(rng, int(rng.integers(1, 200))) for _ in range(7)]
    max_nnz = max(b["_flat_values"].numel() for b, _ in batches)
    stager = pkg.InputStager(max_nnz, S, 200, dev, depth=depth, compact=compact)
    got = []
    for hb, B in batches:
        staged = pkg.move_model_inputs_to_device(hb, dev, S, stager=stager)
        if compact:
            assert staged["_flat_values"].dtype == torch.int32
        got.append(pool(pkg, staged, weight, B).clone())
        stager.release(staged)
    torch.cuda.synchronize()
    for (hb, B), g in zip(batches, got):
        assert np.array_equal(g.cpu().view(torch.int16).numpy().view(np.uint16), oracle_pool(hb, weight, B))
        ref = pool(pkg, pkg.move_model_inputs_to_device(hb, dev, S), weight, B)
        torch.cuda.synchronize()
        assert torch.equal(g.view(torch.int16), ref.view(torch.int16))


def test_stager_requires_release(pkg, dev, weight):
    rng = np.random.default_rng(9)
    hb, B = host_batch(rng, 10)
    stager = pkg.InputStager(hb["_flat_values"].numel(), S, 10, dev, depth=2)
    a = stager.stage(hb)
    b = stager.stage(hb)
    with pytest.raises(RuntimeError, match="release"):
        stager.stage(hb)
    pool(pkg, a, weight, B)
    stager.release(a)
    c = stager.stage(hb)
    pool(pkg, b, weight, B)
    pool(pkg, c, weight, B)
    stager.release(b)
    stager.release(c)
    torch.cuda.synchronize()
    with pytest.raises(ValueError, match="holds"):
        big = dict(hb)
        big["_flat_values"] = torch.zeros(hb["_flat_values"].numel() + 1, dtype=torch.int64)
        stager.stage(big)


def test_per_slot_pairs_are_packed_on_device(pkg, dev, weight):
    rng = np.random.default_rng(11)
    hb, B = host_batch(rng, 30, wide_ids=False)
    v, ro, vo = hb["_flat_values"].numpy(), hb["_flat_row_offsets"].numpy().reshape(S, B + 1), hb["_val_offsets"].numpy()
    pairs = {}
    for s in range(S):
        end = vo[s + 1] if s + 1 < S else v.size
        pairs[s + 1] = (torch.from_numpy(v[vo[s]:end].copy()), torch.from_numpy(ro[s].copy()))
    moved = pkg.move_model_inputs_to_device(pairs, dev, S)
    for k in ("_flat_values", "_flat_row_offsets", "_val_offsets"):
        assert torch.equal(moved[k].cpu(), hb[k])


def test_attention_keys_pass_through_as_the_reference_moves_them(pkg, dev):
    """online_best/infer.py:762-778: ``_attn_groups`` is moved (its tensors to the device, the
    rest unchanged); ``user_offsets`` is moved only when there are no ``_attn_groups``; the
    batch's other keys (label, logid, pred_mask, ...) are not part of the model batch."""
    rng = np.random.default_rng(12)
    hb, B = host_batch(rng, 9, wide_ids=False)
    hb = dict(hb)
    hb["user_offsets"] = torch.arange(4)
    hb["label"] = torch.zeros(B)
    hb["logid"] = ["a"] * B
    for with_groups in (True, False):
        batch = dict(hb)
        if with_groups:
            batch["_attn_groups"] = [{"rows": torch.arange(3), "num_users": 2, "identity": True}]
        for stager in (None, pkg.InputStager(hb["_flat_values"].numel(), S, B, dev)):
            moved = pkg.move_model_inputs_to_device(batch, dev, S, stager=stager)
            assert "label" not in moved and "logid" not in moved
            if with_groups:
                assert "user_offsets" not in moved
                grp = moved["_attn_groups"][0]
                assert grp["rows"].device.type == "cuda" and grp["num_users"] == 2 and grp["identity"] is True
            else:
                assert "_attn_groups" not in moved
                assert moved["user_offsets"].device.type == "cuda"
                assert torch.equal(moved["user_offsets"].cpu(), torch.arange(4))
            got = pool(pkg, moved, weight_of(dev), B)
            torch.cuda.synchronize()
            assert np.array_equal(got.cpu().view(torch.int16).numpy().view(np.uint16),
                                  oracle_pool(hb, weight_of(dev), B))
            if stager is not None:
                stager.release(moved)
