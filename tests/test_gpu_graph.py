"""Pooling calls captured in a HIP graph (a serving loop replays one captured step per batch).

The entry points launch their kernels on the caller's stream, allocate nothing and never wait on
the host, and the binning pass leaves its list counters at zero by itself (no memset node), so a
call can be captured once and replayed on new inputs written into the same buffers. Each replay
must equal the eager call on the same inputs bit for bit (same kernels, same order). Inputs change
between replays (with eager copies and host synchronisation in between); their sizes stay those
of the capture, since sizes are baked into the captured launches.
"""
import numpy as np
import pytest
import torch

from _cases import make_ids, make_table
from test_gpu_parity import to_dev

pytestmark = pytest.mark.gpu


def _length_sets(seed, F, B, n_sets, max_len, long_every, long_len):
    """n_sets length matrices [F, B] with the same per-field totals (bags permuted within a field)."""
    rng = np.random.default_rng(seed)
    L0 = rng.integers(0, max_len + 1, size=(F, B))
    L0[:, ::long_every] = long_len
    return [np.stack([rng.permutation(L0[f]) for f in range(F)]) for _ in range(n_sets)], rng


def _capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def test_binned_mixed_width_call_replays(pkg, dev):
    F, B = 9, 150
    dims = [(32, 64, 128)[f % 3] for f in range(F)]
    vocab = [300 + 97 * f for f in range(F)]
    sets, rng = _length_sets(11, F, B, 4, max_len=30, long_every=13, long_len=400)
    tables = [to_dev(make_table(rng, vocab[f], dims[f], "bf16"), "bf16", dev) for f in range(F)]
    plan = pkg.PooledEmbedding(tables, pooling="mean", use_bins=True, block_threshold=24, split_threshold=120,
                               max_batch=B)
    inputs = []
    for L in sets:
        ids = np.concatenate([make_ids(rng, int(L[f].sum()), vocab[f]) for f in range(F)])
        off = np.zeros(F * B + 1, np.int64)
        np.cumsum(L.reshape(-1), out=off[1:])
        inputs.append((torch.from_numpy(ids).to(dev), torch.from_numpy(off).to(dev)))
    v, o = inputs[0][0].clone(), inputs[0][1].clone()
    out = torch.empty((B, sum(dims)), dtype=torch.bfloat16, device=dev)
    g = _capture(lambda: plan(v, o, out))
    for rep in range(2):
        for vi, oi in inputs:
            want = plan(vi, oi).clone()  # eager, fresh output
            torch.cuda.synchronize()
            v.copy_(vi)
            o.copy_(oi)
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out.view(torch.int16), want.view(torch.int16)), rep
    # the list counters (bytes 0-3 and 8-11) are back at zero after the replays
    assert torch.count_nonzero(plan._ws[0:4]).item() == 0 and torch.count_nonzero(plan._ws[8:12]).item() == 0


def test_reference_layout_and_fused_layernorm_replay(pkg, dev):
    S, B, D, V = 28, 64, 128, 4000
    sets, rng = _length_sets(12, S, B, 3, max_len=14, long_every=17, long_len=70)
    weight = to_dev(make_table(rng, V, D, "bf16"), "bf16", dev)
    gamma = (1 + 0.1 * torch.randn(S * D, generator=torch.Generator().manual_seed(5))).to(dev)
    beta = (0.1 * torch.randn(S * D, generator=torch.Generator().manual_seed(6))).to(dev)
    inputs = []
    for L in sets:
        ids = make_ids(rng, int(L.sum()), V)
        ro = np.concatenate([np.concatenate([[0], np.cumsum(L[s])]) for s in range(S)]).astype(np.int64)
        vo = np.concatenate([[0], np.cumsum(L.sum(axis=1))[:-1]]).astype(np.int64)
        inputs.append(tuple(torch.from_numpy(a).to(dev) for a in (ids, vo, ro)))
    v, vo, ro = (t.clone() for t in inputs[0])
    pooled = torch.empty((B, S * D), dtype=torch.bfloat16, device=dev)
    normed = torch.empty_like(pooled)

    def step(v_, vo_, ro_, pooled_, normed_):
        pkg.fused_all_slots_embedding(v_, vo_, ro_, weight, pooled_, B, D, V - 1)
        pkg.fused_all_slots_embedding_layernorm(v_, vo_, ro_, weight, normed_, B, D, V - 1, gamma, beta, 1e-5)

    g = _capture(lambda: step(v, vo, ro, pooled, normed))
    for rep in range(2):
        for vi, voi, roi in inputs:
            want_p, want_n = torch.empty_like(pooled), torch.empty_like(normed)
            step(vi, voi, roi, want_p, want_n)
            torch.cuda.synchronize()
            v.copy_(vi)
            vo.copy_(voi)
            ro.copy_(roi)
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(pooled.view(torch.int16), want_p.view(torch.int16)), rep
            assert torch.equal(normed.view(torch.int16), want_n.view(torch.int16)), rep


@pytest.mark.parametrize("rows,cols,n", [(96, 3584, 512), (4096, 3584, 512), (300, 136, 64)])
def test_layernorm_linear_replays(pkg, dev, rows, cols, n):
    """Statistics pass + LayerNorm-Linear captured together: K split over workgroups (workspace from
    the graph's pool, a GEMM and a reduction launch per call; 96 and 4096 rows), one launch
    without a split (the general form, K not a multiple of 128). Every replay on new inputs
    equals the eager call bit for bit."""
    print(f"layernorm-linear replay rows={rows} cols={cols} n={n}", flush=True)
    gen = torch.Generator().manual_seed(rows + cols)
    xs = [(0.02 * torch.randn(rows, cols, generator=gen) + 0.01 * k).to(torch.bfloat16).to(dev) for k in range(3)]
    gamma = (1 + 0.1 * torch.randn(cols, generator=gen)).to(torch.bfloat16).to(dev)
    beta = (0.1 * torch.randn(cols, generator=gen)).to(torch.bfloat16).to(dev)
    w = (torch.randn(n, cols, generator=gen) / cols ** 0.5).to(torch.bfloat16).to(dev)
    bias = (0.1 * torch.randn(n, generator=gen)).to(torch.bfloat16).to(dev)
    x = xs[0].clone()
    mean = torch.empty(rows, dtype=torch.float32, device=dev)
    rstd = torch.empty_like(mean)
    out = torch.empty(rows, n, dtype=torch.bfloat16, device=dev)

    def step():
        pkg.layer_norm_stats(x, 1e-5, mean, rstd)
        pkg.layer_norm_linear(x, w, bias, mean=mean, rstd=rstd, norm_weight=gamma, norm_bias=beta, out=out)

    g = _capture(step)
    for rep in range(2):
        for xi in xs:
            m, r = pkg.layer_norm_stats(xi, 1e-5)
            want = pkg.layer_norm_linear(xi, w, bias, mean=m, rstd=r, norm_weight=gamma, norm_bias=beta).clone()
            torch.cuda.synchronize()
            x.copy_(xi)
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out.view(torch.int16), want.view(torch.int16)), rep
