"""The builder and ground-truth paths bench.py runs on the GPU, against the
same code on the CPU and against a float64 numpy brute force."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = [pytest.mark.gpu, pytest.mark.usefixtures("search_form")]


def test_gpu_codebook_equals_cpu_codebook_on_integer_data(gpu_available):
    """On integer-valued data every distance, rotation and factor numerator
    is an exact integer in the builder's float32 / float64 arithmetic, so the
    GPU build (graph, codes, factors, entry) is byte-identical to the CPU
    build."""
    from flashgann_amd import builder, datasets
    base, _ = datasets.integer_mixture(3000, 1, 128, 16, config=1)
    signs = datasets.signs_for(128, 1)
    a = builder.build_codebook(base, 32, signs, device="cpu")
    b = builder.build_codebook(base, 32, signs, device="cuda")
    assert a.entry == b.entry
    assert np.array_equal(a.rows.view(np.uint32), b.rows.view(np.uint32))


def test_gpu_encoding_of_float_data_within_rounding(gpu_available):
    """On float data the GPU and CPU encodings of one graph agree: codes
    bit-for-bit except where a rotated residual is within rounding of zero,
    factors within float64 summation-order rounding."""
    from flashgann_amd import builder, datasets
    base, _ = datasets.normalized_mixture(2500, 1, 96, 16, config=3)
    signs = datasets.signs_for(128, 3)
    import torch
    nbrs = builder.build_graph(torch.as_tensor(base), 16)
    a = builder.codebook_from_graph(base, nbrs, signs, device="cpu")
    b = builder.codebook_from_graph(base, nbrs, signs, device="cuda")
    assert np.array_equal(a.neighbors(), b.neighbors())
    ca, cb_ = a.codes(), b.codes()
    assert (ca == cb_).mean() > 0.9999
    fa, fb = a.factors(), b.factors()
    np.testing.assert_allclose(fb, fa, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("use_ip", [False, True])
def test_gpu_ground_truth_equals_brute_force(gpu_available, use_ip):
    """GPU ground truth (the ids bench.py scores recall against) equals a
    float64 numpy brute force with ties by id, on integer data where every
    distance is exact."""
    from flashgann_amd import builder, datasets
    base, q = datasets.integer_mixture(5000, 64, 128, 16, config=2)
    gt = builder.ground_truth(base, q, 100, device="cuda", use_ip=use_ip)
    b64, q64 = base.astype(np.float64), q.astype(np.float64)
    if use_ip:
        d = -(q64 @ b64.T)
    else:
        d = (q64 * q64).sum(1)[:, None] + (b64 * b64).sum(1)[None, :] - 2.0 * (q64 @ b64.T)
    ids = np.broadcast_to(np.arange(base.shape[0]), d.shape)
    want = np.lexsort((ids, d), axis=1)[:, :100]
    assert np.array_equal(gt, want.astype(np.int32))


def test_gpu_partitioned_knn_reduces_to_exact_knn(gpu_available):
    """On the GPU as on the CPU: every cell probed is the exact search."""
    import torch
    from flashgann_amd import builder, datasets
    base, _ = datasets.integer_mixture(6000, 1, 64, 8, config=1)
    x = torch.as_tensor(base, device="cuda")
    a_ids, a_d = builder.knn(x, 32)
    b_ids, b_d = builder.knn_partitioned(x, 32, cells=8, probes=8)
    assert torch.equal(a_ids, b_ids) and torch.equal(a_d, b_d)


def test_search_on_partitioned_gpu_build_1536(gpu_available):
    """The C5 build path at small scale: data drawn on the GPU, partitioned
    k-NN graph and encoding on the GPU, then the search (generic geometry,
    padded dimension 2048) against the oracle on the same codebook."""
    from flashgann_amd import Index, builder, datasets
    from oracle import oracle as O
    base, q = datasets.anisotropic_unit_mixture_device(6000, 12, 1536, 24, device="cuda")
    cb = builder.build_codebook(base, 32, datasets.signs_for(2048, 5), device="cuda", knn_method="partitioned")
    qn = q.cpu().numpy()
    ix = Index.from_codebook(cb)
    ids, _, cnt = ix.search(qn, 100, 256, counters=True)
    ix.close()
    rids, rcnt = O.OracleIndex.from_codebook(cb).search(qn, 100, 256)
    assert np.array_equal(ids, rids)
    assert np.array_equal(cnt, rcnt.view(np.uint32).reshape(-1, 6))
    gt = builder.ground_truth(base, q, 100, device="cuda")
    from flashgann_amd.metrics import compute_recall
    assert compute_recall(ids, gt, 100) > 0.9
