"""The matrix-core coarse probe (ovvs_amd/csrc/probe.hip) against the oracle.

Searches with dim <= 1024, nprobe <= 256 and at least 2 * nprobe groups of
centroids take the fused probe: approximate scores from one bf16 matrix-core
product of centred operands, a proven candidate bound, exact re-score of the
candidates. Everything else takes the exact score-matrix route. These cases sit
in the fused regime (padded dims, dims held in registers and dims read from LDS
per k-step, nlist not a multiple of 16, the largest nprobe, integer data far from
the origin, data whose bf16 roundings all err the same way) and require results
bit-identical to the oracle's, including queries whose candidates exceed the
re-score capacity (tied centroids) and so go through the exact fallback in the
same batch as ordinary queries.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest

from conftest import assert_results_match
from oracle.pyoracle import Oracle, read_ipq1

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True, file=sys.stderr)


@pytest.fixture(scope="module")
def res(ovvs):
    r = ovvs.Resources()
    if not r.gpu_available():
        pytest.fail("no GPU visible: gpu tests must run on the MI355X box")
    return r


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def _mixture(rng, n, dim, centers):
    return (centers[rng.integers(0, len(centers), n)] +
            0.3 * rng.standard_normal((n, dim))).astype(np.float32)


def _check(ix, orc, q, k, nprobe, krefine, label):
    ids, d = ix.search(q, k, nprobe, krefine)
    oids, od = orc.search(q, k, nprobe, krefine)
    assert_results_match(ids, d, oids, od, label=label)
    assert np.array_equal(_bits(d), _bits(od)), label


@pytest.mark.parametrize("dim,pq_m,nlist,nprobes", [
    (96, 24, 1024, (8, 32, 128)),
    (40, 10, 1000, (16, 64)),
    (128, 32, 2048, (64, 256)),
    (8, 4, 700, (8, 40)),
    (200, 25, 1000, (16, 64)),
    (768, 96, 2048, (32, 128)),
])
def test_matrix_core_probe_matches_oracle(ovvs, res, tmp_path, dim, pq_m, nlist, nprobes):
    rng = np.random.default_rng(dim * 1000 + nlist)
    centers = rng.standard_normal((256, dim)).astype(np.float32)
    data = _mixture(rng, 30000, dim, centers)
    q = _mixture(rng, 300, dim, centers)
    say("build", dict(dim=dim, pq_m=pq_m, nlist=nlist))
    ix = ovvs.neighbors.ivf_pq.build(data, nlist=nlist, pq_m=pq_m, pq_nbits=8, resources=res)
    p = tmp_path / "probe.ipq1"
    ix.serialize(p)
    orc = Oracle(read_ipq1(p))
    for nprobe in nprobes:
        for k, krefine in [(10, 32), (100, 300)]:
            say("search", dict(nprobe=nprobe, k=k, krefine=krefine))
            _check(ix, orc, q, k, nprobe, krefine, f"d{dim} l{nlist} p{nprobe} k{k}")
    ix.close()


@pytest.mark.parametrize("dim,pq_m,nlist,nprobe", [
    (96, 24, 4096, 256),   # 1024 re-score slots: one workgroup per CU, wide instance
    (96, 24, 2048, 256),   # the same LDS, chunks too short for its batches: sixteen waves
    (768, 96, 2048, 32),   # query rows in LDS: wide instance with LDS operands
])
def test_probe_one_workgroup_per_cu_large_batch(ovvs, res, tmp_path, dim, pq_m, nlist, nprobe):
    """Batches of at least 256 workgroups at shapes whose LDS admits one workgroup per
    CU take the sixteen-wave instances (deeper prefetch where the chunks allow)."""
    rng = np.random.default_rng(dim + nlist + nprobe)
    centers = rng.standard_normal((256, dim)).astype(np.float32)
    data = _mixture(rng, 30000, dim, centers)
    q = _mixture(rng, 4200, dim, centers)
    say("build", dict(dim=dim, pq_m=pq_m, nlist=nlist, nprobe=nprobe))
    ix = ovvs.neighbors.ivf_pq.build(data, nlist=nlist, pq_m=pq_m, pq_nbits=8, resources=res)
    p = tmp_path / "probe_wide.ipq1"
    ix.serialize(p)
    orc = Oracle(read_ipq1(p))
    _check(ix, orc, q, 10, nprobe, 32, f"wide d{dim} l{nlist} p{nprobe}")
    ix.close()


def test_probe_fallback_for_tied_centroids(ovvs, res, tmp_path):
    """700 identical centroids tie every approximate score near them, so queries
    there have more candidates than the re-score capacity and are ranked by the
    exact fallback; the other queries of the batch stay on the fused probe.
    With every centroid identical, all queries fall back and the probes are the
    first nprobe centroids by ordinal."""
    rng = np.random.default_rng(5)
    dim, nlist = 32, 1024
    centers = rng.standard_normal((128, dim)).astype(np.float32)
    data = _mixture(rng, 20000, dim, centers)
    say("build tied-centroid index")
    built = ovvs.neighbors.ivf_pq.build(data, nlist=nlist, pq_m=8, pq_nbits=8, resources=res)
    p = tmp_path / "base.ipq1"
    built.serialize(p)
    built.close()
    base = read_ipq1(p)

    base.centroids[100:800] = base.centroids[100]
    tied = tmp_path / "tied.ipq1"
    tied.write_bytes(base.to_bytes())
    ix = ovvs.neighbors.ivf_pq.load(tied, resources=res)
    orc = Oracle(read_ipq1(tied))
    near = (base.centroids[100] + 0.01 * rng.standard_normal((100, dim))).astype(np.float32)
    q = np.concatenate([near, _mixture(rng, 100, dim, centers)])
    q = q[rng.permutation(len(q))]
    for nprobe in (4, 16, 64):
        say("tied search", nprobe)
        _check(ix, orc, q, 10, nprobe, 32, f"tied p{nprobe}")
    ix.close()

    base.centroids[:] = base.centroids[0]
    same = tmp_path / "same.ipq1"
    same.write_bytes(base.to_bytes())
    ix = ovvs.neighbors.ivf_pq.load(same, resources=res)
    orc = Oracle(read_ipq1(same))
    say("all-identical search")
    _check(ix, orc, q, 10, 16, 64, "all identical")
    ix.close()


def test_probe_integer_data_far_from_origin(ovvs, res, tmp_path):
    """Integer coordinates in [0, 255] (C3's distribution): the centring keeps the
    bf16 error relative to the clusters' spread rather than to |x| ~ 1600."""
    rng = np.random.default_rng(255)
    dim = 128
    centers = rng.uniform(0, 255, (512, dim))
    data = np.clip(np.rint(centers[rng.integers(0, 512, 40000)] + 12.0 *
                           rng.standard_normal((40000, dim))), 0, 255).astype(np.float32)
    q = np.clip(np.rint(centers[rng.integers(0, 512, 300)] + 12.0 *
                        rng.standard_normal((300, dim))), 0, 255).astype(np.float32)
    ix = ovvs.neighbors.ivf_pq.build(data, nlist=2048, pq_m=64, pq_nbits=8, resources=res)
    p = tmp_path / "int255.ipq1"
    ix.serialize(p)
    orc = Oracle(read_ipq1(p))
    for nprobe in (32, 128, 256):
        say("int255 search", nprobe)
        _check(ix, orc, q, 100, nprobe, 100, f"int255 p{nprobe}")
    ix.close()


def test_probe_aligned_bf16_rounding(ovvs, res, tmp_path):
    """Centroids and queries whose coordinates bf16 rounds the same way (magnitude
    1 + 3 * 2^-10 rounds down to 1) put the approximate scores as far from the exact
    ones as the bound allows: the candidate sets must still contain the exact probes."""
    rng = np.random.default_rng(17)
    dim, nlist = 64, 1024
    base = np.float32(1.0 + 3.0 * 2.0 ** -10)
    signs = np.where(rng.random((64, dim)) < 0.5, 1.0, -1.0)
    data = (base * signs[rng.integers(0, 64, 20000)] +
            0.05 * rng.standard_normal((20000, dim))).astype(np.float32)
    q = (base * signs[rng.integers(0, 64, 300)] +
         0.05 * rng.standard_normal((300, dim))).astype(np.float32)
    ix = ovvs.neighbors.ivf_pq.build(data, nlist=nlist, pq_m=16, pq_nbits=8, resources=res)
    p = tmp_path / "aligned.ipq1"
    ix.serialize(p)
    orc = Oracle(read_ipq1(p))
    for nprobe in (8, 64, 256):
        say("aligned search", nprobe)
        _check(ix, orc, q, 10, nprobe, 32, f"aligned p{nprobe}")
    ix.close()
