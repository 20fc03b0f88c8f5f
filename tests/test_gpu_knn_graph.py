"""GPU parity of ovvsIvfPqKnnGraph, the CAGRA build's IVF-PQ initializer
(reference src/neighbors/graphs.cpp:767-797).

The reference builds an IVF-PQ index (nlist = max(2, min(8, n/4)), pq_m = the largest
divisor of dim not above 4, 8 bits), searches every row on its own for degree + 1
neighbours with every list probed and krefine = degree + 1, and keeps the results other
than the row itself and -1. The expected graphs here come from that same sequence of
calls on the reference library (oracle/_ref, CPU route), and from the oracle's search
over the index libovvs builds (its build is the reference's, byte for byte). Bar:
identical graphs.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest

from oracle.pyoracle import REF_SO, Oracle, Reference, read_ipq1
from ovvs_amd.synth import lcg_data

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True, file=sys.stderr)


@pytest.fixture(scope="module")
def res(ovvs):
    r = ovvs.Resources()
    if not r.gpu_available():
        pytest.fail("no GPU visible: gpu tests must run on the MI355X box")
    return r


def shape_params(n, dim):
    nlist = max(2, min(8, n // 4))
    pq_m = next(c for c in range(min(4, dim), 0, -1) if dim % c == 0)
    return nlist, pq_m


def assemble(ids, degree):
    """graphs.cpp:788-795: each row's results other than itself and -1, padded."""
    g = np.full((ids.shape[0], degree), -1, dtype=np.int32)
    for i, row in enumerate(ids):
        kept = [int(x) for x in row if x != i and x >= 0][:degree]
        g[i, :len(kept)] = kept
    return g


CASES = [  # (n, dim, metric, degree, data)
    (600, 12, 0, 16, "lcg"),
    (600, 12, 2, 16, "lcg"),
    (30, 8, 0, 40, "lcg"),      # k above n: padded lists
    (2500, 20, 0, 32, "clustered"),
]


def case_data(n, dim, kind, seed):
    if kind == "lcg":
        return lcg_data(n, dim, seed)
    rng = np.random.default_rng(seed)
    c = rng.standard_normal((16, dim)).astype(np.float32)
    return (c[rng.integers(0, 16, n)] + 0.2 * rng.standard_normal((n, dim))).astype(np.float32)


@pytest.mark.parametrize("case", range(len(CASES)))
def test_knn_graph_matches_oracle(ovvs, res, tmp_path, case):
    n, dim, metric, degree, kind = CASES[case]
    x = case_data(n, dim, kind, 40 + case)
    nlist, pq_m = shape_params(n, dim)
    say("knn graph vs oracle", n, dim, metric, degree, nlist, pq_m)
    g = ovvs.neighbors.ivf_pq.knn_graph(x, degree, metric=metric, resources=res)
    ix = ovvs.neighbors.ivf_pq.build(x, metric=metric, nlist=nlist, pq_m=pq_m, pq_nbits=8,
                                     resources=res)
    p = tmp_path / "knn.ipq1"
    ix.serialize(p)
    ix.close()
    ids, _ = Oracle(read_ipq1(p)).search(x, degree + 1, nlist, degree + 1)
    assert np.array_equal(g, assemble(ids, degree))


@pytest.mark.skipif(not REF_SO.exists(), reason="oracle/_ref not built")
@pytest.mark.parametrize("case", range(len(CASES)))
def test_knn_graph_matches_reference_call_sequence(ovvs, res, case):
    n, dim, metric, degree, kind = CASES[case]
    x = case_data(n, dim, kind, 40 + case)
    nlist, pq_m = shape_params(n, dim)
    say("knn graph vs reference", n, dim, metric, degree)
    g = ovvs.neighbors.ivf_pq.knn_graph(x, degree, metric=metric, resources=res)
    ref = Reference()
    rc, h = ref.build(x, metric, nlist, pq_m, 8)
    assert rc == 0
    rows = []
    for i in range(n):  # one row per call, as the reference initializer searches
        rc, ids, _ = ref.search(h, x[i:i + 1], degree + 1, nlist, degree + 1)
        assert rc == 0
        rows.append(ids[0])
    ref.destroy(h)
    ref.close()
    assert np.array_equal(g, assemble(np.stack(rows), degree))


def test_knn_graph_spans_search_batches(ovvs, res, tmp_path):
    """70,000 rows: the graph's searches run in batches of 65,536 rows
    (knn_graph_index.cpp), so the second batch's query offsets into the device rows,
    its self-exclusion (row ids from 65,536 on) and the reuse of the workspace across
    batches are exercised. Rows around the batch boundary, the last rows and a random
    sample are checked against the oracle's search over the index libovvs builds."""
    n, dim, degree = 70_000, 8, 8
    rng = np.random.default_rng(70)
    c = rng.standard_normal((64, dim)).astype(np.float32)
    x = (c[rng.integers(0, 64, n)] + 0.3 * rng.standard_normal((n, dim))).astype(np.float32)
    nlist, pq_m = shape_params(n, dim)
    say("knn graph across batches", n, dim, degree, nlist, pq_m)
    g = ovvs.neighbors.ivf_pq.knn_graph(x, degree, metric=0, resources=res)
    assert g.shape == (n, degree)
    ix = ovvs.neighbors.ivf_pq.build(x, metric=0, nlist=nlist, pq_m=pq_m, pq_nbits=8,
                                     resources=res)
    p = tmp_path / "knn_batches.ipq1"
    ix.serialize(p)
    ix.close()
    rows = np.unique(np.concatenate([np.arange(0, 20), np.arange(65_516, 65_556),
                                     np.arange(n - 20, n), rng.integers(0, n, 300)]))
    say("oracle search of", len(rows), "rows")
    ids, _ = Oracle(read_ipq1(p)).search(x[rows], degree + 1, nlist, degree + 1)
    for r, row in zip(rows, ids):
        kept = [int(v) for v in row if v != r and v >= 0][:degree]
        want = np.full(degree, -1, dtype=np.int32)
        want[:len(kept)] = kept
        assert np.array_equal(g[r], want), f"row {r}"
