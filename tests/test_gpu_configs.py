"""The benchmark configurations' search shapes on the GPU, against the reference.

BASELINE.json configs[1..4] (C2 1M x 96, C3 10M x 128, C4 1M x 768 inner product,
C5 100M x 96) hold 0.4-38 GB of vectors. Here each runs with its own dim, n_lists,
pq_dim, n_probes, k, metric, table precision and data distribution (ovvs_amd.synth)
on the first n rows of its stream, n small enough for the CPU reference and oracle:

  * fp32 tables: ids and distances bit-identical to the reference library's CPU
    search of the same serialized index (oracle/_ref, skipped when not built) and
    to the oracle;
  * binary16 table requests (the configs' own precision, which the reference CPU
    path does not have) are served with fp32 entries: ids and distances identical
    to the fp32-table search.

These shapes reach the matrix-core probe at its largest group count and nprobe
(C5: 65536 lists, 256 probes), the exact probe route for dim 768 (C4), shortlists
of 100 (C3) and dsub 8 (C4).
"""

from __future__ import annotations

import dataclasses
import sys

import numpy as np
import pytest

from conftest import assert_results_match
from oracle.pyoracle import REF_SO, Oracle, Reference, read_ipq1

pytestmark = pytest.mark.gpu

# Rows per reduced configuration: lists keep a few rows each at these n_lists.
REDUCED_N = {"c2": 200_000, "c3": 150_000, "c4": 60_000, "c5": 400_000}
QUERIES = 100


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def res(ovvs):
    r = ovvs.Resources()
    if not r.gpu_available():
        pytest.fail("no GPU visible: gpu tests must run on the MI355X box")
    return r


@pytest.mark.parametrize("name", ["c2", "c3", "c4", "c5"])
def test_config_shapes_against_reference(ovvs, res, tmp_path, name):
    from ovvs_amd import synth

    cfg = dataclasses.replace(synth.CONFIGS[name], n=REDUCED_N[name])
    C = synth.centers(cfg)
    data = synth.base_rows(cfg, 0, cfg.n, C)
    q = synth.query_rows(cfg, 0, QUERIES, C)
    say(name, "build", dict(n=cfg.n, dim=cfg.dim, nlist=cfg.nlist, pq_m=cfg.pq_m,
                            metric=cfg.metric))
    ix = ovvs.neighbors.ivf_pq.build(data, metric=cfg.metric, nlist=cfg.nlist, pq_m=cfg.pq_m,
                                     pq_nbits=8, resources=res)
    p = tmp_path / f"{name}.ipq1"
    ix.serialize(p)
    orc = Oracle(read_ipq1(p))
    k, nprobe = cfg.k, cfg.nprobe

    say(name, "fp32 tables")
    ids32, d32 = ix.search_ex(q, k, nprobe, k, lut_dtype=ovvs.DTYPE_F32)
    oids, od = orc.search(q, k, nprobe, k)
    assert_results_match(ids32, d32, oids, od, label=f"{name} fp32 vs oracle")
    assert np.array_equal(_bits(d32), _bits(od)), name
    if REF_SO.exists():
        ref = Reference()
        rc, h = ref.load(p)
        assert rc == 0
        rc, rids, rd = ref.search(h, q, k, nprobe, k)
        assert rc == 0
        assert np.array_equal(ids32, rids), f"{name}: ids differ from the reference"
        assert np.array_equal(_bits(d32), _bits(rd)), f"{name}: distances differ"
        ref.destroy(h)
        ref.close()

    # Binary16 table requests (the configs' own precision; the reference has none)
    # are served with fp32 entries: the same results, so every rank's distance is
    # within the 2e-3 bar of the fp32-table search (it is the same bits).
    say(name, "fp16 table request")
    ids16, d16 = ix.search_ex(q, k, nprobe, k, lut_dtype=ovvs.DTYPE_F16)
    assert np.array_equal(ids16, ids32), name
    assert np.array_equal(_bits(d16), _bits(d32)), name
    assert_results_match(ids16, d16, ids32, d32, rel=2e-3, label=f"{name} fp16 request")
    ix.close()


# The configurations' rows per list, at fewer lists than the workloads (so that
# data, build and the CPU checks fit a test): each list then holds as many
# segments and groups as the workload's lists do, which is what the scan's bound
# passes, phase-0 rounds and item rounds depend on. Workload rows per list: C2
# 244, C3 610, C4 488, C5 1526; here 122, 305, 250 and 1000 (the probe counts,
# dims, pq_dim, k, metric and data distributions are the configurations' own).
ROWS_PER_LIST = {
    "c2": (4096, 500_000),    # nlist, n
    "c3": (4096, 1_250_000),
    "c4": (1024, 256_000),
    "c5": (2048, 2_048_000),
}
QUERIES_RPL = 50


@pytest.mark.parametrize("name", ["c2", "c3", "c4", "c5"])
def test_config_rows_per_list_against_reference(ovvs, res, tmp_path, name):
    from ovvs_amd import synth

    nlist, n = ROWS_PER_LIST[name]
    cfg = dataclasses.replace(synth.CONFIGS[name], n=n, nlist=nlist)
    C = synth.centers(cfg)
    say(name, "rows per list: generate", dict(n=n, nlist=nlist, rows_per_list=n // nlist))
    data = synth.base_rows(cfg, 0, cfg.n, C)
    q = synth.query_rows(cfg, 0, QUERIES_RPL, C)
    say(name, "rows per list: build")
    ix = ovvs.neighbors.ivf_pq.build(data, metric=cfg.metric, nlist=nlist, pq_m=cfg.pq_m,
                                     pq_nbits=8, resources=res)
    p = tmp_path / f"{name}_rpl.ipq1"
    ix.serialize(p)
    del data
    k, nprobe = cfg.k, cfg.nprobe
    say(name, "rows per list: search")
    ids, d = ix.search(q, k, nprobe, k)
    ids16, d16 = ix.search_ex(q, k, nprobe, k, lut_dtype=ovvs.DTYPE_F16)
    ids32r, d32r = ix.search(q, k, nprobe, 32 if k < 32 else k)
    say(name, "rows per list: oracle")
    orc = Oracle(read_ipq1(p))
    oids, od = orc.search(q, k, nprobe, k)
    assert_results_match(ids, d, oids, od, label=f"{name} rows-per-list vs oracle")
    assert np.array_equal(_bits(d), _bits(od)), name
    assert np.array_equal(ids16, ids) and np.array_equal(_bits(d16), _bits(d)), name
    oids32, od32 = orc.search(q, k, nprobe, 32 if k < 32 else k)
    assert np.array_equal(ids32r, oids32) and np.array_equal(_bits(d32r), _bits(od32)), name
    del orc
    if REF_SO.exists():
        say(name, "rows per list: reference")
        ref = Reference()
        rc, h = ref.load(p)
        assert rc == 0
        rc, rids, rd = ref.search(h, q, k, nprobe, k)
        assert rc == 0
        assert np.array_equal(ids, rids), f"{name}: ids differ from the reference"
        assert np.array_equal(_bits(d), _bits(rd)), f"{name}: distances differ"
        ref.destroy(h)
        ref.close()
    st = res.ivfpq_search_stats()
    say(name, "rows per list: candidate rows per query so far",
        st["candidate_rows"] / max(1, st["queries"]))
    ix.close()
