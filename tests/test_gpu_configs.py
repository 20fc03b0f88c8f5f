"""The benchmark configurations' search shapes on the GPU, against the reference.

BASELINE.json configs[1..4] (C2 1M x 96, C3 10M x 128, C4 1M x 768 inner product,
C5 100M x 96) hold 0.4-38 GB of vectors. Here each runs with its own dim, n_lists,
pq_dim, n_probes, k, metric, table precision and data distribution (ovvs_amd.synth)
on the first n rows of its stream, n small enough for the CPU reference and oracle:

  * fp32 tables: ids and distances bit-identical to the reference library's CPU
    search of the same serialized index (oracle/_ref, skipped when not built) and
    to the oracle;
  * binary16 tables (the configs' own precision, which the reference CPU path does
    not have): ids and distances bit-identical to the oracle's binary16 extension;
    their distance from the fp32-table results is reported.

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

    say(name, "fp16 tables")
    ids16, d16 = ix.search_ex(q, k, nprobe, k, lut_dtype=ovvs.DTYPE_F16)
    hids, hd = orc.search(q, k, nprobe, k, lut_f16=True)
    assert_results_match(ids16, d16, hids, hd, label=f"{name} fp16 vs oracle extension")
    assert np.array_equal(_bits(d16), _bits(hd)), name
    # binary16 tables change the ADC ranking at the level of their rounding (and
    # entries above 65504 become +inf): the neighbors stay close to the fp32-table
    # search. Measured at these sizes: C4 and C5 identical; C3 (integer data,
    # 100 neighbors with close distances) 0.76 id overlap, median k-th distance
    # 5e-3 apart. The bound below is a sanity floor, not the parity bar.
    overlap = np.mean([len(set(a) & set(b)) / k for a, b in zip(ids16, ids32)])
    kth16 = d16[:, -1].astype(np.float64)
    kth32 = d32[:, -1].astype(np.float64)
    fin = np.isfinite(kth32) & np.isfinite(kth16)
    rel = np.abs(kth16[fin] - kth32[fin]) / np.maximum(np.abs(kth32[fin]), 1e-30)
    say(name, f"fp16 vs fp32 tables: id overlap {overlap:.4f}, k-th distance rel. diff "
              f"median {np.median(rel):.2e} max {rel.max():.2e}")
    assert overlap >= 0.5, f"{name}: fp16/fp32 id overlap {overlap:.3f}"
    assert np.median(rel) <= 2e-2, f"{name}: median k-th distance diff {np.median(rel):.2e}"
    ix.close()
