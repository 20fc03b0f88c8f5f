"""Writes tests/golden/scann_cases.{json,npz} (run in the development container).

The ScaNN-style index (reference src/neighbors/graphs.cpp:3286-3385) as answered by
the reference library itself (oracle/_ref, CPU route): for each case, the
reference's ovvsScannBuild on the reference tests' LCG inputs
(tests/test_harness.hpp:71-79) and its ovvsScannSearch answers (status, ids,
distances). The first two cases are the reference test's own shapes
(tests/test_neighbors.cpp:2935-2968); the rest cover the metrics, krefine < k,
k above the candidate count, nprobe above nlist and k = 0.

Each case also stores the IPQ1 bytes of an IVF-PQ index that the reference's
ovvsIvfPqBuild makes from the rows scaled by the oracle's column factors
(oracle_scann_aniso). It equals the reference ScaNN's inner index when those
factors equal the reference's, which the oracle test checks through the answers;
with it the CPU oracle can restate the search without a GPU or the reference.

Usage: make -C oracle all ref && python tests/golden/make_scann_fixtures.py
"""

from __future__ import annotations

import json
import sys
import tempfile
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle.pyoracle import Reference, scann_aniso  # noqa: E402
from ovvs_amd.synth import lcg_data  # noqa: E402

OUT = Path(__file__).resolve().parent

# name, data (n, dim, seed), queries (nq, seed), metric, nlist, pq_m,
# searches [(k, nprobe, krefine)]
CASES = [
    ("ref_a", (40, 8, 500), (4, 501), 0, 8, 4, [(4, 8, 12)]),
    ("ref_b", (40, 8, 500), (4, 501), 0, 4, 4, [(4, 4, 40)]),
    ("l2", (600, 16, 11), (9, 12), 0, 12, 4,
     [(10, 4, 32), (5, 12, 3), (20, 1, 20), (8, 100, 64), (0, 4, 8)]),
    ("ip", (500, 16, 13), (7, 14), 2, 10, 8, [(10, 3, 24), (4, 10, 4)]),
    ("cosine", (500, 12, 15), (6, 16), 3, 6, 2, [(10, 2, 16)]),
    ("l2sqrt", (400, 8, 17), (5, 18), 1, 5, 4, [(6, 2, 12)]),
    ("few", (30, 8, 21), (5, 22), 0, 3, 2, [(10, 1, 50), (40, 3, 40)]),
]


def main():
    ref = Reference()
    arrays = {}
    manifest = []
    for name, (n, dim, seed), (nq, qseed), metric, nlist, pq_m, searches in CASES:
        data = lcg_data(n, dim, seed)
        queries = lcg_data(nq, dim, qseed)
        rc, h = ref.scann_build(data, metric, nlist, pq_m)
        assert rc == 0, (name, rc)
        entry = {"name": name, "data_lcg": [n, dim, seed], "queries_lcg": [nq, dim, qseed],
                 "metric": metric, "nlist": nlist, "pq_m": pq_m, "searches": []}
        for j, (k, nprobe, krefine) in enumerate(searches):
            rc, ids, d = ref.scann_search(h, queries, k, nprobe, krefine)
            entry["searches"].append({"k": k, "nprobe": nprobe, "krefine": krefine, "rc": int(rc)})
            arrays[f"{name}/s{j}/ids"] = ids
            arrays[f"{name}/s{j}/dists"] = d
        ref.scann_destroy(h)
        scaled = data * scann_aniso(data)[None, :]
        rc, inner = ref.build(scaled, metric, nlist, pq_m, 8)
        assert rc == 0, (name, rc)
        with tempfile.TemporaryDirectory() as tmp:
            p = Path(tmp) / "inner.ipq1"
            assert ref.save(inner, p) == 0
            arrays[f"{name}/inner_ipq1"] = np.frombuffer(p.read_bytes(), dtype=np.uint8).copy()
        ref.destroy(inner)
        manifest.append(entry)
    ref.close()
    (OUT / "scann_cases.json").write_text(json.dumps(manifest, indent=1) + "\n")
    np.savez_compressed(OUT / "scann_cases.npz", **arrays)
    print(f"{len(manifest)} cases, {sum(len(c['searches']) for c in manifest)} searches")


if __name__ == "__main__":
    main()
