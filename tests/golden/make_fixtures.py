"""Writes the golden fixtures under tests/golden/ (run in the development container).

1. legacy_ipq1_v1.bin — the 268-byte IPQ1 v1 file the reference's compatibility
   test constructs (reference tests/test_neighbors.cpp:509-544): n=4, dim=2,
   nlist=1, pq_m=1, ks=16, centroid (0,0), codewords 0..3 = (c, 0), the rest
   (100, 100), codes 0..3, rows (0,0),(1,0),(2,0),(3,0), one list [0,1,2,3].
   Expected answers (reference tests/test_neighbors.cpp:1352-1425) are asserted in
   tests/test_abi.py: query (1.1, 0), k=2, nprobe=1, krefine=4 -> ids [1, 2],
   distances [0.01, 0.81] within 1e-5; byte-exact re-serialization; version 2 ->
   UNSUPPORTED; truncation, out-of-range id at byte 236, duplicate id at byte 244
   -> IO.

2. ref_cases.npz — indexes built by the reference library (oracle/_ref, CPU
   route) on the reference tests' LCG inputs, serialized as IPQ1 bytes, with
   queries, filters and the reference's search answers. The cases follow the
   reference tests: recall smoke (test_neighbors.cpp:907-930), filters
   (:1565-1669), equal-score ties (:1767-1822), cross-list ties (:1854-1931),
   extend (:1936-2074), plus one case per metric and a 4-bit case.

Usage: make -C oracle all ref && python tests/golden/make_fixtures.py
"""

from __future__ import annotations

import json
import sys
import tempfile
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle.pyoracle import Reference  # noqa: E402
from ovvs_amd.synth import lcg_data  # noqa: E402

OUT = Path(__file__).resolve().parent


def legacy_blob() -> bytes:
    parts = [
        np.array([0x31515049], dtype=np.uint32).tobytes(),
        np.array([1], dtype=np.int32).tobytes(),
        np.array([4, 2], dtype=np.int64).tobytes(),
        np.array([1, 1, 16, 2, 0], dtype=np.int32).tobytes(),
        np.zeros(2, dtype=np.float32).tobytes(),
    ]
    cb = np.full((16, 2), 100.0, dtype=np.float32)
    cb[:4, 0] = np.arange(4, dtype=np.float32)
    cb[:4, 1] = 0.0
    parts += [
        cb.tobytes(),
        np.arange(4, dtype=np.uint8).tobytes(),
        np.array([0, 0, 1, 0, 2, 0, 3, 0], dtype=np.float32).tobytes(),
        np.zeros(4, dtype=np.int32).tobytes(),
        np.array([4], dtype=np.int32).tobytes(),
        np.arange(4, dtype=np.int64).tobytes(),
    ]
    blob = b"".join(parts)
    assert len(blob) == 268
    return blob


def bitset(n, ids, tail_all=False):
    b = np.zeros((n + 7) // 8, dtype=np.uint8)
    for i in ids:
        b[i >> 3] |= np.uint8(1 << (i & 7))
    if tail_all:
        b[-1] = 0xFF
    return b


def main():
    (OUT / "legacy_ipq1_v1.bin").write_bytes(legacy_blob())
    ref = Reference()
    arrays = {}
    manifest = []

    def add_case(name, data, metric, nlist, pq_m, nbits, queries, searches, extra=None):
        """data/extra: an explicit array, or ("lcg", n, dim, seed) for lcg_data inputs."""
        source = data
        if isinstance(data, tuple):
            data = lcg_data(*data[1:])
        extra_source = extra
        if isinstance(extra, tuple):
            extra = lcg_data(*extra[1:])
        rc, h = ref.build(data, metric, nlist, pq_m, nbits)
        assert rc == 0, (name, rc)
        if extra is not None:
            assert ref.extend(h, extra) == 0, name
        with tempfile.TemporaryDirectory() as d:
            p = Path(d) / "ix.ipq1"
            assert ref.save(h, p) == 0
            arrays[f"{name}/ipq1"] = np.frombuffer(p.read_bytes(), dtype=np.uint8).copy()
        entry = {"name": name, "metric": metric, "nlist": nlist, "pq_m": pq_m, "nbits": nbits,
                 "extended": extra is not None, "searches": []}
        if isinstance(source, tuple):
            entry["data_lcg"] = list(source[1:])
        else:
            arrays[f"{name}/data"] = np.ascontiguousarray(data, dtype=np.float32)
        if isinstance(extra_source, tuple):
            entry["extra_lcg"] = list(extra_source[1:])
        elif extra is not None:
            arrays[f"{name}/extra"] = np.ascontiguousarray(extra, dtype=np.float32)
        arrays[f"{name}/queries"] = np.ascontiguousarray(queries, dtype=np.float32)
        for j, (k, nprobe, krefine, filt) in enumerate(searches):
            key = f"{name}/s{j}"
            if filt is not None:
                arrays[f"{key}/bitset"] = filt
            rc, ids, dist = ref.search(h, queries, k, nprobe, krefine, filt)
            assert rc == 0, (name, j, rc)
            arrays[f"{key}/ids"] = ids
            arrays[f"{key}/dists"] = dist
            entry["searches"].append({"k": k, "nprobe": nprobe, "krefine": krefine,
                                      "filtered": filt is not None})
        manifest.append(entry)
        ref.destroy(h)

    # Recall smoke (test_neighbors.cpp:907-930).
    add_case("recall", ("lcg", 64, 8, 210), 0, 8, 4, 8, lcg_data(5, 8, 211),
             [(4, 8, 16, None), (4, 2, 4, None)])
    # Filters, tail bits and 33-query batches (test_neighbors.cpp:1565-1669).
    n = 65
    allowed = np.full((n + 7) // 8, 0xFF, dtype=np.uint8)
    selective = bitset(n, [0, 1, 31, 32], tail_all=True)
    empty = np.zeros((n + 7) // 8, dtype=np.uint8)
    add_case("filters", ("lcg", n, 8, 224), 0, 7, 4, 4, lcg_data(33, 8, 225),
             [(8, 7, n, None), (8, 7, n, allowed), (8, 7, n, selective), (8, 7, n, empty),
              (3, 2, 5, selective)])
    # Equal scores: 129 zero vectors, one list (test_neighbors.cpp:1767-1822).
    add_case("ties", np.zeros((129, 4), dtype=np.float32), 0, 1, 2, 4,
             np.zeros((1, 4), dtype=np.float32), [(1, 1, 1, None), (8, 1, 128, None)])
    # Cross-list equal scores (test_neighbors.cpp:1854-1931).
    pts = np.array([[-1.0, 0.0], [1.0, 0.0]], dtype=np.float32)
    add_case("crosslist", pts, 0, 2, 1, 4, np.array([[0.0, 0.0], [-1.0, 0.0], [1.0, 0.0]],
                                                    dtype=np.float32),
             [(1, 2, 1, None), (2, 2, 2, None), (1, 1, 1, None)])
    # Extend: build on 65 rows, append 7 (test_neighbors.cpp:1936-2074).
    add_case("extend", ("lcg", 65, 8, 300), 0, 6, 4, 8, lcg_data(9, 8, 302),
             [(5, 6, 72, None), (5, 3, 10, None)], extra=("lcg", 7, 8, 301))
    # Every metric on one shape.
    for metric in range(6):
        add_case(f"metric{metric}", ("lcg", 300, 16, 400 + metric), metric, 12, 8, 8,
                 lcg_data(20, 16, 500 + metric), [(10, 4, 32, None), (5, 12, 300, None)])
    # A mid-size case with 4-bit and 8-bit codes.
    add_case("mid8", ("lcg", 3000, 16, 600), 0, 40, 8, 8, lcg_data(64, 16, 601),
             [(10, 8, 32, None), (10, 3, 10, None), (100, 40, 256, None)])
    add_case("mid4", ("lcg", 3000, 16, 610), 0, 40, 4, 4, lcg_data(64, 16, 611),
             [(10, 8, 32, None)])
    ref.close()
    np.savez_compressed(OUT / "ref_cases.npz", **arrays)
    (OUT / "ref_cases.json").write_text(json.dumps(manifest, indent=1) + "\n")
    print("wrote", OUT / "ref_cases.npz", sum(a.nbytes for a in arrays.values()), "bytes raw")


if __name__ == "__main__":
    main()
