"""Pins the CPU oracle (oracle/ivfpq_oracle.c) before it is trusted as the checker.

Checks, each chosen so a plausible slip (a dropped term, FMA contraction, a wrong
tie order, a sign error) fails one of them:
  * bit-identical ids and distances against answers produced by the reference
    library itself (tests/golden/ref_cases.*, reference CPU route);
  * the same against the live reference build in oracle/_ref on fresh inputs
    (skipped when it is not built);
  * the reference tests' known answers: legacy IPQ1 query, equal-score ties,
    cross-list ties, filters;
  * the closed form nprobe = nlist, krefine >= n, which is exact brute force;
  * binary16 conversion against numpy's independent IEEE implementation;
  * the ScaNN-style search: the reference's own ScaNN answers
    (tests/golden/scann_cases.*, and oracle/_ref live), closed-form column
    statistics, and brute force at full probe and refine.
"""

from __future__ import annotations

import numpy as np
import pytest

from conftest import GOLDEN, case_data, write_case_ipq1
from oracle.pyoracle import (REF_SO, Oracle, Reference, brute_force, oracle_lib, read_ipq1,
                             scann_aniso)
from ovvs_amd.synth import lcg_data


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_oracle_reproduces_reference_answers_bit_exact(ref_cases, tmp_path):
    manifest, arrays = ref_cases
    checked = 0
    for case in manifest:
        ix = read_ipq1(write_case_ipq1(case, arrays, tmp_path))
        orc = Oracle(ix)
        q = arrays[f"{case['name']}/queries"]
        for j, s in enumerate(case["searches"]):
            key = f"{case['name']}/s{j}"
            bits = arrays.get(f"{key}/bitset")
            ids, d = orc.search(q, s["k"], s["nprobe"], s["krefine"], bits)
            assert np.array_equal(ids, arrays[f"{key}/ids"]), key
            assert np.array_equal(_bits(d), _bits(arrays[f"{key}/dists"])), key
            checked += 1
    assert checked >= 25


@pytest.mark.skipif(not REF_SO.exists(), reason="oracle/_ref not built")
@pytest.mark.parametrize("seed", [1, 2, 3])
def test_oracle_matches_live_reference(seed, tmp_path):
    rng = np.random.default_rng(seed)
    ref = Reference()
    dim = int(rng.choice([8, 12, 32]))
    pq_m = int(rng.choice([d for d in (1, 2, 4, 8) if dim % d == 0]))
    n = int(rng.integers(200, 1500))
    nlist = int(rng.integers(2, 40))
    nbits = int(rng.choice([4, 6, 8]))
    metric = int(rng.integers(0, 6))
    data = rng.standard_normal((n, dim)).astype(np.float32)
    q = rng.standard_normal((17, dim)).astype(np.float32)
    rc, h = ref.build(data, metric, nlist, pq_m, nbits)
    assert rc == 0
    path = tmp_path / "live.ipq1"
    assert ref.save(h, path) == 0
    orc = Oracle(read_ipq1(path))
    bits = (rng.random((n + 7) // 8 * 8) < 0.6).astype(np.uint8)
    bitset = np.packbits(bits, bitorder="little")
    for k, nprobe, krefine, filt in [(10, 3, 20, None), (7, nlist, 7, None), (5, 4, 64, bitset),
                                     (3, 0, 1, None)]:
        rc, rids, rd = ref.search(h, q, k, nprobe, krefine, filt)
        assert rc == 0
        oids, od = orc.search(q, k, nprobe, krefine, filt)
        assert np.array_equal(oids, rids)
        assert np.array_equal(_bits(od), _bits(rd))
    ref.destroy(h)
    ref.close()


def test_legacy_ipq1_known_answer():
    orc = Oracle(read_ipq1(GOLDEN / "legacy_ipq1_v1.bin"))
    ids, d = orc.search(np.array([[1.1, 0.0]], np.float32), 2, 1, 4)
    assert ids.tolist() == [[1, 2]]
    assert abs(d[0, 0] - 0.01) < 1e-5 and abs(d[0, 1] - 0.81) < 1e-5


def test_equal_score_ties_use_dense_ordinal(ref_cases, tmp_path):
    manifest, arrays = ref_cases
    case = next(c for c in manifest if c["name"] == "ties")
    orc = Oracle(read_ipq1(write_case_ipq1(case, arrays, tmp_path)))
    q = np.zeros((1, 4), np.float32)
    ids, d = orc.search(q, 1, 1, 1)
    assert ids.tolist() == [[0]] and d[0, 0] == 0.0
    ids, d = orc.search(q, 8, 1, 128)
    assert ids.tolist() == [list(range(8))] and np.all(d == 0.0)


def test_cross_list_ties_follow_probe_order(ref_cases, tmp_path):
    manifest, arrays = ref_cases
    case = next(c for c in manifest if c["name"] == "crosslist")
    orc = Oracle(read_ipq1(write_case_ipq1(case, arrays, tmp_path)))
    mid = np.zeros((1, 2), np.float32)
    ids, d = orc.search(mid, 2, 2, 2)
    assert sorted(ids[0].tolist()) == [0, 1] and d.tolist() == [[1.0, 1.0]]
    # The winner of the tie is the row of the first-probed list.
    probes = orc.probes(mid, 2)[0]
    first_list_rows = orc.packed_ids[orc.offsets[probes[0]]:orc.offsets[probes[0] + 1]]
    ids1, _ = orc.search(mid, 1, 2, 1)
    assert ids1[0, 0] == first_list_rows[0]


def test_filters_known_answers(ref_cases, tmp_path):
    manifest, arrays = ref_cases
    case = next(c for c in manifest if c["name"] == "filters")
    orc = Oracle(read_ipq1(write_case_ipq1(case, arrays, tmp_path)))
    q = arrays["filters/queries"]
    sel = arrays["filters/s2/bitset"]
    ids, d = orc.search(q, 8, 7, 65, sel)
    allowed = {0, 1, 31, 32, 64}
    for row_ids, row_d in zip(ids, d):
        assert set(row_ids[:5].tolist()) == allowed
        assert np.all(row_ids[5:] == -1) and np.all(np.isposinf(row_d[5:]))
    ids, d = orc.search(q, 8, 7, 65, arrays["filters/s3/bitset"])
    assert np.all(ids == -1) and np.all(np.isposinf(d))
    a_ids, a_d = orc.search(q, 8, 7, 65, arrays["filters/s1/bitset"])
    n_ids, n_d = orc.search(q, 8, 7, 65)
    assert np.array_equal(a_ids, n_ids) and np.array_equal(_bits(a_d), _bits(n_d))


@pytest.mark.parametrize("metric", [0, 1, 2, 3, 4, 5])
def test_full_probe_full_refine_is_brute_force(ref_cases, tmp_path, metric):
    manifest, arrays = ref_cases
    case = next(c for c in manifest if c["name"] == f"metric{metric}")
    ix = read_ipq1(write_case_ipq1(case, arrays, tmp_path))
    orc = Oracle(ix)
    q = arrays[f"metric{metric}/queries"]
    k = 10
    ids, d = orc.search(q, k, ix.nlist, ix.n)
    bids, bd = brute_force(ix.dataset, q, k, metric)
    if metric == 4:  # Hamming distances tie heavily: compare distance multisets
        assert np.array_equal(np.sort(d, axis=1), np.sort(bd, axis=1))
        return
    assert np.array_equal(_bits(d), _bits(bd))
    assert np.array_equal(ids, bids)


def test_f16_conversion_matches_ieee_round_to_nearest_even():
    lib = oracle_lib()
    rng = np.random.default_rng(7)
    special = np.array([0.0, -0.0, 1.0, 65504.0, 65519.99, 65520.0, 1e6, -1e6, 6.0e-8, 5.96e-8,
                        2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 3 * 2.0 ** -26, 2.0 ** -14,
                        2.0 ** -14 * (1 - 2.0 ** -11), 1e-40, np.inf, -np.inf, 0.1, 1 / 3],
                       dtype=np.float32)
    vals = np.concatenate([special,
                           (rng.standard_normal(20000) * np.exp(rng.uniform(-25, 12, 20000)))
                           .astype(np.float32),
                           rng.integers(0, 2**31, 20000, dtype=np.uint32).view(np.float32)])
    vals = vals[~np.isnan(vals)]
    got = np.array([lib.oracle_f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    back = np.array([lib.oracle_f16_to_f32(int(h)) for h in want], dtype=np.float32)
    assert np.array_equal(_bits(back), _bits(want.view(np.float16).astype(np.float32)))
    nan16 = lib.oracle_f32_to_f16(float("nan"))
    assert (nan16 & 0x7C00) == 0x7C00 and (nan16 & 0x3FF) != 0


def test_checks_catch_a_contracted_oracle(ref_cases, tmp_path):
    """Planted mistake on the CPU: an ADC/LUT computed with fused multiply-add
    (one rounding for t*t + s) or summed pairwise must disagree with the
    reference answers somewhere, which is what makes the bit-exact checks above
    meaningful."""
    manifest, arrays = ref_cases
    case = next(c for c in manifest if c["name"] == "mid8")
    ix = read_ipq1(write_case_ipq1(case, arrays, tmp_path))
    orc = Oracle(ix)
    q = arrays["mid8/queries"][:16]
    probes = orc.probes(q, 8)
    mismatches = 0
    for qi in range(len(q)):
        for l in probes[qi][:2]:
            exact = orc.lut(q[qi], int(l))
            r = (q[qi] - ix.centroids[l]).astype(np.float64).reshape(ix.pq_m, 1, ix.dsub)
            fused = ((r - ix.codebooks.astype(np.float64)) ** 2).sum(-1).astype(np.float32)
            mismatches += int(np.count_nonzero(_bits(fused) != _bits(exact)))
    assert mismatches > 0


def test_ipq1_writer_round_trips_reference_files(ref_cases, tmp_path):
    """Ipq1.to_bytes (used to write indexes with hand-made centroids) reproduces
    every reference-written file byte for byte."""
    manifest, arrays = ref_cases
    for case in manifest:
        raw = arrays[f"{case['name']}/ipq1"].tobytes()
        ix = read_ipq1(write_case_ipq1(case, arrays, tmp_path))
        assert ix.to_bytes() == raw, case["name"]
    legacy = (GOLDEN / "legacy_ipq1_v1.bin").read_bytes()
    p = tmp_path / "legacy.ipq1"
    p.write_bytes(legacy)
    assert read_ipq1(p).to_bytes() == legacy


# ---- ScaNN-style index (reference src/neighbors/graphs.cpp:3286-3374) ----

def scann_cases():
    import json

    manifest = json.loads((GOLDEN / "scann_cases.json").read_text())
    arrays = np.load(GOLDEN / "scann_cases.npz")
    return manifest, {k: arrays[k] for k in arrays.files}


def _scann_inputs(case):
    return lcg_data(*case["data_lcg"]), lcg_data(*case["queries_lcg"])


def _inner_oracle(case, arrays, tmp_path):
    p = tmp_path / f"{case['name']}_inner.ipq1"
    p.write_bytes(arrays[f"{case['name']}/inner_ipq1"].tobytes())
    return Oracle(read_ipq1(p))


def test_scann_aniso_closed_forms():
    """Columns whose mean and population variance are exact in fp32: a constant
    column (variance 0, so the factor is sqrt(1e-6)), two- and four-valued columns,
    one far from zero (the mean must be subtracted) and one centred at zero. A
    sample variance (n - 1), a dropped 1e-6 or a missing centring fails."""
    n = 8
    x = np.zeros((n, 5), np.float32)
    x[:, 0] = 3.0
    x[:, 1] = np.tile([0.0, 2.0], n // 2)
    x[:, 2] = np.tile([1.0, 2.0, 3.0, 4.0], n // 4)
    x[:, 3] = 1000.0 + np.tile([0.0, 1.0], n // 2)
    x[:, 4] = np.tile([-2.0, 0.0, 0.0, 2.0], n // 4)
    var = np.array([0.0, 1.0, 1.25, 0.25, 2.0], np.float32)
    want = np.sqrt(var + np.float32(1e-6)).astype(np.float32)
    assert np.array_equal(_bits(scann_aniso(x)), _bits(want))
    # One row: variance 0 over max(n, 1) = 1.
    assert np.array_equal(_bits(scann_aniso(x[:1])), _bits(np.full(5, want[0], np.float32)))


def test_scann_aniso_tracks_float64_statistics():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((3000, 12)) * np.linspace(0.1, 8.0, 12) + 3.0).astype(np.float32)
    a = scann_aniso(x)
    want = np.sqrt(x.astype(np.float64).var(axis=0) + 1e-6)
    assert np.allclose(a, want, rtol=2e-5, atol=0)


def test_scann_oracle_reproduces_reference_answers(tmp_path):
    """The oracle's ScaNN search over the fixture's inner index (the reference's
    IVF-PQ build of the rows scaled by the oracle's factors) gives the reference
    ScaNN's own answers bit for bit, so both the factors and the re-rank agree."""
    manifest, arrays = scann_cases()
    checked = 0
    for case in manifest:
        data, q = _scann_inputs(case)
        aniso = scann_aniso(data)
        orc = _inner_oracle(case, arrays, tmp_path)
        assert np.array_equal(_bits(orc.ix.dataset), _bits(data * aniso[None, :])), case["name"]
        for j, s in enumerate(case["searches"]):
            key = f"{case['name']}/s{j}"
            assert s["rc"] == 0, key
            if s["k"] == 0:
                continue
            ids, d = orc.scann_search(data, aniso, q, s["k"], s["nprobe"], s["krefine"])
            assert np.array_equal(ids, arrays[f"{key}/ids"]), key
            assert np.array_equal(_bits(d), _bits(arrays[f"{key}/dists"])), key
            checked += 1
    assert checked >= 10


def test_scann_full_probe_full_refine_is_brute_force(tmp_path):
    """The reference test's closed form (tests/test_neighbors.cpp:2958-2967): every
    list probed and krefine = n make the search exact nearest neighbours of the
    original rows."""
    manifest, arrays = scann_cases()
    case = next(c for c in manifest if c["name"] == "ref_b")
    data, q = _scann_inputs(case)
    orc = _inner_oracle(case, arrays, tmp_path)
    ids, d = orc.scann_search(data, scann_aniso(data), q, 4, case["nlist"], data.shape[0])
    bids, bd = brute_force(data, q, 4, 0)
    assert np.array_equal(ids, bids) and np.array_equal(_bits(d), _bits(bd))


@pytest.mark.skipif(not REF_SO.exists(), reason="oracle/_ref not built")
@pytest.mark.parametrize("seed", [1, 2])
def test_scann_oracle_matches_live_reference(seed, tmp_path):
    rng = np.random.default_rng(100 + seed)
    ref = Reference()
    dim = int(rng.choice([8, 16, 24]))
    pq_m = int(rng.choice([d for d in (2, 4, 8) if dim % d == 0]))
    n = int(rng.integers(300, 1200))
    nlist = int(rng.integers(2, 24))
    metric = int(rng.choice([0, 1, 2, 3, 5]))
    data = (rng.standard_normal((n, dim)) * rng.uniform(0.2, 5.0, dim)).astype(np.float32)
    q = (rng.standard_normal((11, dim)) * rng.uniform(0.2, 5.0, dim)).astype(np.float32)
    rc, h = ref.scann_build(data, metric, nlist, pq_m)
    assert rc == 0
    aniso = scann_aniso(data)
    rc, inner = ref.build(data * aniso[None, :], metric, nlist, pq_m, 8)
    assert rc == 0
    path = tmp_path / "inner.ipq1"
    assert ref.save(inner, path) == 0
    orc = Oracle(read_ipq1(path))
    for k, nprobe, krefine in [(10, 3, 30), (6, nlist, 4), (12, 1, 12)]:
        rc, rids, rd = ref.scann_search(h, q, k, nprobe, krefine)
        assert rc == 0
        oids, od = orc.scann_search(data, aniso, q, k, nprobe, krefine)
        assert np.array_equal(oids, rids)
        assert np.array_equal(_bits(od), _bits(rd))
    ref.scann_destroy(h)
    ref.destroy(inner)
    ref.close()


def test_ipq1_stream_reader_matches_file_reader(ref_cases, tmp_path):
    """The streaming IPQ1 reader (bench.py's C5 parity path: the index serialized
    into a pipe, the dataset section dropped and replaced by the rows in memory)
    yields the same index as the file reader."""
    import io

    from oracle.pyoracle import read_ipq1_stream

    manifest, arrays = ref_cases
    for case in manifest:
        raw = arrays[f"{case['name']}/ipq1"].tobytes()
        p = tmp_path / "c.ipq1"
        p.write_bytes(raw)
        a = read_ipq1(p)
        b = read_ipq1_stream(io.BytesIO(raw), a.dataset.copy())
        assert b.to_bytes() == raw, case["name"]
    with pytest.raises(ValueError):
        read_ipq1_stream(io.BytesIO(raw[:-3]), a.dataset.copy())
