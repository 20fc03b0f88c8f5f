"""GPU parity: libovvs on the MI355X against the reference and the oracle.

Bar (north star): neighbor ids identical to the reference's, distances within
1e-4 relative for fp32 tables (2e-3 for binary16 table requests, which are
served with fp32 entries); every comparison here also checks that the results
are bit-identical, which is what the kernels are built for (separately rounded
fp32 in the reference's order).
"""

from __future__ import annotations

import ctypes
import sys
import threading

import numpy as np
import pytest

from conftest import assert_results_match, case_data, write_case_ipq1
from oracle.pyoracle import REF_SO, Oracle, Reference, read_ipq1

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


# The LP metric re-ranks with glibc powf(|t|, 2) and powf(s, 0.5) on the
# reference side (reference internal.hpp:262-268); the kernel evaluates the
# correctly rounded t*t and sqrt(s), which powf (error bound 0.82 ulp) can miss
# by one ulp. LP distances are therefore held to the tolerance bar only.
METRIC_LP = 5


def assert_bits_unless_lp(metric, got, want, label):
    if metric != METRIC_LP:
        assert np.array_equal(_bits(got), _bits(want)), label


def test_reference_cases_bit_exact(ovvs, res, ref_cases, tmp_path):
    manifest, arrays = ref_cases
    for case in manifest:
        say("case", case["name"])
        ix = ovvs.neighbors.ivf_pq.load(write_case_ipq1(case, arrays, tmp_path), resources=res)
        q = arrays[f"{case['name']}/queries"]
        for j, s in enumerate(case["searches"]):
            key = f"{case['name']}/s{j}"
            ids, d = ix.search(q, s["k"], s["nprobe"], s["krefine"],
                               bitset=arrays.get(f"{key}/bitset"))
            assert_results_match(ids, d, arrays[f"{key}/ids"], arrays[f"{key}/dists"], label=key)
            assert_bits_unless_lp(case["metric"], d, arrays[f"{key}/dists"], key)
        ix.close()


def test_legacy_ipq1_on_gpu(ovvs, res):
    from conftest import GOLDEN

    ix = ovvs.neighbors.ivf_pq.load(GOLDEN / "legacy_ipq1_v1.bin", resources=res)
    ids, d = ix.search(np.array([[1.1, 0.0]], np.float32), k=2, nprobe=1, krefine=4)
    assert ids.tolist() == [[1, 2]]
    assert abs(d[0, 0] - 0.01) < 1e-5 and abs(d[0, 1] - 0.81) < 1e-5


def test_gpu_build_matches_reference_build_bytes(ovvs, res, ref_cases, tmp_path):
    """ovvsIvfPqBuild (+Extend) on the GPU against the reference's own build on the
    same inputs: k-means seeding, assignment, row-order means and encoding are
    reproduced exactly, so the serialized indexes must be byte-identical."""
    manifest, arrays = ref_cases
    for case in manifest:
        data = case_data(case, arrays)
        say("build", case["name"], data.shape)
        ix = ovvs.neighbors.ivf_pq.build(data, metric=case["metric"], nlist=case["nlist"],
                                         pq_m=case["pq_m"], pq_nbits=case["nbits"], resources=res)
        if case["extended"]:
            ix.extend(case_data(case, arrays, "extra"))
        out = tmp_path / "ours.ipq1"
        ix.serialize(out)
        ours = read_ipq1(out)
        theirs = read_ipq1(write_case_ipq1(case, arrays, tmp_path))
        assert np.array_equal(_bits(ours.centroids), _bits(theirs.centroids)), case["name"]
        assert np.array_equal(_bits(ours.codebooks), _bits(theirs.codebooks)), case["name"]
        assert np.array_equal(ours.assign, theirs.assign), case["name"]
        assert np.array_equal(ours.codes, theirs.codes), case["name"]
        assert out.read_bytes() == arrays[f"{case['name']}/ipq1"].tobytes(), case["name"]
        ix.close()


def test_fp16_requests_return_the_reference_results(ovvs, res, ref_cases, tmp_path):
    """A binary16 table request is served with fp32 entries: the results are the
    reference's own, bit for bit (the scan stores no table, so binary16 entries
    would only change the ranking)."""
    manifest, arrays = ref_cases
    for name in ("mid8", "mid4", "metric0", "metric2", "filters"):
        case = next(c for c in manifest if c["name"] == name)
        say("fp16 request", name)
        path = write_case_ipq1(case, arrays, tmp_path)
        orc = Oracle(read_ipq1(path))
        ix = ovvs.neighbors.ivf_pq.load(path, resources=res)
        q = arrays[f"{name}/queries"]
        for j, s in enumerate(case["searches"]):
            bits = arrays.get(f"{name}/s{j}/bitset")
            ids, d = ix.search_ex(q, s["k"], s["nprobe"], s["krefine"], bitset=bits,
                                  lut_dtype=ovvs.DTYPE_F16)
            oids, od = orc.search(q, s["k"], s["nprobe"], s["krefine"], bits)
            assert_results_match(ids, d, oids, od, rel=2e-3, label=f"{name}/s{j}")
            assert_bits_unless_lp(case["metric"], d, od, f"{name}/s{j}")
            assert np.array_equal(ids, arrays[f"{name}/s{j}/ids"]), f"{name}/s{j}"
        ix.close()
    assert res.last_compute_dtype() == ovvs.DTYPE_F32


def test_fp16_request_with_entries_beyond_binary16_range(ovvs, res, tmp_path):
    """Data whose table entries exceed 65504, the largest binary16 value: a
    binary16 table would hold +inf there. The search returns the reference's
    fp32 results whatever precision is requested."""
    rng = np.random.default_rng(31)
    dim, n, nlist, pq_m = 16, 4000, 8, 8
    centers = (400.0 * rng.standard_normal((8, dim))).astype(np.float32)
    data = (centers[rng.integers(0, 8, n)] + 150.0 * rng.standard_normal((n, dim))).astype(
        np.float32)
    q = (centers[rng.integers(0, 8, 200)] + 150.0 * rng.standard_normal((200, dim))).astype(
        np.float32)
    ix = ovvs.neighbors.ivf_pq.build(data, nlist=nlist, pq_m=pq_m, pq_nbits=8, resources=res)
    p = tmp_path / "wide.ipq1"
    ix.serialize(p)
    orc = Oracle(read_ipq1(p))
    # The probed lists' tables do reach past the binary16 range.
    probes = orc.probes(q[:20], 4)
    big = max(float(orc.lut(q[i], int(probes[i, j])).max()) for i in range(20) for j in range(4))
    say("largest table entry of the probed lists", big)
    assert big > 65504.0
    oids, od = orc.search(q, 10, 4, 32)
    for dt in (ovvs.DTYPE_F32, ovvs.DTYPE_F16):
        ids, d = ix.search_ex(q, 10, 4, 32, lut_dtype=dt)
        assert np.array_equal(ids, oids), dt
        assert np.array_equal(_bits(d), _bits(od)), dt
    if REF_SO.exists():
        ref = Reference()
        rc, h = ref.load(p)
        assert rc == 0
        rc, rids, rd = ref.search(h, q, 10, 4, 32)
        assert rc == 0 and np.array_equal(rids, oids) and np.array_equal(_bits(rd), _bits(od))
        ref.destroy(h)
        ref.close()
    ix.close()


def test_random_indexes_against_oracle(ovvs, res, tmp_path):
    rng = np.random.default_rng(11)
    for trial in range(6):
        dim = int(rng.choice([8, 16, 24, 48, 96]))
        pq_m = int(rng.choice([d for d in (1, 2, 3, 4, 8, 12, 16, 24, 32, 48) if dim % d == 0]))
        n = int(rng.integers(500, 6000))
        nlist = int(rng.integers(4, 96))
        nbits = int(rng.choice([4, 5, 8]))
        metric = int(rng.integers(0, 6))
        say("trial", trial, dict(n=n, dim=dim, pq_m=pq_m, nlist=nlist, nbits=nbits, metric=metric))
        centers = rng.standard_normal((32, dim)).astype(np.float32)
        data = (centers[rng.integers(0, 32, n)] +
                0.3 * rng.standard_normal((n, dim))).astype(np.float32)
        q = (centers[rng.integers(0, 32, 100)] +
             0.3 * rng.standard_normal((100, dim))).astype(np.float32)
        ix = ovvs.neighbors.ivf_pq.build(data, metric=metric, nlist=nlist, pq_m=pq_m,
                                         pq_nbits=nbits, resources=res)
        p = tmp_path / "rand.ipq1"
        ix.serialize(p)
        orc = Oracle(read_ipq1(p))
        bitset = np.packbits((rng.random(n) < 0.7).astype(np.uint8), bitorder="little")
        for k, nprobe, krefine, bits in [(10, 8, 10, None), (10, 4, 64, None), (1, 1, 1, None),
                                         (32, nlist, 200, None), (10, 6, 40, bitset),
                                         (256, 3, 256, None), (20, 5, 700, None)]:
            ids, d = ix.search(q, k, nprobe, krefine, bitset=bits)
            oids, od = orc.search(q, k, nprobe, krefine, bits)
            assert_results_match(ids, d, oids, od, label=f"trial{trial} k{k} p{nprobe} r{krefine}")
            assert_bits_unless_lp(metric, d, od, f"trial{trial}")
        ix.close()


def test_multi_chunk_lists_against_oracle(ovvs, res, tmp_path):
    """Lists of several thousand rows hold dozens of segments (several bound
    passes of 16), phase 0 spans whole large lists, and a tight shortlist
    (k = krefine = 10) prunes most segments. Results must match the oracle on
    every one of several repeats."""
    rng = np.random.default_rng(23)
    dim, n, nlist = 32, 60000, 8
    centers = rng.standard_normal((16, dim)).astype(np.float32)
    data = (centers[rng.integers(0, 16, n)] + 0.3 * rng.standard_normal((n, dim))).astype(
        np.float32)
    q = (centers[rng.integers(0, 16, 2000)] + 0.3 * rng.standard_normal((2000, dim))).astype(
        np.float32)
    ix = ovvs.neighbors.ivf_pq.build(data, nlist=nlist, pq_m=16, pq_nbits=8, resources=res)
    p = tmp_path / "chunks.ipq1"
    ix.serialize(p)
    orc = Oracle(read_ipq1(p))
    assert max(len(l) for l in orc.ix.lists) > 3 * 2048
    oids, od = orc.search(q, 10, 4, 10)
    for rep in range(3):
        say("multi-chunk repeat", rep)
        ids, d = ix.search(q, 10, 4, 10)
        assert_results_match(ids, d, oids, od, label=f"repeat {rep}")
        assert np.array_equal(_bits(d), _bits(od)), f"repeat {rep}"
    ix.close()


def test_ties_across_segments_keep_reference_order(ovvs, res, tmp_path):
    """300 exact copies of one vector sit in one list, split over several segments
    the scan visits in bound order; queries at and near the copy make the K-th
    score a tie shared by every copy, so only the in-list ordinal decides which
    copies are returned. Pruning compares strictly (a row is dropped only when its
    bound exceeds the K-th score), so the result must be the reference's."""
    rng = np.random.default_rng(31)
    dim, n = 32, 4000
    centers = rng.standard_normal((8, dim)).astype(np.float32)
    data = (centers[rng.integers(0, 8, n)] + 0.3 * rng.standard_normal((n, dim))).astype(np.float32)
    v = data[17].copy()
    dup = rng.choice(n, 300, replace=False)
    data[dup] = v
    q = np.vstack([np.repeat(v[None], 8, 0),
                   v[None] + 0.01 * rng.standard_normal((24, dim)).astype(np.float32)]).astype(np.float32)
    ix = ovvs.neighbors.ivf_pq.build(data, nlist=6, pq_m=8, pq_nbits=8, resources=res)
    p = tmp_path / "ties.ipq1"
    ix.serialize(p)
    orc = Oracle(read_ipq1(p))
    for k, nprobe, krefine in [(10, 2, 10), (50, 3, 120), (1, 1, 1), (200, 6, 400)]:
        ids, d = ix.search(q, k, nprobe, krefine)
        oids, od = orc.search(q, k, nprobe, krefine)
        assert np.array_equal(ids, oids), f"k{k} p{nprobe} r{krefine}"
        assert np.array_equal(_bits(d), _bits(od)), f"k{k} p{nprobe} r{krefine}"
    if REF_SO.exists():
        ref = Reference()
        rc, h = ref.load(p)
        assert rc == 0
        rc, rids, rd = ref.search(h, q, 10, 2, 10)
        ids, d = ix.search(q, 10, 2, 10)
        assert rc == 0 and np.array_equal(ids, rids) and np.array_equal(_bits(d), _bits(rd))
        ref.destroy(h)
        ref.close()
    ix.close()


def test_far_from_origin_data_against_oracle(ovvs, res, tmp_path):
    """Vectors around +1000 in every coordinate: the segment boxes (absolute
    coordinates, binary16 rounded outward) are coarse there and the residual
    rounding allowance is at its largest; pruning must stay exact."""
    rng = np.random.default_rng(37)
    dim, n = 48, 8000
    centers = (1000.0 + rng.standard_normal((24, dim))).astype(np.float32)
    data = (centers[rng.integers(0, 24, n)] + 0.2 * rng.standard_normal((n, dim))).astype(np.float32)
    q = (centers[rng.integers(0, 24, 300)] + 0.2 * rng.standard_normal((300, dim))).astype(np.float32)
    ix = ovvs.neighbors.ivf_pq.build(data, nlist=24, pq_m=24, pq_nbits=8, resources=res)
    p = tmp_path / "far.ipq1"
    ix.serialize(p)
    orc = Oracle(read_ipq1(p))
    for k, nprobe, krefine in [(10, 6, 10), (10, 24, 64)]:
        ids, d = ix.search(q, k, nprobe, krefine)
        oids, od = orc.search(q, k, nprobe, krefine)
        assert_results_match(ids, d, oids, od, label=f"k{k} p{nprobe}")
        assert np.array_equal(_bits(d), _bits(od)), f"k{k} p{nprobe}"
    ix.close()


def test_many_groups_and_odd_batches_against_oracle(ovvs, res, tmp_path):
    """Four lists of about 60,000 rows hold hundreds of segment groups each, so one
    query's groups exceed what the scan holds in LDS at a time (several item
    rounds) and phase 0's per-list candidate cap; batches of 1, 7 and 13 queries
    take the XCD-aware query order with a batch that is not a multiple of 8."""
    rng = np.random.default_rng(41)
    dim, n = 16, 240000
    centers = rng.standard_normal((64, dim)).astype(np.float32)
    data = (centers[rng.integers(0, 64, n)] + 0.3 * rng.standard_normal((n, dim))).astype(np.float32)
    ix = ovvs.neighbors.ivf_pq.build(data, nlist=4, pq_m=8, pq_nbits=8, resources=res)
    p = tmp_path / "groups.ipq1"
    ix.serialize(p)
    orc = Oracle(read_ipq1(p))
    assert min(len(l) for l in orc.ix.lists) > 20000
    for nq in (1, 7, 13, 64):
        q = (centers[rng.integers(0, 64, nq)] + 0.3 * rng.standard_normal((nq, dim))).astype(np.float32)
        for k, nprobe, krefine in [(10, 4, 10), (10, 3, 32), (100, 4, 100)]:
            say("nq", nq, "k", k, "nprobe", nprobe)
            ids, d = ix.search(q, k, nprobe, krefine)
            oids, od = orc.search(q, k, nprobe, krefine)
            assert_results_match(ids, d, oids, od, label=f"nq{nq} k{k} p{nprobe}")
            assert np.array_equal(_bits(d), _bits(od)), f"nq{nq} k{k} p{nprobe}"
    ix.close()


def test_limits_against_oracle(ovvs, res, tmp_path):
    """The largest shortlist the kernels hold (krefine = k = 1024, more than the
    probed rows: -1 / +inf padding) and probe counts in the thousands (2048 of 2048
    lists, nprobe 4096 clamped to nlist), bit-identical to the oracle."""
    rng = np.random.default_rng(23)
    n, dim, nlist = 30000, 16, 2048
    centers = rng.standard_normal((64, dim)).astype(np.float32)
    data = (centers[rng.integers(0, 64, n)] + 0.3 * rng.standard_normal((n, dim))).astype(np.float32)
    q = (centers[rng.integers(0, 64, 20)] + 0.3 * rng.standard_normal((20, dim))).astype(np.float32)
    say("limits build", n, dim, nlist)
    ix = ovvs.neighbors.ivf_pq.build(data, metric=0, nlist=nlist, pq_m=4, pq_nbits=8, resources=res)
    p = tmp_path / "limits.ipq1"
    ix.serialize(p)
    orc = Oracle(read_ipq1(p))
    for k, nprobe, krefine in [(1024, 64, 1024), (10, 2048, 10), (100, 4096, 1000), (5, 1500, 1024)]:
        say("limits search", k, nprobe, krefine)
        ids, d = ix.search(q, k, nprobe, krefine)
        oids, od = orc.search(q, k, nprobe, krefine)
        assert np.array_equal(ids, oids), (k, nprobe, krefine)
        assert np.array_equal(_bits(d), _bits(od)), (k, nprobe, krefine)
        if k == 1024 and nprobe == 64:
            # 64 lists of about 15 rows: the padded tail is part of what was compared.
            assert np.any(oids[:, -1] == -1)
    ix.close()


def test_device_pointer_entry_matches_host_entry(ovvs, res, ref_cases, tmp_path):
    import torch

    manifest, arrays = ref_cases
    case = next(c for c in manifest if c["name"] == "mid8")
    ix = ovvs.neighbors.ivf_pq.load(write_case_ipq1(case, arrays, tmp_path), resources=res)
    q = arrays["mid8/queries"]
    ids, d = ix.search(q, 10, 8, 32)
    dq = torch.from_numpy(q).to("cuda:0")
    did = torch.empty((q.shape[0], 10), dtype=torch.int64, device="cuda:0")
    dd = torch.empty((q.shape[0], 10), dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    ix.search_device(dq.data_ptr(), q.shape[0], 10, 8, 32, did.data_ptr(), dd.data_ptr())
    assert np.array_equal(did.cpu().numpy(), ids)
    assert np.array_equal(_bits(dd.cpu().numpy()), _bits(d))
    ix.close()


def test_batch_independence_and_determinism(ovvs, res, ref_cases, tmp_path):
    manifest, arrays = ref_cases
    case = next(c for c in manifest if c["name"] == "mid8")
    ix = ovvs.neighbors.ivf_pq.load(write_case_ipq1(case, arrays, tmp_path), resources=res)
    q = arrays["mid8/queries"]
    full_ids, full_d = ix.search(q, 10, 8, 32)
    same = np.repeat(q[:1], 33, axis=0)
    ids33, d33 = ix.search(same, 10, 8, 32)
    assert np.all(ids33 == full_ids[0]) and np.all(_bits(d33) == _bits(full_d[0]))
    for lo, hi in [(0, 1), (5, 37), (37, 64)]:
        ids, d = ix.search(q[lo:hi], 10, 8, 32)
        assert np.array_equal(ids, full_ids[lo:hi])
    again_ids, again_d = ix.search(q, 10, 8, 32)
    assert np.array_equal(again_ids, full_ids) and np.array_equal(_bits(again_d), _bits(full_d))
    ix.close()


def test_concurrent_searches_share_one_index(ovvs, ref_cases, tmp_path):
    manifest, arrays = ref_cases
    case = next(c for c in manifest if c["name"] == "mid8")
    path = write_case_ipq1(case, arrays, tmp_path)
    owner = ovvs.Resources()
    ix = ovvs.neighbors.ivf_pq.load(path, resources=owner)
    q = arrays["mid8/queries"]
    want = ix.search(q, 10, 8, 32)
    results = {}

    def worker(t):
        r = ovvs.Resources()
        h = ix._h
        ids = np.empty((q.shape[0], 10), np.int64)
        d = np.empty((q.shape[0], 10), np.float32)
        rcs = []
        for _ in range(5):
            rcs.append(ovvs._lib.ovvsIvfPqSearch(
                r._h, h, q.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), q.shape[0], 10, 8, 32,
                None, ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                d.ctypes.data_as(ctypes.POINTER(ctypes.c_float))))
        results[t] = (rcs, ids.copy(), d.copy())
        r.close()

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    for rcs, ids, d in results.values():
        assert rcs == [0] * 5
        assert np.array_equal(ids, want[0]) and np.array_equal(_bits(d), _bits(want[1]))
    ix.close()


def test_telemetry_counts_and_failure_atomicity(ovvs, res, ref_cases, tmp_path):
    manifest, arrays = ref_cases
    case = next(c for c in manifest if c["name"] == "mid8")
    path = write_case_ipq1(case, arrays, tmp_path)
    r = ovvs.Resources()
    ix = ovvs.neighbors.ivf_pq.load(path, resources=r)
    orc = Oracle(read_ipq1(path))
    q = arrays["mid8/queries"]
    before = r.ivfpq_search_stats()
    ix.search(q, 10, 8, 32)
    after = r.ivfpq_search_stats()
    probes = orc.probes(q, 8)
    sizes = np.diff(orc.offsets)
    rows = int(sizes[probes].sum())
    tasks = int((sizes[probes] > 0).sum())
    assert after["successful_calls"] - before["successful_calls"] == 1
    assert after["queries"] - before["queries"] == q.shape[0]
    assert after["candidate_rows"] - before["candidate_rows"] == rows
    assert after["tasks"] - before["tasks"] == tasks
    assert after["selected_rows"] - before["selected_rows"] == q.shape[0] * 32
    assert after["adc_scan_select_ns"] > before["adc_scan_select_ns"]
    assert after["gpu_kernel_launches"] > before["gpu_kernel_launches"]
    assert r.last_device() == ovvs.DEVICE_GPU
    with pytest.raises(ovvs.OvvsError):
        ix.search(q, 10, 8, 5000)  # krefine beyond the register list
    assert r.ivfpq_search_stats() == after
    ix.close()


def test_stage_times_for_small_and_large_batches(ovvs, tmp_path):
    """Stage times come from the launches' device-clock stamps: batches under 256
    queries take the refine's end from its last workgroup (no events), larger ones
    from an event pair around the search. Either way every stage is counted and the
    stages fit inside the call's host wall time; results do not depend on the path."""
    rng = np.random.default_rng(5)
    dim, n = 32, 20000
    centers = rng.standard_normal((64, dim)).astype(np.float32)
    data = (centers[rng.integers(0, 64, n)] + 0.3 * rng.standard_normal((n, dim))).astype(np.float32)
    q = (centers[rng.integers(0, 64, 600)] + 0.3 * rng.standard_normal((600, dim))).astype(np.float32)
    r = ovvs.Resources()
    ix = ovvs.neighbors.ivf_pq.build(data, nlist=128, pq_m=16, pq_nbits=8, resources=r)
    stages = ["coarse_pairwise_ns", "coarse_topk_ns", "adc_scan_select_ns", "refine_distance_ns"]
    whole_ids, whole_d = ix.search(q, 10, 16, 32)
    for nq in (1, 100, 255, 256, 600):
        say("stage times", nq)
        before = r.ivfpq_search_stats()
        ids, d = ix.search(q[:nq], 10, 16, 32)
        after = r.ivfpq_search_stats()
        delta = {k: after[k] - before[k] for k in stages + ["total_wall_ns"]}
        for k in stages:
            assert delta[k] > 0, (nq, k, delta)
        assert sum(delta[k] for k in stages) <= delta["total_wall_ns"], (nq, delta)
        assert np.array_equal(ids, whole_ids[:nq]) and np.array_equal(_bits(d), _bits(whole_d[:nq]))
    ix.close()


@pytest.mark.skipif(not REF_SO.exists(), reason="oracle/_ref not built")
def test_c1_scale_against_reference(ovvs, res, tmp_path):
    """Config 1 (100k x 128, 256 lists, pq 32, 16 probes, k 10, fp32 tables): the
    quantizers are trained on the 20k-row prefix, the rest is appended with
    extend; the reference library searches the same serialized index."""
    from ovvs_amd import synth

    cfg = synth.CONFIGS["c1"]
    C = synth.centers(cfg)
    data = synth.base_rows(cfg, 0, cfg.n, C)
    q = synth.query_rows(cfg, 0, 200, C)
    say("c1 build")
    ix = ovvs.neighbors.ivf_pq.build(data[:cfg.train_rows], nlist=cfg.nlist, pq_m=cfg.pq_m,
                                     resources=res)
    ix.extend(data[cfg.train_rows:])
    p = tmp_path / "c1.ipq1"
    ix.serialize(p)
    say("c1 search")
    ids, d = ix.search(q, cfg.k, cfg.nprobe, cfg.k)
    ref = Reference()
    rc, h = ref.load(p)
    assert rc == 0
    rc, rids, rd = ref.search(h, q, cfg.k, cfg.nprobe, cfg.k)
    assert rc == 0
    assert_results_match(ids, d, rids, rd, label="c1")
    assert np.array_equal(_bits(d), _bits(rd))
    ref.destroy(h)
    ref.close()
    ix.close()


def test_extend_is_transactional(ovvs, res, tmp_path):
    """The reference's transactional-extend contract (reference
    tests/test_neighbors.cpp:1427-1524, src/neighbors/indexes.cpp:1320-1427): a
    failed extend leaves the serialized bytes and the search results unchanged;
    after a successful one every extended row is its own nearest neighbour at
    distance < 1e-5, and the extended index survives a reload byte for byte."""
    from ovvs_amd.synth import lcg_data

    n, dim, nq, k, nlist, pq_m = 64, 8, 4, 4, 8, 4
    data = lcg_data(n, dim, 218)
    extra = lcg_data(nq, dim, 219)
    ix = ovvs.neighbors.ivf_pq.build(data, nlist=nlist, pq_m=pq_m, pq_nbits=4, resources=res)
    base_ids, base_d = ix.search(data[:nq], k, nlist, n)
    before = tmp_path / "before.ipq1"
    ix.serialize(before)
    before_bytes = before.read_bytes()

    failing = extra.copy()
    failing[0, 0] = np.nan
    res.set_policy(ovvs.POLICY_FORCE_NPU)
    try:
        with pytest.raises(ovvs.OvvsError) as err:
            ix.extend(failing)
        assert err.value.status == ovvs.STATUS_DEVICE_UNAVAILABLE
    finally:
        res.set_policy(ovvs.POLICY_AUTO)
    after = tmp_path / "after.ipq1"
    ix.serialize(after)
    assert after.read_bytes() == before_bytes, "failed extend changed the index"
    ids, d = ix.search(data[:nq], k, nlist, n)
    assert np.array_equal(ids, base_ids) and np.array_equal(_bits(d), _bits(base_d))

    ix.extend(extra)
    ext_ids, ext_d = ix.search(extra, 1, nlist, n + nq)
    assert np.array_equal(ext_ids[:, 0], np.arange(n, n + nq)), ext_ids
    assert np.all(np.abs(ext_d[:, 0]) < 1e-5), ext_d
    ix.serialize(after)
    re = ovvs.neighbors.ivf_pq.load(after, resources=res)
    r_ids, r_d = re.search(extra, 1, nlist, n + nq)
    assert np.array_equal(r_ids, ext_ids) and np.array_equal(_bits(r_d), _bits(ext_d))
    again = tmp_path / "again.ipq1"
    re.serialize(again)
    assert again.read_bytes() == after.read_bytes(), "extended IPQ1 not byte stable"
    if REF_SO.exists():
        ref = Reference()
        rc, h = ref.build(data, 0, nlist, pq_m, 4)
        assert rc == 0
        assert ref.extend(h, extra) == 0
        ref_path = tmp_path / "ref.ipq1"
        ref.save(h, ref_path)
        assert ref_path.read_bytes() == after.read_bytes(), "extended bytes differ from the reference's"
        ref.destroy(h)
        ref.close()
    re.close()
    ix.close()


def test_table_mode_unclustered_and_mixed_against_oracle(ovvs, res, tmp_path):
    """Queries whose lower bounds prune little (isotropic data, no clusters) are
    handed off by the bounded scan to the full-table scan (each probed list's whole
    table in LDS, every row scored); an index over clusters plus an isotropic
    background serves, in one batch, queries the bounds prune (from the clusters)
    and queries they do not (from the background). Both must match the oracle bit
    for bit, with filters and long shortlists too, and the isotropic searches must
    actually have taken the full-table scan."""
    rng = np.random.default_rng(41)
    dim = 32
    iso = rng.standard_normal((40000, dim)).astype(np.float32)
    q_iso = rng.standard_normal((300, dim)).astype(np.float32)
    ix = ovvs.neighbors.ivf_pq.build(iso, nlist=64, pq_m=16, pq_nbits=8, resources=res)
    p = tmp_path / "iso.ipq1"
    ix.serialize(p)
    orc = Oracle(read_ipq1(p))
    bitset = np.packbits((rng.random(40000) < 0.5).astype(np.uint8), bitorder="little")
    # Shortlists of 10, 64 and 128 keys take the per-wave scan (codebook in LDS), 129 and
    # 300 the whole-table scan.
    for k, nprobe, krefine, bits in [(10, 16, 10, None), (10, 32, 64, bitset), (100, 8, 300, None),
                                     (1, 64, 1, None), (10, 16, 128, bitset), (10, 16, 129, None)]:
        say("iso", dict(k=k, nprobe=nprobe, krefine=krefine, bitset=bits is not None))
        before = res.ivfpq_table_queries()
        ids, d = ix.search(q_iso, k, nprobe, krefine, bitset=bits)
        handed = res.ivfpq_table_queries() - before
        say("handed off", handed)
        if nprobe >= 16:
            assert handed > 0, "isotropic queries never reached the full-table scan"
        oids, od = orc.search(q_iso, k, nprobe, krefine, bits)
        assert_results_match(ids, d, oids, od, label=f"iso k{k} p{nprobe}")
        assert np.array_equal(_bits(d), _bits(od)), f"iso k{k} p{nprobe}"
    ix.close()

    # The other register layouts of the codebook (one, four and eight coordinates per
    # entry) and the table read from memory (dsub 16).
    for pq_m in (32, 8, 4, 2):
        say("iso pq_m", pq_m)
        ix = ovvs.neighbors.ivf_pq.build(iso[:20000], nlist=32, pq_m=pq_m, pq_nbits=8, resources=res)
        p = tmp_path / f"iso{pq_m}.ipq1"
        ix.serialize(p)
        orc = Oracle(read_ipq1(p))
        before = res.ivfpq_table_queries()
        ids, d = ix.search(q_iso[:100], 10, 16, 32)
        say("handed off", res.ivfpq_table_queries() - before)
        oids, od = orc.search(q_iso[:100], 10, 16, 32)
        assert_results_match(ids, d, oids, od, label=f"iso pq_m{pq_m}")
        assert np.array_equal(_bits(d), _bits(od)), f"iso pq_m{pq_m}"
        ix.close()

    centers = 4.0 * rng.standard_normal((32, dim)).astype(np.float32)
    clustered = (centers[rng.integers(0, 32, 30000)] +
                 0.2 * rng.standard_normal((30000, dim))).astype(np.float32)
    data = np.concatenate([clustered, 2.0 * iso[:30000]])
    q = np.concatenate([(centers[rng.integers(0, 32, 200)] +
                         0.2 * rng.standard_normal((200, dim))).astype(np.float32),
                        2.0 * q_iso[:200]])
    q = q[rng.permutation(len(q))]
    ix = ovvs.neighbors.ivf_pq.build(data, nlist=128, pq_m=16, pq_nbits=8, resources=res)
    p = tmp_path / "mixed.ipq1"
    ix.serialize(p)
    orc = Oracle(read_ipq1(p))
    for k, nprobe, krefine in [(10, 16, 10), (10, 48, 32)]:
        say("mixed", dict(k=k, nprobe=nprobe, krefine=krefine))
        before = res.ivfpq_table_queries()
        ids, d = ix.search(q, k, nprobe, krefine)
        say("handed off", res.ivfpq_table_queries() - before, "of", len(q))
        oids, od = orc.search(q, k, nprobe, krefine)
        assert_results_match(ids, d, oids, od, label=f"mixed k{k} p{nprobe}")
        assert np.array_equal(_bits(d), _bits(od)), f"mixed k{k} p{nprobe}"
    ix.close()
