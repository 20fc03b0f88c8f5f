"""C-ABI boundary tests that need no GPU.

They pin what a caller of the reference ABI relies on (reference
include/ovvs/ovvs.h, src/neighbors/indexes.cpp, tests/test_neighbors.cpp):
exported symbols, enum/struct layouts, status codes and their order of checks,
untouched outputs on failure, IPQ1 v1 compatibility and corruption handling.
"""

from __future__ import annotations

import ctypes
import re
from ctypes import POINTER, byref, c_float, c_int32, c_int64, c_uint8, c_void_p

import numpy as np
import pytest

from conftest import GOLDEN, ROOT, write_case_ipq1

HEADER = ROOT / "include" / "ovvs" / "ovvs.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"OVVS_API\s+[\w\s\*]+?\b(ovvs\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol(ovvs):
    syms = declared_symbols()
    assert len(syms) >= 20
    lib = ctypes.CDLL(str(ovvs.library_path()))
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing


def test_library_exports_nothing_undeclared(ovvs):
    import subprocess

    out = subprocess.run(["nm", "-D", "--defined-only", str(ovvs.library_path())],
                         capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    ours = {s for s in exported if s.startswith("ovvs")}
    assert ours == set(declared_symbols())


def test_version_and_status_strings(ovvs):
    assert ovvs.version() == "0.2.0"
    lib = ovvs._lib
    expected = {0: b"success", 1: b"error", 2: b"invalid argument", 3: b"unsupported",
                4: b"out of memory", 5: b"compile fail", 6: b"shape mismatch",
                7: b"device unavailable", 8: b"io error", 99: b"unknown"}
    for code, text in expected.items():
        assert lib.ovvsStatusString(code) == text


def test_stats_struct_layout(ovvs):
    s = ovvs._StatsV1
    assert ctypes.sizeof(s) == 200
    assert s.abi_version.offset == 0 and s.struct_size.offset == 4
    for i, name in enumerate(ovvs._STATS_FIELDS):
        assert getattr(s, name).offset == 8 + 8 * i


def test_fresh_stats_snapshot(ovvs):
    res = ovvs.Resources()
    st = res.ivfpq_search_stats()
    assert st["abi_version"] == 1 and st["struct_size"] == 200
    assert all(st[k] == 0 for k in ovvs._STATS_FIELDS)


def test_resources_policy_roundtrip(ovvs):
    res = ovvs.Resources()
    assert res.get_policy() == ovvs.POLICY_AUTO
    for p in range(7):
        res.set_policy(p)
        assert res.get_policy() == p
    lib = ovvs._lib
    assert lib.ovvsResourcesSetPolicy(None, 0) == ovvs.STATUS_INVALID_ARGUMENT
    assert lib.ovvsResourcesCreate(None) == ovvs.STATUS_INVALID_ARGUMENT
    v = c_int32(5)
    assert lib.ovvsResourcesNpuAvailable(res._h, byref(v)) == 0 and v.value == 0


def test_bitset_from_allow_list_matches_lsb_first_packing(ovvs):
    rng = np.random.default_rng(3)
    n = 203
    ids = rng.choice(n, 57, replace=False)
    got = ovvs.bitset_from_allow_list(n, list(ids) + [-1, n, n + 100])
    want = np.zeros(n, dtype=np.uint8)
    want[ids] = 1
    assert np.array_equal(got, np.packbits(want, bitorder="little"))
    lib = ovvs._lib
    buf = (c_uint8 * 4)()
    assert lib.ovvsBitsetFromAllowList(0, None, 0, buf) == ovvs.STATUS_INVALID_ARGUMENT
    assert lib.ovvsBitsetFromAllowList(8, None, -1, buf) == ovvs.STATUS_INVALID_ARGUMENT
    assert lib.ovvsBitsetFromAllowList(8, None, 0, None) == ovvs.STATUS_INVALID_ARGUMENT


def _load(ovvs, res, path):
    h = c_void_p(1)
    rc = ovvs._lib.ovvsIvfPqDeserialize(res._h, str(path).encode(), byref(h))
    return rc, h


def test_legacy_ipq1_roundtrip_is_byte_exact(ovvs, tmp_path):
    res = ovvs.Resources()
    src = GOLDEN / "legacy_ipq1_v1.bin"
    rc, h = _load(ovvs, res, src)
    assert rc == 0 and h.value
    out = tmp_path / "round.ipq1"
    assert ovvs._lib.ovvsIvfPqSerialize(h, str(out).encode()) == 0
    assert out.read_bytes() == src.read_bytes()
    ovvs._lib.ovvsIvfPqDestroy(h)


@pytest.mark.parametrize("edit,status", [
    ("version2", 3),       # UNSUPPORTED
    ("truncate", 8),       # IO
    ("id_out_of_range", 8),
    ("duplicate_id", 8),
    ("bad_magic", 8),
    ("extra_byte", 8),
    ("code_ge_ks", 8),
    ("assign_mismatch", 8),
])
def test_legacy_ipq1_corruption(ovvs, tmp_path, edit, status):
    blob = bytearray((GOLDEN / "legacy_ipq1_v1.bin").read_bytes())
    if edit == "version2":
        blob[4:8] = np.int32(2).tobytes()
    elif edit == "truncate":
        blob = blob[:-1]
    elif edit == "id_out_of_range":
        blob[236:244] = np.int64(4).tobytes()
    elif edit == "duplicate_id":
        blob[244:252] = np.int64(0).tobytes()
    elif edit == "bad_magic":
        blob[0] ^= 0xFF
    elif edit == "extra_byte":
        blob += b"\x00"
    elif edit == "code_ge_ks":
        blob[44 + 8 + 128] = 16          # first code byte; ks = 16
    elif edit == "assign_mismatch":
        blob[44 + 8 + 128 + 4 + 32: 44 + 8 + 128 + 4 + 36] = np.int32(1).tobytes()
    p = tmp_path / "corrupt.ipq1"
    p.write_bytes(bytes(blob))
    res = ovvs.Resources()
    rc, h = _load(ovvs, res, p)
    assert rc == status
    assert not h.value  # the handle is cleared on failure


def test_deserialize_argument_errors(ovvs, tmp_path):
    lib = ovvs._lib
    res = ovvs.Resources()
    h = c_void_p(1)
    assert lib.ovvsIvfPqDeserialize(res._h, str(tmp_path / "missing").encode(), byref(h)) == 8
    assert not h.value
    assert lib.ovvsIvfPqDeserialize(None, b"x", byref(h)) == ovvs.STATUS_INVALID_ARGUMENT
    assert lib.ovvsIvfPqDeserialize(res._h, None, byref(h)) == ovvs.STATUS_INVALID_ARGUMENT
    assert lib.ovvsIvfPqSerialize(None, b"x") == ovvs.STATUS_INVALID_ARGUMENT


def test_reference_built_indexes_roundtrip(ovvs, ref_cases, tmp_path):
    manifest, arrays = ref_cases
    res = ovvs.Resources()
    for case in manifest:
        src = write_case_ipq1(case, arrays, tmp_path)
        rc, h = _load(ovvs, res, src)
        assert rc == 0, case["name"]
        out = tmp_path / "again.ipq1"
        assert ovvs._lib.ovvsIvfPqSerialize(h, str(out).encode()) == 0
        assert out.read_bytes() == src.read_bytes(), case["name"]
        ovvs._lib.ovvsIvfPqDestroy(h)


def _search(ovvs, res, h, q, nq, k, nprobe, krefine, bitset=None, dtype=None):
    ids = np.full(max(nq * k, 1), 0x123456789ABCDEF, dtype=np.int64)
    d = np.full(max(nq * k, 1), -12345.25, dtype=np.float32)
    qp = None if q is None else np.ascontiguousarray(q, np.float32).ctypes.data_as(POINTER(c_float))
    args = (res._h if res else None, h, qp, c_int64(nq), c_int64(k), c_int32(nprobe),
            c_int32(krefine), bitset)
    outs = (ids.ctypes.data_as(POINTER(c_int64)), d.ctypes.data_as(POINTER(c_float)))
    if dtype is None:
        rc = ovvs._lib.ovvsIvfPqSearch(*args, *outs)
    else:
        rc = ovvs._lib.ovvsIvfPqSearchEx(*args, c_int32(dtype), *outs)
    untouched = bool(np.all(ids == 0x123456789ABCDEF) and np.all(d == np.float32(-12345.25)))
    return rc, untouched


def test_search_argument_checks_leave_outputs_untouched(ovvs):
    res = ovvs.Resources()
    rc, h = _load(ovvs, res, GOLDEN / "legacy_ipq1_v1.bin")
    assert rc == 0
    q = np.array([[1.1, 0.0]], dtype=np.float32)
    INV, SHAPE, UNSUP, DEV = 2, 6, 3, 7
    cases = [
        ((None, h, q, 1, 2, 1, 4), INV),           # null resources
        ((res, None, q, 1, 2, 1, 4), INV),         # null index
        ((res, h, None, 1, 2, 1, 4), INV),         # null queries
        ((res, h, q, 0, 2, 1, 4), INV),            # nq <= 0
        ((res, h, q, 1, 0, 1, 4), INV),            # k <= 0
        ((res, h, q, 1, 2**31, 1, 4), INV),        # k > INT32_MAX
        ((res, h, q, 2**62, 2**30, 1, 4), SHAPE),  # nq * k overflows
        ((res, h, q, 1, 2, 1, 1025), DEV),         # krefine beyond the kernels' register list
        ((res, h, q, 1, 1100, 1, 4), DEV),         # k beyond it as well
    ]
    for args, want in cases:
        r, hh, qq, nq, k, nprobe, kr = args
        ids = np.full(1200, 7, dtype=np.int64)
        d = np.full(1200, -3.0, dtype=np.float32)
        qp = None if qq is None else qq.ctypes.data_as(POINTER(c_float))
        rc = ovvs._lib.ovvsIvfPqSearch(r._h if r else None, hh, qp, c_int64(nq), c_int64(k),
                                       c_int32(nprobe), c_int32(kr), None,
                                       ids.ctypes.data_as(POINTER(c_int64)),
                                       d.ctypes.data_as(POINTER(c_float)))
        assert rc == want, (args, rc)
        assert np.all(ids == 7) and np.all(d == -3.0)
    rc, untouched = _search(ovvs, res, h, q, 1, 2, 1, 4, dtype=2)  # int8 tables: unsupported
    assert rc == UNSUP and untouched
    for policy in (ovvs.POLICY_FORCE_CPU, ovvs.POLICY_FORCE_NPU):
        res.set_policy(policy)
        rc, untouched = _search(ovvs, res, h, q, 1, 2, 1, 4)
        assert rc == DEV and untouched
    res.set_policy(ovvs.POLICY_AUTO)
    assert res.ivfpq_search_stats()["successful_calls"] == 0
    ovvs._lib.ovvsIvfPqDestroy(h)


def test_no_gpu_means_device_unavailable(ovvs):
    res = ovvs.Resources()
    if res.gpu_available():
        pytest.skip("a GPU is present")
    rc, h = _load(ovvs, res, GOLDEN / "legacy_ipq1_v1.bin")
    q = np.array([[1.1, 0.0]], dtype=np.float32)
    rc, untouched = _search(ovvs, res, h, q, 1, 2, 1, 4)
    assert rc == 7 and untouched
    x = np.zeros((16, 4), dtype=np.float32)
    with pytest.raises(ovvs.OvvsError) as e:
        ovvs.neighbors.ivf_pq.build(x, nlist=2, pq_m=2, resources=res)
    assert e.value.status == 7
    ovvs._lib.ovvsIvfPqDestroy(h)


def test_build_and_extend_argument_checks(ovvs):
    lib = ovvs._lib
    res = ovvs.Resources()
    x = np.zeros((8, 4), dtype=np.float32)
    xp = x.ctypes.data_as(POINTER(c_float))
    h = c_void_p(1)
    assert lib.ovvsIvfPqBuild(res._h, None, 8, 4, 0, 2, 2, 8, byref(h)) == 2 and not h.value
    assert lib.ovvsIvfPqBuild(None, xp, 8, 4, 0, 2, 2, 8, byref(h)) == 2
    assert lib.ovvsIvfPqBuild(res._h, xp, 0, 4, 0, 2, 2, 8, byref(h)) == 2
    assert lib.ovvsIvfPqBuild(res._h, xp, 8, 4, 0, 0, 2, 8, byref(h)) == 2
    assert lib.ovvsIvfPqBuild(res._h, xp, 8, 4, 6, 2, 2, 8, byref(h)) == 2    # bad metric
    assert lib.ovvsIvfPqBuild(res._h, xp, 8, 4, 0, 2, 3, 8, byref(h)) == 6    # dim % pq_m
    assert lib.ovvsIvfPqBuild(res._h, xp, 2**31, 4, 0, 2, 2, 8, byref(h)) == 6
    assert lib.ovvsIvfPqBuild(res._h, xp, 8, 4, 0, 2, 2, 8, None) == 2
    rc, ix = _load(ovvs, res, GOLDEN / "legacy_ipq1_v1.bin")
    assert lib.ovvsIvfPqExtend(res._h, ix, None, 1) == 2
    assert lib.ovvsIvfPqExtend(res._h, ix, xp, 0) == 2
    assert lib.ovvsIvfPqExtend(None, ix, xp, 1) == 2
    lib.ovvsIvfPqDestroy(ix)


def test_scann_argument_checks(ovvs):
    """ScaNN entry points (reference src/neighbors/graphs.cpp:3286-3385): null
    pointers are INVALID_ARGUMENT, a failed build leaves *index as it was, the inner
    IVF-PQ build's argument checks apply, and destroying NULL succeeds."""
    lib = ovvs._lib
    res = ovvs.Resources()
    x = np.zeros((8, 4), dtype=np.float32)
    xp = x.ctypes.data_as(POINTER(c_float))
    h = c_void_p(5)
    assert lib.ovvsScannBuild(None, xp, 8, 4, 0, 2, 2, byref(h)) == 2
    assert lib.ovvsScannBuild(res._h, None, 8, 4, 0, 2, 2, byref(h)) == 2
    assert lib.ovvsScannBuild(res._h, xp, 8, 4, 0, 2, 2, None) == 2
    assert lib.ovvsScannBuild(res._h, xp, 0, 4, 0, 2, 2, byref(h)) == 2
    assert lib.ovvsScannBuild(res._h, xp, 8, 4, 6, 2, 2, byref(h)) == 2   # bad metric
    assert lib.ovvsScannBuild(res._h, xp, 8, 4, 0, 0, 2, byref(h)) == 2   # nlist <= 0
    assert lib.ovvsScannBuild(res._h, xp, 8, 4, 0, 2, 3, byref(h)) == 6   # dim % pq_m
    assert h.value == 5
    q = np.zeros((1, 4), dtype=np.float32)
    qp = q.ctypes.data_as(POINTER(c_float))
    ids = np.full(4, 7, dtype=np.int64)
    d = np.full(4, -3.0, dtype=np.float32)
    ip, dp = ids.ctypes.data_as(POINTER(c_int64)), d.ctypes.data_as(POINTER(c_float))
    fake = c_void_p(1)  # never dereferenced: the null checks come first
    assert lib.ovvsScannSearch(None, fake, qp, 1, 4, 1, 4, ip, dp) == 2
    assert lib.ovvsScannSearch(res._h, None, qp, 1, 4, 1, 4, ip, dp) == 2
    assert lib.ovvsScannSearch(res._h, fake, None, 1, 4, 1, 4, ip, dp) == 2
    assert lib.ovvsScannSearch(res._h, fake, qp, 1, 4, 1, 4, None, dp) == 2
    assert lib.ovvsScannSearch(res._h, fake, qp, 1, 4, 1, 4, ip, None) == 2
    assert np.all(ids == 7) and np.all(d == -3.0)
    assert lib.ovvsScannDestroy(None) == 0


def test_scann_build_without_gpu_is_device_unavailable(ovvs):
    res = ovvs.Resources()
    if res.gpu_available():
        pytest.skip("a GPU is present")
    x = np.zeros((16, 4), dtype=np.float32)
    h = c_void_p(5)
    rc = ovvs._lib.ovvsScannBuild(res._h, x.ctypes.data_as(POINTER(c_float)), 16, 4, 0, 2, 2,
                                  byref(h))
    assert rc == 7 and h.value == 5


def test_knn_graph_argument_checks(ovvs):
    """ovvsIvfPqKnnGraph (additive; the reference's CAGRA IVF-PQ initializer,
    src/neighbors/graphs.cpp:767-797): null pointers and a negative degree are
    INVALID_ARGUMENT, a degree past the shortlist limit DEVICE_UNAVAILABLE, the inner
    build's checks pass through, and the graph is untouched on failure."""
    lib = ovvs._lib
    res = ovvs.Resources()
    x = np.zeros((8, 4), dtype=np.float32)
    xp = x.ctypes.data_as(POINTER(c_float))
    g = np.full(64, 7, dtype=np.int32)
    gp = g.ctypes.data_as(POINTER(c_int32))
    assert lib.ovvsIvfPqKnnGraph(None, xp, 8, 4, 0, 4, gp) == 2
    assert lib.ovvsIvfPqKnnGraph(res._h, None, 8, 4, 0, 4, gp) == 2
    assert lib.ovvsIvfPqKnnGraph(res._h, xp, 8, 4, 0, 4, None) == 2
    assert lib.ovvsIvfPqKnnGraph(res._h, xp, 8, 4, 0, -1, gp) == 2
    assert lib.ovvsIvfPqKnnGraph(res._h, xp, 8, 4, 0, 1024, gp) == 7
    assert lib.ovvsIvfPqKnnGraph(res._h, xp, 0, 4, 0, 4, gp) == 2     # the build's n check
    assert lib.ovvsIvfPqKnnGraph(res._h, xp, 8, 4, 9, 4, gp) == 2     # the build's metric check
    assert np.all(g == 7)
    if not res.gpu_available():
        assert lib.ovvsIvfPqKnnGraph(res._h, xp, 8, 4, 0, 4, gp) == 7
        assert np.all(g == 7)


# Every symbol the reference's Python package binds unconditionally when it loads the
# library (reference python/ovvs/__init__.py:150-306, the `_lib.<name>.argtypes` and
# `.restype` assignments at module level): with all of them exported, that package
# loads libovvs.so through OVVS_LIBRARY and its IVF-PQ and ScaNN calls reach this
# library (the others answer OVVS_STATUS_UNSUPPORTED).
REFERENCE_PACKAGE_BINDS = (
    "ovvsBatcherCreate", "ovvsBatcherDestroy", "ovvsBatcherSearch", "ovvsBitsetFromAllowList",
    "ovvsBruteForceBuild", "ovvsBruteForceDestroy", "ovvsBruteForceSearch", "ovvsCagraBuild",
    "ovvsCagraDestroy", "ovvsCagraExtend", "ovvsCagraSearch", "ovvsGatherRows", "ovvsGemm",
    "ovvsGemmEx", "ovvsGetVersion", "ovvsHnswDeserialize", "ovvsHnswDestroy",
    "ovvsHnswFromCagra", "ovvsHnswSearch", "ovvsHnswSerialize", "ovvsIvfFlatBuild",
    "ovvsIvfFlatDestroy", "ovvsIvfFlatSearch", "ovvsIvfPqBuild", "ovvsIvfPqDeserialize",
    "ovvsIvfPqDestroy", "ovvsIvfPqExtend", "ovvsIvfPqSearch", "ovvsIvfPqSerialize",
    "ovvsIvfRabitqBuild", "ovvsIvfRabitqDeserialize", "ovvsIvfRabitqDestroy",
    "ovvsIvfRabitqExtend", "ovvsIvfRabitqSearch", "ovvsIvfRabitqSerialize",
    "ovvsKMeansDestroy", "ovvsKMeansFit", "ovvsKMeansPredict", "ovvsResourcesCreate",
    "ovvsResourcesDestroy", "ovvsResourcesEnergyUj", "ovvsResourcesLastComputeDtype",
    "ovvsResourcesLastDevice", "ovvsResourcesSetPolicy", "ovvsScannBuild", "ovvsScannDestroy",
    "ovvsScannSearch", "ovvsStatusString", "ovvsSyclEnabled", "ovvsTopk", "ovvsVamanaBuild",
    "ovvsVamanaDestroy", "ovvsVamanaSearch",
)


def test_reference_python_package_symbols_are_exported(ovvs):
    lib = ctypes.CDLL(str(ovvs.library_path()))
    assert len(REFERENCE_PACKAGE_BINDS) == 53
    missing = [s for s in REFERENCE_PACKAGE_BINDS if not hasattr(lib, s)]
    assert not missing, missing


def test_other_algorithms_answer_unsupported(ovvs):
    lib = ovvs._lib
    res = ovvs.Resources()
    h = c_void_p()
    x = np.zeros((4, 8), dtype=np.float32)
    assert lib.ovvsCagraBuild(res._h, x.ctypes.data_as(POINTER(c_float)), c_int64(4), c_int64(8),
                              c_int32(0), c_int32(4), c_int32(8), byref(h)) == ovvs.STATUS_UNSUPPORTED
    assert h.value is None
    assert lib.ovvsBruteForceDestroy(None) == ovvs.STATUS_SUCCESS
    assert lib.ovvsSyclEnabled() == 0
    e = c_int64(-5)
    assert lib.ovvsResourcesEnergyUj(res._h, byref(e)) == ovvs.STATUS_UNSUPPORTED and e.value == -5
