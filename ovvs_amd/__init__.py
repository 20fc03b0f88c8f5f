"""ovvs_amd — Python bindings for libovvs, the MI355X IVF-PQ library.

This is the IVF-PQ slice of the reference's ctypes package
(reference python/ovvs/__init__.py): the same names, argument order, defaults
and return shapes, so code written against ``ovvs`` for IVF-PQ runs unchanged:

    res = ovvs_amd.Resources()
    index = ovvs_amd.neighbors.ivf_pq.build(data, nlist=4096, pq_m=48, resources=res)
    ids, dists = index.search(queries, k=10, nprobe=64, krefine=32)

``ids`` is int64 [nq, k] and ``dists`` float32 [nq, k]; empty slots are
(-1, +inf). The library is found through $OVVS_LIBRARY, else
``ovvs_amd/lib/libovvs.so`` (built by ``__graft_entry__.build()``). There is no
Python fallback: a missing library raises at import, and every search runs on
the GPU (a host without one gets OvvsError with status DEVICE_UNAVAILABLE).
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int32, c_int64, c_uint8, c_uint32, c_void_p
from pathlib import Path

import numpy as np

__all__ = [
    "OvvsError",
    "Resources",
    "IvfPqIndex",
    "ScannIndex",
    "neighbors",
    "bitset_from_allow_list",
    "version",
    "library_path",
]

# Enum values of include/ovvs/ovvs.h (reference include/ovvs/ovvs.h:13-48).
STATUS_SUCCESS = 0
STATUS_ERROR = 1
STATUS_INVALID_ARGUMENT = 2
STATUS_UNSUPPORTED = 3
STATUS_OOM = 4
STATUS_SHAPE_MISMATCH = 6
STATUS_DEVICE_UNAVAILABLE = 7
STATUS_IO = 8

DEVICE_AUTO, DEVICE_CPU, DEVICE_NPU, DEVICE_GPU, DEVICE_HETERO = range(5)
(POLICY_AUTO, POLICY_NPU_IF_FASTER, POLICY_GPU_IF_FASTER, POLICY_HETERO, POLICY_FORCE_NPU,
 POLICY_FORCE_GPU, POLICY_FORCE_CPU) = range(7)
METRIC_L2 = 0
METRIC_L2_SQRT = 1
METRIC_INNER_PRODUCT = 2
METRIC_COSINE = 3
METRIC_HAMMING = 4
METRIC_LP = 5
DTYPE_F32 = 0
DTYPE_F16 = 1
# Size of the device scratch ovvsIvfPqSearchDeviceNoAlloc carves its workspace from.
NOALLOC_SCRATCH_BYTES = 64 << 20

OVVS_IVF_PQ_SEARCH_STATS_ABI_V1 = 1
_STATS_FIELDS = (
    "successful_calls", "blocks", "queries", "tasks", "candidate_rows", "selected_rows",
    "total_wall_ns", "coarse_pairwise_ns", "coarse_topk_ns", "planning_ns", "lut_build_ns",
    "adc_scan_select_ns", "shortlist_select_validate_ns", "refine_gather_ns",
    "refine_distance_ns", "refine_topk_ns", "gpu_allocation_calls", "gpu_allocation_bytes",
    "gpu_h2d_calls", "gpu_h2d_bytes", "gpu_d2h_calls", "gpu_d2h_bytes", "gpu_kernel_launches",
    "gpu_wait_calls",
)


class _StatsV1(ctypes.Structure):
    _fields_ = [("abi_version", c_uint32), ("struct_size", c_uint32)] + [
        (name, c_int64) for name in _STATS_FIELDS
    ]


assert ctypes.sizeof(_StatsV1) == 200


def library_path() -> Path:
    env = os.environ.get("OVVS_LIBRARY")
    if env:
        return Path(env)
    return Path(__file__).resolve().parent / "lib" / "libovvs.so"


def _load() -> ctypes.CDLL:
    path = library_path()
    if not path.exists():
        raise OSError(
            f"libovvs not found at {path}; build it with `python -c 'import __graft_entry__ as g; "
            "g.build()'` or point OVVS_LIBRARY at it"
        )
    return ctypes.CDLL(str(path))


_lib = _load()

_V = c_void_p
_SIGS = {
    "ovvsGetVersion": (c_char_p, []),
    "ovvsStatusString": (c_char_p, [c_int32]),
    "ovvsResourcesCreate": (c_int32, [POINTER(_V)]),
    "ovvsResourcesDestroy": (c_int32, [_V]),
    "ovvsResourcesSetPolicy": (c_int32, [_V, c_int32]),
    "ovvsResourcesGetPolicy": (c_int32, [_V, POINTER(c_int32)]),
    "ovvsResourcesGpuAvailable": (c_int32, [_V, POINTER(c_int32)]),
    "ovvsResourcesNpuAvailable": (c_int32, [_V, POINTER(c_int32)]),
    "ovvsResourcesLastDevice": (c_int32, [_V, POINTER(c_int32)]),
    "ovvsResourcesLastComputeDtype": (c_int32, [_V, POINTER(c_int32)]),
    "ovvsResourcesIvfPqSearchStatsV1": (c_int32, [_V, POINTER(_StatsV1)]),
    "ovvsResourcesIvfPqTableQueries": (c_int32, [_V, POINTER(c_int64)]),
    "ovvsIvfPqBuild": (c_int32, [_V, POINTER(c_float), c_int64, c_int64, c_int32, c_int32,
                                 c_int32, c_int32, POINTER(_V)]),
    "ovvsIvfPqSearch": (c_int32, [_V, _V, POINTER(c_float), c_int64, c_int64, c_int32, c_int32,
                                  _V, POINTER(c_int64), POINTER(c_float)]),
    "ovvsIvfPqSearchEx": (c_int32, [_V, _V, POINTER(c_float), c_int64, c_int64, c_int32,
                                    c_int32, _V, c_int32, POINTER(c_int64), POINTER(c_float)]),
    "ovvsIvfPqSearchDevice": (c_int32, [_V, _V, _V, c_int64, c_int64, c_int32, c_int32, _V,
                                        c_int32, _V, _V]),
    "ovvsIvfPqSearchDeviceNoAlloc": (c_int32, [_V, _V, _V, c_int64, c_int64, c_int32, c_int32,
                                               _V, c_int32, _V, _V]),
    "ovvsIvfPqSerialize": (c_int32, [_V, c_char_p]),
    "ovvsIvfPqDeserialize": (c_int32, [_V, c_char_p, POINTER(_V)]),
    "ovvsIvfPqExtend": (c_int32, [_V, _V, POINTER(c_float), c_int64]),
    "ovvsIvfPqDestroy": (c_int32, [_V]),
    "ovvsBitsetFromAllowList": (c_int32, [c_int64, POINTER(c_int64), c_int64, POINTER(c_uint8)]),
    "ovvsScannBuild": (c_int32, [_V, POINTER(c_float), c_int64, c_int64, c_int32, c_int32, c_int32,
                                 POINTER(_V)]),
    "ovvsScannSearch": (c_int32, [_V, _V, POINTER(c_float), c_int64, c_int64, c_int32, c_int32,
                                  POINTER(c_int64), POINTER(c_float)]),
    "ovvsScannDestroy": (c_int32, [_V]),
    "ovvsIvfPqKnnGraph": (c_int32, [_V, POINTER(c_float), c_int64, c_int64, c_int32, c_int32,
                                    POINTER(c_int32)]),
}
for _name, (_res, _args) in _SIGS.items():
    _fn = getattr(_lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args


class OvvsError(RuntimeError):
    """A libovvs call returned a non-success ovvsStatus."""

    def __init__(self, operation: str, status: int):
        self.operation = operation
        self.status = int(status)
        text = _lib.ovvsStatusString(c_int32(self.status))
        detail = text.decode(errors="replace") if text else "unknown"
        super().__init__(f"{operation} failed: {detail} (status={self.status})")


def _check_status(status: int, operation: str) -> None:
    if status != STATUS_SUCCESS:
        raise OvvsError(operation, status)


def version() -> str:
    return _lib.ovvsGetVersion().decode()


def _f32_matrix(x, dim=None):
    a = np.ascontiguousarray(x, dtype=np.float32)
    if a.ndim == 1:
        if dim is None:
            raise ValueError("a flat array needs dim")
        a = a.reshape(-1, int(dim))
    if a.ndim != 2 or (dim is not None and a.shape[1] != int(dim)):
        raise ValueError(f"expected a [n, {dim}] float32 matrix, got shape {a.shape}")
    return a


class Resources:
    """One caller thread's stream, device workspace and telemetry."""

    def __init__(self):
        self._h = c_void_p()
        _check_status(_lib.ovvsResourcesCreate(ctypes.byref(self._h)), "ovvsResourcesCreate")

    def close(self):
        # At interpreter exit the module's globals may already be cleared.
        if self._h and _lib is not None:
            _lib.ovvsResourcesDestroy(self._h)
        self._h = None

    def __del__(self):
        self.close()

    def set_policy(self, policy: int) -> None:
        _check_status(_lib.ovvsResourcesSetPolicy(self._h, c_int32(policy)), "set_policy")

    def get_policy(self) -> int:
        v = c_int32()
        _check_status(_lib.ovvsResourcesGetPolicy(self._h, ctypes.byref(v)), "get_policy")
        return int(v.value)

    def gpu_available(self) -> bool:
        v = c_int32()
        _check_status(_lib.ovvsResourcesGpuAvailable(self._h, ctypes.byref(v)), "gpu_available")
        return bool(v.value)

    def last_device(self) -> int:
        v = c_int32()
        _check_status(_lib.ovvsResourcesLastDevice(self._h, ctypes.byref(v)), "last_device")
        return int(v.value)

    def last_compute_dtype(self) -> int:
        v = c_int32()
        _check_status(_lib.ovvsResourcesLastComputeDtype(self._h, ctypes.byref(v)),
                      "last_compute_dtype")
        return int(v.value)

    def ivfpq_table_queries(self) -> int:
        """Queries handed off to the full-table scan (bounds that did not prune), over
        all searches on these Resources."""
        v = c_int64()
        _check_status(_lib.ovvsResourcesIvfPqTableQueries(self._h, ctypes.byref(v)),
                      "ovvsResourcesIvfPqTableQueries")
        return int(v.value)

    def ivfpq_search_stats(self) -> dict:
        s = _StatsV1()
        _check_status(_lib.ovvsResourcesIvfPqSearchStatsV1(self._h, ctypes.byref(s)),
                      "ovvsResourcesIvfPqSearchStatsV1")
        if s.abi_version != OVVS_IVF_PQ_SEARCH_STATS_ABI_V1 or s.struct_size != ctypes.sizeof(s):
            raise RuntimeError("ovvsResourcesIvfPqSearchStatsV1 returned an incompatible layout")
        out = {"abi_version": int(s.abi_version), "struct_size": int(s.struct_size)}
        out.update({name: int(getattr(s, name)) for name in _STATS_FIELDS})
        return out


def bitset_from_allow_list(n, ids) -> np.ndarray:
    """LSB-first allow bitset of (n+7)//8 bytes (ids outside [0, n) are ignored)."""
    n = int(n)
    arr = np.ascontiguousarray(np.asarray(list(ids) if not isinstance(ids, np.ndarray) else ids,
                                          dtype=np.int64).ravel())
    out = np.zeros(max((n + 7) // 8, 1), dtype=np.uint8)
    rc = _lib.ovvsBitsetFromAllowList(
        c_int64(n), arr.ctypes.data_as(POINTER(c_int64)) if arr.size else None,
        c_int64(arr.size), out.ctypes.data_as(POINTER(c_uint8)))
    _check_status(rc, "ovvsBitsetFromAllowList")
    return out


def _bitset_arg(n, bitset=None, allow_list=None):
    if allow_list is not None:
        b = bitset_from_allow_list(n, allow_list)
        return b, b.ctypes.data_as(c_void_p)
    if bitset is None:
        return None, None
    b = np.ascontiguousarray(np.frombuffer(bytes(bitset), dtype=np.uint8)
                             if isinstance(bitset, (bytes, bytearray)) else bitset, dtype=np.uint8)
    if b.size < (int(n) + 7) // 8:
        raise ValueError(f"bitset needs {(int(n) + 7) // 8} bytes, got {b.size}")
    return b, b.ctypes.data_as(c_void_p)


class IvfPqIndex:
    """Handle of a built or loaded IVF-PQ index (reference python/ovvs/__init__.py:905-937)."""

    def __init__(self, res: Resources, handle: c_void_p, dim: int, own_res: bool, n: int = 0):
        self._res = res
        self._h = handle
        self.dim = int(dim)
        self.n = int(n)
        self._own = own_res

    def close(self):
        if self._h and _lib is not None:
            _lib.ovvsIvfPqDestroy(self._h)
        self._h = None
        if self._own and self._res is not None:
            self._res.close()
            self._res = None

    def __del__(self):
        self.close()

    @property
    def resources(self) -> Resources:
        return self._res

    def search(self, queries, k=10, nprobe=8, krefine=32, bitset=None, allow_list=None):
        return self.search_ex(queries, k, nprobe, krefine, bitset, allow_list, lut_dtype=DTYPE_F32)

    def search_ex(self, queries, k=10, nprobe=8, krefine=32, bitset=None, allow_list=None,
                  lut_dtype=DTYPE_F32):
        q = _f32_matrix(queries, self.dim)
        nq = q.shape[0]
        keep, bsp = _bitset_arg(self.n, bitset, allow_list)
        ids = np.empty((nq, int(k)), dtype=np.int64)
        dists = np.empty((nq, int(k)), dtype=np.float32)
        args = (self._res._h, self._h, q.ctypes.data_as(POINTER(c_float)), c_int64(nq),
                c_int64(k), c_int32(nprobe), c_int32(krefine), bsp)
        outs = (ids.ctypes.data_as(POINTER(c_int64)), dists.ctypes.data_as(POINTER(c_float)))
        if lut_dtype == DTYPE_F32:
            rc = _lib.ovvsIvfPqSearch(*args, *outs)
        else:
            rc = _lib.ovvsIvfPqSearchEx(*args, c_int32(lut_dtype), *outs)
        del keep
        _check_status(rc, "IVF-PQ search")
        return ids, dists

    def search_device(self, queries_ptr: int, nq: int, k: int, nprobe: int, krefine: int,
                      ids_ptr: int, dists_ptr: int, bitset_ptr: int | None = None,
                      lut_dtype=DTYPE_F32) -> None:
        """Search with every buffer already in device memory (raw device addresses)."""
        rc = _lib.ovvsIvfPqSearchDevice(self._res._h, self._h, c_void_p(queries_ptr),
                                        c_int64(nq), c_int64(k), c_int32(nprobe),
                                        c_int32(krefine), c_void_p(bitset_ptr or 0),
                                        c_int32(lut_dtype), c_void_p(ids_ptr),
                                        c_void_p(dists_ptr))
        _check_status(rc, "IVF-PQ device search")

    def search_device_noalloc(self, queries_ptr: int, nq: int, k: int, nprobe: int,
                              krefine: int, ids_ptr: int, dists_ptr: int,
                              bitset_ptr: int | None = None, lut_dtype=DTYPE_F32) -> None:
        """search_device without any allocation: the workspace is the library's fixed
        device scratch (NOALLOC_SCRATCH_BYTES); the index must already be on the GPU."""
        rc = _lib.ovvsIvfPqSearchDeviceNoAlloc(self._res._h, self._h, c_void_p(queries_ptr),
                                               c_int64(nq), c_int64(k), c_int32(nprobe),
                                               c_int32(krefine), c_void_p(bitset_ptr or 0),
                                               c_int32(lut_dtype), c_void_p(ids_ptr),
                                               c_void_p(dists_ptr))
        _check_status(rc, "IVF-PQ no-allocation device search")

    def serialize(self, path) -> None:
        _check_status(_lib.ovvsIvfPqSerialize(self._h, str(path).encode()), "IVF-PQ serialize")

    def extend(self, extra):
        x = _f32_matrix(extra, self.dim)
        rc = _lib.ovvsIvfPqExtend(self._res._h, self._h, x.ctypes.data_as(POINTER(c_float)),
                                  c_int64(x.shape[0]))
        _check_status(rc, "IVF-PQ extend")
        self.n += x.shape[0]
        return x


class ScannIndex:
    """Handle of a ScaNN-style index (reference python/ovvs/__init__.py:1189-1243)."""

    def __init__(self, res: Resources, handle: c_void_p, dim: int, own_res: bool, n: int = 0):
        self._res = res
        self._h = handle
        self.dim = int(dim)
        self.n = int(n)
        self._own = own_res

    def close(self):
        if self._h and _lib is not None:
            _lib.ovvsScannDestroy(self._h)
        self._h = None
        if self._own and self._res is not None:
            self._res.close()
            self._res = None

    def __del__(self):
        self.close()

    @property
    def resources(self) -> Resources:
        return self._res

    def search(self, queries, k=10, nprobe=8, krefine=32):
        q = _f32_matrix(queries, self.dim)
        nq = q.shape[0]
        ids = np.empty((nq, int(k)), dtype=np.int64)
        dists = np.empty((nq, int(k)), dtype=np.float32)
        rc = _lib.ovvsScannSearch(self._res._h, self._h, q.ctypes.data_as(POINTER(c_float)),
                                  c_int64(nq), c_int64(k), c_int32(nprobe), c_int32(krefine),
                                  ids.ctypes.data_as(POINTER(c_int64)),
                                  dists.ctypes.data_as(POINTER(c_float)))
        _check_status(rc, "ScaNN search")
        return ids, dists


class neighbors:
    class scann:
        @staticmethod
        def build(dataset, dim=None, metric=0, nlist=8, pq_m=8, resources=None):
            res = resources or Resources()
            x = _f32_matrix(dataset, dim)
            h = c_void_p()
            rc = _lib.ovvsScannBuild(res._h, x.ctypes.data_as(POINTER(c_float)),
                                     c_int64(x.shape[0]), c_int64(x.shape[1]), c_int32(metric),
                                     c_int32(nlist), c_int32(pq_m), ctypes.byref(h))
            _check_status(rc, "ScaNN build")
            return ScannIndex(res, h, x.shape[1], own_res=resources is None, n=x.shape[0])

    class ivf_pq:
        @staticmethod
        def build(dataset, dim=None, metric=0, nlist=8, pq_m=8, pq_nbits=8, resources=None):
            res = resources or Resources()
            x = _f32_matrix(dataset, dim)
            h = c_void_p()
            rc = _lib.ovvsIvfPqBuild(res._h, x.ctypes.data_as(POINTER(c_float)),
                                     c_int64(x.shape[0]), c_int64(x.shape[1]), c_int32(metric),
                                     c_int32(nlist), c_int32(pq_m), c_int32(pq_nbits),
                                     ctypes.byref(h))
            _check_status(rc, "IVF-PQ build")
            return IvfPqIndex(res, h, x.shape[1], own_res=resources is None, n=x.shape[0])

        @staticmethod
        def knn_graph(dataset, degree, dim=None, metric=0, resources=None):
            """k-nearest-neighbour graph [n, degree] int32 of the rows by IVF-PQ (the
            CAGRA build's IVF-PQ initializer, reference src/neighbors/graphs.cpp:767-797)."""
            res = resources or Resources()
            x = _f32_matrix(dataset, dim)
            g = np.empty((x.shape[0], int(degree)), dtype=np.int32)
            rc = _lib.ovvsIvfPqKnnGraph(res._h, x.ctypes.data_as(POINTER(c_float)),
                                        c_int64(x.shape[0]), c_int64(x.shape[1]),
                                        c_int32(metric), c_int32(degree),
                                        g.ctypes.data_as(POINTER(c_int32)))
            _check_status(rc, "IVF-PQ knn graph")
            return g

        @staticmethod
        def load(path, resources=None):
            """Deserialize an IPQ1 v1 file."""
            res = resources or Resources()
            h = c_void_p()
            _check_status(_lib.ovvsIvfPqDeserialize(res._h, str(path).encode(), ctypes.byref(h)),
                          "IVF-PQ deserialize")
            with open(path, "rb") as f:
                head = f.read(24)
            n = int(np.frombuffer(head, dtype=np.int64, count=1, offset=8)[0])
            dim = int(np.frombuffer(head, dtype=np.int64, count=1, offset=16)[0])
            return IvfPqIndex(res, h, dim, own_res=resources is None, n=n)
