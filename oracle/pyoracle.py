"""Python handles on the CPU parity checkers (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module; libovvs never does.

* ``Oracle``  — our C restatement of the reference search (oracle/ivfpq_oracle.c,
  built into oracle/liboracle.so).
* ``Reference`` — the reference library itself, compiled from /root/reference by
  ``make -C oracle ref`` into oracle/_ref/libovvs_ref.so, driven through its own C
  ABI with the FORCE_CPU policy (its CPU route, reference
  src/neighbors/indexes.cpp:538-1134).
* ``read_ipq1`` — parses an IPQ1 v1 file (reference src/neighbors/indexes.cpp:1141-1178)
  into the list-major arrays both searchers consume.
"""

from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_float, c_int32, c_int64, c_uint8, c_uint16, c_void_p
from dataclasses import dataclass
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "liboracle.so"
REF_SO = HERE / "_ref" / "libovvs_ref.so"

FORCE_CPU = 6


@dataclass
class Ipq1:
    n: int
    dim: int
    nlist: int
    pq_m: int
    pq_ks: int
    dsub: int
    metric: int
    centroids: np.ndarray   # [nlist, dim] f32
    codebooks: np.ndarray   # [pq_m, ks, dsub] f32
    codes: np.ndarray       # [n, pq_m] u8 by id
    dataset: np.ndarray     # [n, dim] f32
    assign: np.ndarray      # [n] i32
    lists: list             # nlist arrays of i64 ids

    def to_bytes(self) -> bytes:
        """The IPQ1 v1 file of this index (the inverse of read_ipq1), used by tests to
        write indexes with hand-made centroids."""
        head = np.array([0x31515049, 1], dtype=np.uint32).tobytes()
        head += np.array([self.n, self.dim], dtype=np.int64).tobytes()
        head += np.array([self.nlist, self.pq_m, self.pq_ks, self.dsub, self.metric],
                         dtype=np.int32).tobytes()
        parts = [head,
                 np.ascontiguousarray(self.centroids, dtype=np.float32).tobytes(),
                 np.ascontiguousarray(self.codebooks, dtype=np.float32).tobytes(),
                 np.ascontiguousarray(self.codes, dtype=np.uint8).tobytes(),
                 np.ascontiguousarray(self.dataset, dtype=np.float32).tobytes(),
                 np.ascontiguousarray(self.assign, dtype=np.int32).tobytes()]
        for l in self.lists:
            parts.append(np.int32(len(l)).tobytes())
            parts.append(np.ascontiguousarray(l, dtype=np.int64).tobytes())
        return b"".join(parts)

    def packed(self):
        """List-major (packed_codes [n, pq_m], packed_ids [n], offsets [nlist+1])."""
        ids = np.concatenate([np.asarray(l, dtype=np.int64) for l in self.lists]) \
            if self.n else np.zeros(0, np.int64)
        offsets = np.zeros(self.nlist + 1, dtype=np.int64)
        offsets[1:] = np.cumsum([len(l) for l in self.lists])
        return np.ascontiguousarray(self.codes[ids]), ids, offsets


def read_ipq1(path) -> Ipq1:
    raw = Path(path).read_bytes()
    head = np.frombuffer(raw, dtype=np.uint8, count=44)
    magic, version = np.frombuffer(head[:8].tobytes(), dtype=np.int32)
    if np.uint32(magic) != 0x31515049 or version != 1:
        raise ValueError("not an IPQ1 v1 file")
    n, dim = (int(v) for v in np.frombuffer(head[8:24].tobytes(), dtype=np.int64))
    nlist, pq_m, pq_ks, dsub, metric = (int(v) for v in np.frombuffer(head[24:44].tobytes(),
                                                                       dtype=np.int32))
    off = 44

    def take(dtype, count):
        nonlocal off
        a = np.frombuffer(raw, dtype=dtype, count=count, offset=off)
        off += a.nbytes
        return a.copy()

    centroids = take(np.float32, nlist * dim).reshape(nlist, dim)
    codebooks = take(np.float32, pq_m * pq_ks * dsub).reshape(pq_m, pq_ks, dsub)
    codes = take(np.uint8, n * pq_m).reshape(n, pq_m)
    dataset = take(np.float32, n * dim).reshape(n, dim)
    assign = take(np.int32, n)
    lists = []
    for _ in range(nlist):
        size = int(take(np.int32, 1)[0])
        lists.append(take(np.int64, size))
    if off != len(raw):
        raise ValueError("trailing bytes in IPQ1 file")
    return Ipq1(n, dim, nlist, pq_m, pq_ks, dsub, metric, centroids, codebooks, codes, dataset,
                assign, lists)


def read_ipq1_stream(f, dataset) -> Ipq1:
    """read_ipq1 from a sequential stream (a pipe the library serializes into), with
    the dataset section read and dropped in pieces: `dataset` ([n, dim] f32, the rows
    the index was built from, by id) stands in for it. For indexes whose IPQ1 file
    would not fit a disk (C5: 43 GB, 38.4 GB of it the dataset)."""

    def read_exact(nbytes):
        buf = bytearray(nbytes)
        view = memoryview(buf)
        got = 0
        while got < nbytes:
            m = f.readinto(view[got:])
            if not m:
                raise ValueError("IPQ1 stream ended early")
            got += m
        return buf

    def take(dtype, count):
        return np.frombuffer(read_exact(int(np.dtype(dtype).itemsize) * count), dtype=dtype)

    head = bytes(read_exact(44))
    magic, version = np.frombuffer(head[:8], dtype=np.int32)
    if np.uint32(magic) != 0x31515049 or version != 1:
        raise ValueError("not an IPQ1 v1 stream")
    n, dim = (int(v) for v in np.frombuffer(head[8:24], dtype=np.int64))
    nlist, pq_m, pq_ks, dsub, metric = (int(v) for v in np.frombuffer(head[24:44], dtype=np.int32))
    if dataset.shape != (n, dim):
        raise ValueError("dataset does not match the stream's shape")
    centroids = take(np.float32, nlist * dim).reshape(nlist, dim)
    codebooks = take(np.float32, pq_m * pq_ks * dsub).reshape(pq_m, pq_ks, dsub)
    codes = take(np.uint8, n * pq_m).reshape(n, pq_m)
    left = n * dim * 4
    while left:
        left -= len(read_exact(min(left, 1 << 26)))
    assign = take(np.int32, n)
    lists = []
    for _ in range(nlist):
        size = int(take(np.int32, 1)[0])
        lists.append(take(np.int64, size))
    if f.read(1):
        raise ValueError("trailing bytes in IPQ1 stream")
    return Ipq1(n, dim, nlist, pq_m, pq_ks, dsub, metric, centroids, codebooks, codes, dataset,
                assign, lists)


class _OracleIndex(ctypes.Structure):
    _fields_ = [
        ("n", c_int64), ("dim", c_int64), ("nlist", c_int32), ("pq_m", c_int32),
        ("pq_ks", c_int32), ("dsub", c_int32), ("metric", c_int32), ("pad_", c_int32),
        ("centroids", POINTER(c_float)), ("codebooks", POINTER(c_float)),
        ("packed_codes", POINTER(c_uint8)), ("packed_ids", POINTER(c_int64)),
        ("list_offsets", POINTER(c_int64)), ("dataset", POINTER(c_float)),
    ]


def _f32p(a):
    return a.ctypes.data_as(POINTER(c_float))


def _i64p(a):
    return a.ctypes.data_as(POINTER(c_int64))


class Oracle:
    """ctypes front end of oracle/liboracle.so over one IPQ1 index."""

    def __init__(self, ix: Ipq1):
        self.lib = ctypes.CDLL(str(ORACLE_SO))
        L = self.lib
        L.oracle_ivfpq_search.restype = c_int32
        L.oracle_ivfpq_search.argtypes = [POINTER(_OracleIndex), POINTER(c_float), c_int64,
                                          c_int64, c_int32, c_int32, c_void_p, c_int32,
                                          POINTER(c_int64), POINTER(c_float)]
        L.oracle_probe.restype = c_int32
        L.oracle_probe.argtypes = [POINTER(_OracleIndex), POINTER(c_float), c_int64, c_int32,
                                   POINTER(c_int64)]
        L.oracle_shortlist.restype = c_int64
        L.oracle_shortlist.argtypes = [POINTER(_OracleIndex), POINTER(c_float), POINTER(c_int64),
                                       c_int32, c_int32, c_void_p, c_int32, POINTER(c_int64),
                                       POINTER(c_float), POINTER(c_int64)]
        L.oracle_lut.restype = None
        L.oracle_lut.argtypes = [POINTER(_OracleIndex), POINTER(c_float), c_int32, c_int32,
                                 POINTER(c_float)]
        self.ix = ix
        codes, ids, offsets = ix.packed()
        self._keep = [np.ascontiguousarray(ix.centroids), np.ascontiguousarray(ix.codebooks),
                      codes, ids, offsets, np.ascontiguousarray(ix.dataset)]
        c, cb, pc, pi, po, ds = self._keep
        self.packed_ids = ids
        self.offsets = offsets
        self.s = _OracleIndex(ix.n, ix.dim, ix.nlist, ix.pq_m, ix.pq_ks, ix.dsub, ix.metric, 0,
                              _f32p(c), _f32p(cb), pc.ctypes.data_as(POINTER(c_uint8)), _i64p(pi),
                              _i64p(po), _f32p(ds))

    def search(self, queries, k, nprobe, krefine, bitset=None, lut_f16=False):
        q = np.ascontiguousarray(queries, dtype=np.float32).reshape(-1, self.ix.dim)
        nq = q.shape[0]
        ids = np.empty((nq, k), dtype=np.int64)
        dists = np.empty((nq, k), dtype=np.float32)
        b = None if bitset is None else np.ascontiguousarray(bitset, dtype=np.uint8)
        rc = self.lib.oracle_ivfpq_search(ctypes.byref(self.s), _f32p(q), nq, k, nprobe, krefine,
                                          None if b is None else b.ctypes.data_as(c_void_p),
                                          int(bool(lut_f16)), _i64p(ids), _f32p(dists))
        if rc != 0:
            raise MemoryError("oracle search failed")
        return ids, dists

    def probes(self, queries, nprobe):
        q = np.ascontiguousarray(queries, dtype=np.float32).reshape(-1, self.ix.dim)
        P = max(1, min(int(nprobe), self.ix.nlist))
        out = np.empty((q.shape[0], P), dtype=np.int64)
        if self.lib.oracle_probe(ctypes.byref(self.s), _f32p(q), q.shape[0], P, _i64p(out)) != 0:
            raise MemoryError("oracle probe failed")
        return out

    def search_threads(self, queries, k, nprobe, krefine, threads):
        """search() over `threads` threads, each on a contiguous shard of the queries
        (ctypes releases the GIL during each call; the C search keeps no shared state)."""
        import threading

        q = np.ascontiguousarray(queries, dtype=np.float32).reshape(-1, self.ix.dim)
        nq = q.shape[0]
        ids = np.empty((nq, k), dtype=np.int64)
        dists = np.empty((nq, k), dtype=np.float32)
        bounds = np.linspace(0, nq, threads + 1).astype(np.int64)
        rcs = [0] * threads

        def work(t):
            a, b = int(bounds[t]), int(bounds[t + 1])
            if b > a:
                sub = np.ascontiguousarray(q[a:b])
                si = np.empty((b - a, k), dtype=np.int64)
                sd = np.empty((b - a, k), dtype=np.float32)
                rcs[t] = self.lib.oracle_ivfpq_search(ctypes.byref(self.s), _f32p(sub), b - a, k,
                                                      nprobe, krefine, None, 0, _i64p(si),
                                                      _f32p(sd))
                ids[a:b] = si
                dists[a:b] = sd

        ts = [threading.Thread(target=work, args=(t,)) for t in range(threads)]
        for t in ts:
            t.start()
        for t in ts:
            t.join()
        if any(rcs):
            raise MemoryError("oracle search failed")
        return ids, dists

    def shortlist(self, query, probes, R, bitset=None, lut_f16=False):
        q = np.ascontiguousarray(query, dtype=np.float32).reshape(self.ix.dim)
        p = np.ascontiguousarray(probes, dtype=np.int64)
        pos = np.empty(int(R), dtype=np.int64)
        sc = np.empty(int(R), dtype=np.float32)
        total = c_int64()
        b = None if bitset is None else np.ascontiguousarray(bitset, dtype=np.uint8)
        kr = self.lib.oracle_shortlist(ctypes.byref(self.s), _f32p(q), _i64p(p), p.size, int(R),
                                       None if b is None else b.ctypes.data_as(c_void_p),
                                       int(bool(lut_f16)), _i64p(pos), _f32p(sc),
                                       ctypes.byref(total))
        return pos[:kr], sc[:kr], int(total.value)

    def scann_search(self, rows, aniso, queries, k, nprobe, krefine):
        """ScaNN-style search (reference graphs.cpp:3316-3374) with this index as the
        IVF-PQ over the scaled rows, `rows` the original rows and `aniso` the column
        factors (oracle_scann_aniso)."""
        L = self.lib
        L.oracle_scann_search.restype = c_int32
        L.oracle_scann_search.argtypes = [POINTER(_OracleIndex), POINTER(c_float), c_int64,
                                          POINTER(c_float), POINTER(c_float), c_int64, c_int64,
                                          c_int32, c_int32, POINTER(c_int64), POINTER(c_float)]
        x = np.ascontiguousarray(rows, dtype=np.float32)
        a = np.ascontiguousarray(aniso, dtype=np.float32)
        q = np.ascontiguousarray(queries, dtype=np.float32).reshape(-1, self.ix.dim)
        nq = q.shape[0]
        ids = np.empty((nq, k), dtype=np.int64)
        dists = np.empty((nq, k), dtype=np.float32)
        rc = L.oracle_scann_search(ctypes.byref(self.s), _f32p(x), x.shape[0], _f32p(a), _f32p(q),
                                   nq, k, nprobe, krefine, _i64p(ids), _f32p(dists))
        if rc != 0:
            raise MemoryError("oracle ScaNN search failed")
        return ids, dists

    def lut(self, query, list_id, lut_f16=False):
        q = np.ascontiguousarray(query, dtype=np.float32).reshape(self.ix.dim)
        t = np.empty((self.ix.pq_m, self.ix.pq_ks), dtype=np.float32)
        self.lib.oracle_lut(ctypes.byref(self.s), _f32p(q), int(list_id), int(bool(lut_f16)),
                            _f32p(t))
        return t


def oracle_lib():
    lib = ctypes.CDLL(str(ORACLE_SO))
    lib.oracle_f32_to_f16.restype = c_uint16
    lib.oracle_f32_to_f16.argtypes = [c_float]
    lib.oracle_f16_to_f32.restype = c_float
    lib.oracle_f16_to_f32.argtypes = [c_uint16]
    lib.oracle_topk.restype = c_int64
    lib.oracle_topk.argtypes = [POINTER(c_float), c_int64, c_int64, POINTER(c_int64),
                                POINTER(c_float)]
    lib.oracle_brute_force.restype = c_int32
    lib.oracle_brute_force.argtypes = [POINTER(c_float), c_int64, c_int64, c_int32,
                                       POINTER(c_float), c_int64, c_int64, POINTER(c_int64),
                                       POINTER(c_float)]
    lib.oracle_refine_distance.restype = c_float
    lib.oracle_refine_distance.argtypes = [c_int32, POINTER(c_float), POINTER(c_float), c_int64]
    return lib


def scann_aniso(rows):
    """Column factors of the ScaNN-style build (oracle_scann_aniso)."""
    x = np.ascontiguousarray(rows, dtype=np.float32)
    lib = ctypes.CDLL(str(ORACLE_SO))
    lib.oracle_scann_aniso.restype = None
    lib.oracle_scann_aniso.argtypes = [POINTER(c_float), c_int64, c_int64, POINTER(c_float)]
    out = np.empty(x.shape[1], dtype=np.float32)
    lib.oracle_scann_aniso(_f32p(x), x.shape[0], x.shape[1], _f32p(out))
    return out


def brute_force(dataset, queries, k, metric=0):
    lib = oracle_lib()
    x = np.ascontiguousarray(dataset, dtype=np.float32)
    q = np.ascontiguousarray(queries, dtype=np.float32)
    ids = np.empty((q.shape[0], k), dtype=np.int64)
    d = np.empty((q.shape[0], k), dtype=np.float32)
    lib.oracle_brute_force(_f32p(x), x.shape[0], x.shape[1], metric, _f32p(q), q.shape[0], k,
                           _i64p(ids), _f32p(d))
    return ids, d


class Reference:
    """The reference libovvs (built from /root/reference into oracle/_ref), CPU route."""

    def __init__(self):
        if not REF_SO.exists():
            raise FileNotFoundError(f"{REF_SO} is not built (make -C oracle ref)")
        L = ctypes.CDLL(str(REF_SO))
        V = c_void_p
        sigs = {
            "ovvsResourcesCreate": [POINTER(V)],
            "ovvsResourcesDestroy": [V],
            "ovvsResourcesSetPolicy": [V, c_int32],
            "ovvsIvfPqBuild": [V, POINTER(c_float), c_int64, c_int64, c_int32, c_int32, c_int32,
                               c_int32, POINTER(V)],
            "ovvsIvfPqSearch": [V, V, POINTER(c_float), c_int64, c_int64, c_int32, c_int32, V,
                                POINTER(c_int64), POINTER(c_float)],
            "ovvsIvfPqSerialize": [V, c_char_p],
            "ovvsIvfPqDeserialize": [V, c_char_p, POINTER(V)],
            "ovvsIvfPqExtend": [V, V, POINTER(c_float), c_int64],
            "ovvsIvfPqDestroy": [V],
            "ovvsScannBuild": [V, POINTER(c_float), c_int64, c_int64, c_int32, c_int32, c_int32,
                               POINTER(V)],
            "ovvsScannSearch": [V, V, POINTER(c_float), c_int64, c_int64, c_int32, c_int32,
                                POINTER(c_int64), POINTER(c_float)],
            "ovvsScannDestroy": [V],
        }
        for name, args in sigs.items():
            fn = getattr(L, name)
            fn.restype = c_int32
            fn.argtypes = args
        self.lib = L
        self.res = c_void_p()
        assert L.ovvsResourcesCreate(ctypes.byref(self.res)) == 0
        assert L.ovvsResourcesSetPolicy(self.res, FORCE_CPU) == 0

    def close(self):
        if self.res:
            self.lib.ovvsResourcesDestroy(self.res)
            self.res = None

    def build(self, data, metric, nlist, pq_m, nbits):
        x = np.ascontiguousarray(data, dtype=np.float32)
        h = c_void_p()
        rc = self.lib.ovvsIvfPqBuild(self.res, _f32p(x), x.shape[0], x.shape[1], metric, nlist,
                                     pq_m, nbits, ctypes.byref(h))
        return rc, h

    def load(self, path):
        h = c_void_p()
        rc = self.lib.ovvsIvfPqDeserialize(self.res, str(path).encode(), ctypes.byref(h))
        return rc, h

    def save(self, h, path):
        return self.lib.ovvsIvfPqSerialize(h, str(path).encode())

    def extend(self, h, extra):
        x = np.ascontiguousarray(extra, dtype=np.float32)
        return self.lib.ovvsIvfPqExtend(self.res, h, _f32p(x), x.shape[0])

    def search(self, h, queries, k, nprobe, krefine, bitset=None):
        q = np.ascontiguousarray(queries, dtype=np.float32)
        nq = q.shape[0]
        ids = np.full((nq, k), -9, dtype=np.int64)
        d = np.full((nq, k), -9.0, dtype=np.float32)
        b = None if bitset is None else np.ascontiguousarray(bitset, dtype=np.uint8)
        rc = self.lib.ovvsIvfPqSearch(self.res, h, _f32p(q), nq, k, nprobe, krefine,
                                      None if b is None else b.ctypes.data_as(c_void_p),
                                      _i64p(ids), _f32p(d))
        return rc, ids, d

    def search_threads(self, h, queries, k, nprobe, krefine, threads):
        """The reference's documented concurrency model (include/ovvs/ovvs.h:165-166):
        `threads` threads, each with its own Resources (FORCE_CPU), search contiguous
        query shards of one shared index. ctypes releases the GIL during each call."""
        import threading

        q = np.ascontiguousarray(queries, dtype=np.float32)
        nq = q.shape[0]
        ids = np.full((nq, k), -9, dtype=np.int64)
        d = np.full((nq, k), -9.0, dtype=np.float32)
        bounds = np.linspace(0, nq, threads + 1).astype(np.int64)
        rcs = [0] * threads
        handles = []
        for _ in range(threads):
            r = c_void_p()
            assert self.lib.ovvsResourcesCreate(ctypes.byref(r)) == 0
            assert self.lib.ovvsResourcesSetPolicy(r, FORCE_CPU) == 0
            handles.append(r)

        def work(t):
            a, b = int(bounds[t]), int(bounds[t + 1])
            if b > a:
                rcs[t] = self.lib.ovvsIvfPqSearch(handles[t], h, _f32p(q[a:b]), b - a, k, nprobe,
                                                  krefine, None, _i64p(ids[a:b]), _f32p(d[a:b]))

        pool = [threading.Thread(target=work, args=(t,)) for t in range(threads)]
        for t in pool:
            t.start()
        for t in pool:
            t.join()
        for r in handles:
            self.lib.ovvsResourcesDestroy(r)
        rc = next((x for x in rcs if x != 0), 0)
        return rc, ids, d

    def destroy(self, h):
        if h:
            self.lib.ovvsIvfPqDestroy(h)

    def scann_build(self, data, metric, nlist, pq_m):
        x = np.ascontiguousarray(data, dtype=np.float32)
        h = c_void_p()
        rc = self.lib.ovvsScannBuild(self.res, _f32p(x), x.shape[0], x.shape[1], metric, nlist,
                                     pq_m, ctypes.byref(h))
        return rc, h

    def scann_search(self, h, queries, k, nprobe, krefine):
        q = np.ascontiguousarray(queries, dtype=np.float32)
        nq = q.shape[0]
        ids = np.full((nq, max(k, 0)), -9, dtype=np.int64)
        d = np.full((nq, max(k, 0)), -9.0, dtype=np.float32)
        rc = self.lib.ovvsScannSearch(self.res, h, _f32p(q), nq, k, nprobe, krefine, _i64p(ids),
                                      _f32p(d))
        return rc, ids, d

    def scann_destroy(self, h):
        if h:
            self.lib.ovvsScannDestroy(h)
