"""ovvsIvfPqSearchDeviceNoAlloc against ovvsIvfPqSearchDevice, through the C ABI.

The no-allocation entry point carves its workspace from the library's fixed
device scratch instead of the Resources' workspace; its results must be the
device-pointer search's, bit for bit, on consecutive calls (the second with a
smaller batch, so stale scratch contents from the first cannot go unnoticed),
and it must refuse what it cannot serve without allocating.
"""

from __future__ import annotations

import ctypes
import sys
from ctypes import c_int32, c_int64, c_void_p

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True, file=sys.stderr)


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def _call(lib, fn, res, ix, dq, nq, k, nprobe, krefine, did, dd, bits=None):
    return getattr(lib, fn)(res._h, ix._h, c_void_p(dq), c_int64(nq), c_int64(k), c_int32(nprobe),
                            c_int32(krefine), c_void_p(bits or 0), c_int32(0), c_void_p(did),
                            c_void_p(dd))


def test_no_alloc_matches_device_entry(ovvs, tmp_path):
    import torch

    res = ovvs.Resources()
    if not res.gpu_available():
        pytest.fail("no GPU visible: gpu tests must run on the MI355X box")
    lib = ovvs._lib
    rng = np.random.default_rng(5)
    dim, n, nlist, pq_m = 48, 40000, 128, 24
    centers = rng.standard_normal((64, dim)).astype(np.float32)
    data = (centers[rng.integers(0, 64, n)] + 0.3 * rng.standard_normal((n, dim))).astype(
        np.float32)
    q = (centers[rng.integers(0, 64, 3000)] + 0.3 * rng.standard_normal((3000, dim))).astype(
        np.float32)
    say("no-alloc: build", dict(n=n, dim=dim, nlist=nlist, pq_m=pq_m))
    ix = ovvs.neighbors.ivf_pq.build(data, nlist=nlist, pq_m=pq_m, pq_nbits=8, resources=res)
    dq = torch.from_numpy(q).to("cuda:0")
    bitset = np.packbits((rng.random(n) < 0.6).astype(np.uint8), bitorder="little")
    dbits = torch.from_numpy(bitset).to("cuda:0")
    torch.cuda.synchronize()

    # Before the index has a device copy nothing can be served without allocating.
    k = 10
    did = torch.full((3000, k), -7, dtype=torch.int64, device="cuda:0")
    dd = torch.full((3000, k), -7.0, dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    rc = _call(lib, "ovvsIvfPqSearchDeviceNoAlloc", res, ix, dq.data_ptr(), 100, k, 8, 32,
               did.data_ptr(), dd.data_ptr())
    assert rc == ovvs.STATUS_INVALID_ARGUMENT
    assert torch.all(did == -7).item() and torch.all(dd == -7.0).item()

    # Two calls in a row with different shapes, the second smaller; then the
    # first shape again (the scratch keeps the previous call's contents).
    cases = [(3000, 10, 16, 64, False), (700, 5, 4, 5, True), (3000, 10, 16, 64, False),
             (1, 1, 1, 1, False)]
    for nq, kk, nprobe, krefine, use_bits in cases:
        say("no-alloc case", dict(nq=nq, k=kk, nprobe=nprobe, krefine=krefine, bitset=use_bits))
        bp = dbits.data_ptr() if use_bits else None
        rid = torch.empty((nq, kk), dtype=torch.int64, device="cuda:0")
        rd = torch.empty((nq, kk), dtype=torch.float32, device="cuda:0")
        nid = torch.full((nq, kk), -9, dtype=torch.int64, device="cuda:0")
        nd = torch.full((nq, kk), -9.0, dtype=torch.float32, device="cuda:0")
        torch.cuda.synchronize()
        rc = _call(lib, "ovvsIvfPqSearchDevice", res, ix, dq.data_ptr(), nq, kk, nprobe, krefine,
                   rid.data_ptr(), rd.data_ptr(), bp)
        assert rc == ovvs.STATUS_SUCCESS
        rc = _call(lib, "ovvsIvfPqSearchDeviceNoAlloc", res, ix, dq.data_ptr(), nq, kk, nprobe,
                   krefine, nid.data_ptr(), nd.data_ptr(), bp)
        assert rc == ovvs.STATUS_SUCCESS
        a_ids, b_ids = rid.cpu().numpy(), nid.cpu().numpy()
        assert np.array_equal(a_ids, b_ids)
        assert np.array_equal(_bits(rd.cpu().numpy()), _bits(nd.cpu().numpy()))
        assert np.all(a_ids[:, 0] >= 0)

    # The allocation counters of the telemetry do not move for no-alloc calls.
    before = res.ivfpq_search_stats()
    rc = _call(lib, "ovvsIvfPqSearchDeviceNoAlloc", res, ix, dq.data_ptr(), 700, 5, 4, 5,
               did.data_ptr(), dd.data_ptr())
    assert rc == ovvs.STATUS_SUCCESS
    after = res.ivfpq_search_stats()
    assert after["successful_calls"] == before["successful_calls"] + 1
    assert after["gpu_allocation_calls"] == before["gpu_allocation_calls"]
    assert after["gpu_allocation_bytes"] == before["gpu_allocation_bytes"]

    # A batch whose workspace exceeds the scratch is refused, outputs untouched.
    # krefine 1024: 12 KiB of shortlist per query, 6000 queries hold 72 MiB.
    big_nq = 6000
    assert big_nq * 12 * 1024 > ovvs.NOALLOC_SCRATCH_BYTES
    big_q = torch.zeros((big_nq, dim), dtype=torch.float32, device="cuda:0")
    bid = torch.full((big_nq, 1), -3, dtype=torch.int64, device="cuda:0")
    bd = torch.full((big_nq, 1), -3.0, dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    rc = _call(lib, "ovvsIvfPqSearchDeviceNoAlloc", res, ix, big_q.data_ptr(), big_nq, 1, 16,
               1024, bid.data_ptr(), bd.data_ptr())
    assert rc == ovvs.STATUS_SHAPE_MISMATCH
    assert torch.all(bid == -3).item() and torch.all(bd == -3.0).item()
    ix.close()
    res.close()
