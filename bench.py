#!/usr/bin/env python3
"""IVF-PQ search throughput on one MI355X — the BASELINE.json headline metric.

Workload (default config c2): 1M x 96 fp32 synthetic
Gaussian mixture (4096 centers, sigma 0.25, seed 1); IVF-PQ index with
n_lists=4096, pq_dim=48, 8-bit codes, built on the GPU by libovvs (quantizers
trained on a 262,144-row prefix, the rest appended with extend); search
n_probes=64, k=10, krefine=k, fp32 lookup tables, 10k-query batch.

A step is one ovvsIvfPqSearchDevice call over the whole batch with queries and
results already in HBM. value = queries / second over the timed steps.
The JSON line also carries:
  roofline      the dominant kernel, the code scan + select (k_scan). It reads
                only the code bytes of rows its lower bounds cannot rule out, so
                its busiest resource is VALU issue, not HBM: achieved = its VALU
                instructions per launch (rocprofv3 SQ_INSTS_VALU, committed under
                profiles/) over its average duration measured here (HIP events on
                the library's stream), against two wave64 VALU instructions per CU
                per clock (the fp32 vector peak); beside it the HBM fraction of its
                measured traffic and, labelled as such, the rate a full scan of the
                same code bytes would need;
  probe         the coarse probe on the matrix cores: the reference's GEMM flops
                (2 nq nlist dim) and the bf16 flops executed, over its duration;
  measured_peaks  streaming-read HBM GB/s, bf16 / fp32 MFMA TFLOP/s and VALU
                issue, measured on this GPU by ovvs_amd/lib/libovvs_peaks.so;
  cpu_baseline  the reference library's own CPU search (oracle/_ref, built
                from /root/reference) on the same index: the whole batch over
                --cpu-threads threads (one Resources each, the reference's
                concurrency model; `value`, `cores`) and one thread on a
                --cpu-sample prefix (`value_1_thread`);
  parity_vs_reference  the whole batch, GPU fp32-table answers against the
                reference's: identical rows, bit-identical distances;
  recall_at_k   against exact brute force (fp32 on the GPU, torch matmul);
  host_io       the same batch through the host-pointer ABI (ovvsIvfPqSearch,
                PCIe copies included), timed over the same number of steps;
  krefine_32    QPS and recall with a re-rank shortlist of 32 (the reference
                Python default) beside the configuration's krefine = k.
Progress lines go to stderr; stdout carries exactly one JSON line.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = ("IVF-PQ search QPS @k=10 (10k-query batch) at matched recall; "
          "scan HBM GB/s %peak")
HBM_PEAK_GBS = 8000.0
# MI355X: 256 CUs at 2.4 GHz; its 157.3 TFLOP/s fp32 vector peak (FMA = 2 flops) is
# 128 lanes per CU per clock, two wave64 fp32 VALU instructions per CU per clock.
VALU_PEAK_GINSTS = 157.3e3 / 2 / 64
MFMA_BF16_PEAK_TFLOPS = 2500.0
MFMA_F32_PEAK_TFLOPS = 157.3
T0 = time.time()


def log(*a):
    print(f"[bench {time.time() - T0:7.1f}s]", *a, file=sys.stderr, flush=True)


def exact_topk(base_t, q_t, k, torch):
    """Exact L2 top-k ids by fp32 matmul in chunks of the base (ground truth for recall)."""
    qn = (q_t * q_t).sum(1, keepdim=True)
    best_d = None
    best_i = None
    chunk = 131072
    for s in range(0, base_t.shape[0], chunk):
        b = base_t[s:s + chunk]
        d = qn + (b * b).sum(1)[None, :] - 2.0 * (q_t @ b.T)
        dv, di = torch.topk(d, k, dim=1, largest=False)
        di = di + s
        if best_d is None:
            best_d, best_i = dv, di
        else:
            cd = torch.cat([best_d, dv], 1)
            ci = torch.cat([best_i, di], 1)
            best_d, o = torch.topk(cd, k, dim=1, largest=False)
            best_i = torch.gather(ci, 1, o)
    return best_i.cpu().numpy()


def profile_value(profile, key):
    """A `key: value` figure of a committed rocprofv3 summary (profiles/<profile>.md)
    and the summary's path, or (None, None)."""
    path = ROOT / "profiles" / f"{profile}.md"
    if not path.exists():
        return None, None
    for line in path.read_text().splitlines():
        if line.startswith(f"{key}:"):
            return float(line.split(":", 1)[1]), str(path.relative_to(ROOT))
    return None, None


def measure_peaks(torch, dev):
    """Ceilings measured on this GPU (ovvs_amd/lib/libovvs_peaks.so): a 4 GiB
    streaming read (far beyond the 256 MB Infinity Cache), bf16 and fp32 MFMA and
    VALU issue loops; best of five launches each."""
    import ctypes

    path = ROOT / "ovvs_amd" / "lib" / "libovvs_peaks.so"
    if not path.exists():
        return None
    lib = ctypes.CDLL(str(path))
    for fn in ("peaks_hbm_read", "peaks_mfma_bf16", "peaks_mfma_f32", "peaks_valu"):
        getattr(lib, fn).restype = ctypes.c_double
    lib.peaks_hbm_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int]
    for fn in ("peaks_mfma_bf16", "peaks_mfma_f32", "peaks_valu"):
        getattr(lib, fn).argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
    scratch = torch.zeros(1 << 16, dtype=torch.float32, device=dev)
    buf = torch.ones(1 << 30, dtype=torch.float32, device=dev)  # 4 GiB
    torch.cuda.synchronize()
    out = {
        "hbm_read_GBps": lib.peaks_hbm_read(buf.data_ptr(), buf.numel() * 4, scratch.data_ptr(), 5),
        "mfma_bf16_TFLOPs": lib.peaks_mfma_bf16(scratch.data_ptr(), 4096, 5),
        "mfma_f32_TFLOPs": lib.peaks_mfma_f32(scratch.data_ptr(), 4096, 5),
        "valu_G_wave64_insts_per_s": lib.peaks_valu(scratch.data_ptr(), 16384, 5),
    }
    clock, cus = ctypes.c_int(0), ctypes.c_int(0)
    lib.peaks_device_info.argtypes = [ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]
    if lib.peaks_device_info(ctypes.byref(clock), ctypes.byref(cus)) == 0:
        out["clock_MHz"] = clock.value
        out["compute_units"] = cus.value
    del buf, scratch
    torch.cuda.synchronize()
    return out


def recall(got, truth):
    hits = 0
    for g, t in zip(got, truth):
        hits += len(set(int(x) for x in g if x >= 0) & set(int(x) for x in t))
    return hits / truth.size


def same_up_to_ties(ids_a, d_a, ids_b, d_b, rel=1e-5):
    """Rows where ids differ only at positions whose distances tie within rel."""
    bad = 0
    for ia, da, ib, db in zip(ids_a, d_a, ids_b, d_b):
        if np.array_equal(ia, ib):
            continue
        ok = True
        for t in np.nonzero(ia != ib)[0]:
            ref = max(abs(float(db[t])), 1e-30)
            if abs(float(da[t]) - float(db[t])) > rel * ref:
                ok = False
                break
        bad += not ok
    return bad


def cpu_baseline(index, queries, gpu_ids, gpu_d, k, nprobe, krefine, sample, threads,
                 lut_f16, ovvs_amd):
    """The reference library (oracle/_ref, FORCE_CPU) on this host: one thread on a
    `sample`-query prefix, then `threads` threads (one Resources each over query
    shards, the reference's concurrency model) on the whole batch. Parity compares
    the whole batch with the GPU's fp32-table results (for binary16-table configs
    the GPU search is repeated with fp32 tables, the reference's only precision)."""
    from oracle.pyoracle import REF_SO, Reference

    if not REF_SO.exists():
        return None, None
    with tempfile.TemporaryDirectory() as d:
        path = Path(d) / "bench.ipq1"
        log("cpu baseline: serializing index for the reference library")
        index.serialize(path)
        ref = Reference()
        rc, h = ref.load(path)
        if rc != 0:
            raise RuntimeError(f"reference deserialize failed: {rc}")
    q1 = np.ascontiguousarray(queries[:sample])
    log(f"cpu baseline: reference CPU search of {len(q1)} queries, 1 thread")
    ref.search(h, q1[:8], k, nprobe, krefine)  # warm-up
    t = time.perf_counter()
    rc, _, _ = ref.search(h, q1, k, nprobe, krefine)
    dt1 = time.perf_counter() - t
    if rc != 0:
        raise RuntimeError(f"reference search failed: {rc}")
    log(f"cpu baseline: reference CPU search of {len(queries)} queries, {threads} threads")
    t = time.perf_counter()
    rc, rids, rd = ref.search_threads(h, queries, k, nprobe, krefine, threads)
    dtn = time.perf_counter() - t
    if rc != 0:
        raise RuntimeError(f"reference threaded search failed: {rc}")
    ref.destroy(h)
    ref.close()
    if lut_f16:
        gpu_ids, gpu_d = index.search_ex(queries, k, nprobe, krefine,
                                         lut_dtype=ovvs_amd.DTYPE_F32)
    exact_rows = int(np.sum(np.all(rids == gpu_ids, axis=1)))
    bits_equal = bool(np.array_equal(np.ascontiguousarray(gpu_d).view(np.uint32),
                                     np.ascontiguousarray(rd).view(np.uint32)))
    mism = same_up_to_ties(gpu_ids, gpu_d, rids, rd)
    fin = np.isfinite(rd)
    dist_err = float(np.max(np.abs(gpu_d[fin].astype(np.float64) - rd[fin]) /
                            np.maximum(1.0, np.abs(rd[fin])))) if fin.any() else 0.0
    base = {"value": len(queries) / dtn, "unit": "queries/s", "cores": threads,
            "kind": "reference",
            "sample": f"the whole {len(queries)}-query batch over {threads} threads "
                      f"({dtn:.1f} s wall), same index, reference ovvsIvfPqSearch FORCE_CPU",
            "value_1_thread": len(q1) / dt1,
            "sample_1_thread": f"first {len(q1)} queries, 1 thread ({dt1:.1f} s)",
            "host_nproc": os.cpu_count(), "host_cpu_model": cpu_model()}
    parity = {"queries": len(queries), "tables": "f32",
              "rows_identical": exact_rows, "distances_bit_identical": bits_equal,
              "rows_differing_beyond_ties": mism, "max_rel_distance_error": dist_err}
    return base, parity


def cpu_baseline_port(index, base, queries, gpu_ids, gpu_d, k, nprobe, krefine, sample, threads):
    """Our C restatement of the reference CPU search (oracle/liboracle.so) on this host,
    for indexes whose IPQ1 file the reference library would have to load from disk
    (C5: 43 GB): the library serializes the index into a pipe, the reader keeps every
    section but the dataset, and the bench's own rows stand in for it. Timed on the
    first `sample` queries over `threads` threads (and a tenth of them on one thread);
    parity is checked on the same queries."""
    import threading

    from oracle.pyoracle import ORACLE_SO, Oracle, read_ipq1_stream

    if not ORACLE_SO.exists():
        return None, None
    log("cpu baseline (port): streaming the index out of the library")
    with tempfile.TemporaryDirectory() as d:
        fifo = Path(d) / "index.pipe"
        os.mkfifo(fifo)
        errs = []

        def writer():
            try:
                index.serialize(fifo)
            except Exception as e:  # noqa: BLE001 (reported after the join)
                errs.append(e)

        th = threading.Thread(target=writer)
        th.start()
        with open(fifo, "rb", buffering=1 << 20) as f:
            try:
                ipq = read_ipq1_stream(f, base)
            except Exception:
                while f.read(1 << 26):
                    pass
                th.join()
                raise
        th.join()
        if errs:
            raise errs[0]
    orc = Oracle(ipq)
    q = np.ascontiguousarray(queries[:sample])
    n1 = max(1, sample // 10)
    log(f"cpu baseline (port): oracle search of {n1} queries, 1 thread")
    t = time.perf_counter()
    orc.search(q[:n1], k, nprobe, krefine)
    dt1 = time.perf_counter() - t
    log(f"cpu baseline (port): oracle search of {sample} queries, {threads} threads")
    t = time.perf_counter()
    oids, od = orc.search_threads(q, k, nprobe, krefine, threads)
    dtn = time.perf_counter() - t
    g_ids, g_d = gpu_ids[:sample], gpu_d[:sample]
    base_rec = {"value": sample / dtn, "unit": "queries/s", "cores": threads, "kind": "port",
                "sample": f"first {sample} queries of the batch over {threads} threads "
                          f"({dtn:.1f} s wall), same index (streamed out of the library, "
                          f"dataset rows from memory), oracle/ivfpq_oracle.c",
                "value_1_thread": n1 / dt1,
                "sample_1_thread": f"first {n1} queries, 1 thread ({dt1:.1f} s)",
                "host_nproc": os.cpu_count(), "host_cpu_model": cpu_model()}
    fin = np.isfinite(od)
    parity = {"queries": sample, "checker": "oracle", "tables": "f32",
              "rows_identical": int(np.sum(np.all(oids == g_ids, axis=1))),
              "distances_bit_identical": bool(np.array_equal(
                  np.ascontiguousarray(g_d).view(np.uint32), np.ascontiguousarray(od).view(np.uint32))),
              "rows_differing_beyond_ties": same_up_to_ties(g_ids, g_d, oids, od),
              "max_rel_distance_error": float(np.max(np.abs(g_d[fin].astype(np.float64) - od[fin]) /
                                                     np.maximum(1.0, np.abs(od[fin])))) if fin.any() else 0.0}
    return base_rec, parity


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), or None."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def _fill_rows(shm_name, shape, cfg, C, a, b):
    from multiprocessing import shared_memory

    from ovvs_amd import synth

    shm = shared_memory.SharedMemory(name=shm_name)
    out = np.ndarray(shape, dtype=np.float32, buffer=shm.buf)
    for s in range(a, b, 65536):
        e = min(b, s + 65536)
        out[s:e] = synth.base_rows(cfg, s, e - s, C)
    del out
    shm.close()


def generate_base(cfg, C, workers):
    """The config's base rows. Large configs are generated by `workers` forked
    processes into shared memory (each row is a pure function of its index, so
    the result is the same as the single-process generator); returns the array and
    the shared-memory handle to release (None for the in-process path)."""
    from ovvs_amd import synth

    nbytes = cfg.n * cfg.dim * 4
    if nbytes < (2 << 30) or workers <= 1:
        return synth.base_rows(cfg, 0, cfg.n, C), None
    from multiprocessing import get_context, shared_memory

    shm = shared_memory.SharedMemory(create=True, size=nbytes)
    shape = (cfg.n, cfg.dim)
    bounds = np.linspace(0, cfg.n, 4 * workers + 1).astype(np.int64)
    ctx = get_context("fork")
    pending = [(int(bounds[i]), int(bounds[i + 1])) for i in range(len(bounds) - 1)]
    running = []
    while pending or running:
        while pending and len(running) < workers:
            a, b = pending.pop(0)
            pr = ctx.Process(target=_fill_rows, args=(shm.name, shape, cfg, C, a, b))
            pr.start()
            running.append(pr)
        pr = running.pop(0)
        pr.join()
        if pr.exitcode != 0:
            shm.close()
            shm.unlink()
            raise RuntimeError("base row generation failed")
        log(f"generated rows: {len(bounds) - 1 - len(pending) - len(running)}/{len(bounds) - 1} "
            f"slices")
    return np.ndarray(shape, dtype=np.float32, buffer=shm.buf), shm


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c2")
    ap.add_argument("--no-small-batches", action="store_true",
                    help="skip the 1- and 100-query batches (profiling runs)")
    ap.add_argument("--nq", type=int, default=None, help="query batch (default: config's)")
    ap.add_argument("--rows", type=int, default=None,
                    help="base rows (default: config's; a prefix of its stream)")
    ap.add_argument("--krefine", type=int, default=None, help="default: k")
    ap.add_argument("--cpu-sample", type=int, default=1000,
                    help="queries of the single-thread reference timing")
    ap.add_argument("--cpu-threads", type=int, default=min(16, os.cpu_count() or 1),
                    help="threads of the whole-batch reference timing")
    ap.add_argument("--gen-workers", type=int, default=min(16, os.cpu_count() or 1),
                    help="processes generating the base rows of large configs")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-kind", choices=("auto", "reference", "port"), default="auto",
                    help="CPU baseline and parity checker: the reference library (it loads an "
                         "IPQ1 file), our C oracle on in-memory arrays, or auto (the reference "
                         "below 8 GiB of vectors)")
    ap.add_argument("--no-recall", action="store_true")
    ap.add_argument("--no-peaks", action="store_true", help="skip the measured-peak kernels")
    ap.add_argument("--no-host-io", action="store_true",
                    help="skip the host-pointer (PCIe-inclusive) timing")
    ap.add_argument("--extra-krefine", type=int, default=32,
                    help="also time and score this krefine (0: skip)")
    ap.add_argument("--unclustered", action="store_true",
                    help="isotropic N(0, I) rows and queries of the config's shape (no "
                         "clusters: the scan's worst case)")
    ap.add_argument("--calibrate-copy-mb", type=int, default=0,
                    help="run one device-to-device copy and one elementwise copy of this many "
                         "MiB before the timed steps (known-size kernels that scale rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one MI355X: this build runs on a single GPU; "
              "multi-GPU sharding is a design, not built", file=sys.stderr)
        return 2

    import torch

    import ovvs_amd
    from ovvs_amd import synth

    import dataclasses

    cfg = synth.CONFIGS[args.config]
    if args.rows:
        cfg = dataclasses.replace(cfg, n=args.rows, train_rows=min(cfg.train_rows, args.rows))
    if args.unclustered:
        cfg = dataclasses.replace(cfg, kind="iso")
    nq = args.nq or cfg.nq
    k = cfg.k
    krefine = args.krefine or k
    lut = ovvs_amd.DTYPE_F16 if cfg.lut_f16 else ovvs_amd.DTYPE_F32
    log(f"config {cfg.name}: n={cfg.n} dim={cfg.dim} nlist={cfg.nlist} pq_m={cfg.pq_m} "
        f"nprobe={cfg.nprobe} k={k} krefine={krefine} nq={nq}")
    C = synth.centers(cfg)
    # Forked generator processes: no HIP runtime has been initialised yet.
    base, shm = generate_base(cfg, C, args.gen_workers)
    queries = synth.query_rows(cfg, 0, nq, C)
    log("data generated")
    try:
        return run(args, torch, ovvs_amd, cfg, nq, k, krefine, lut, base, queries)
    finally:
        if shm is not None:
            del base
            shm.close()
            shm.unlink()


def run(args, torch, ovvs_amd, cfg, nq, k, krefine, lut, base, queries) -> int:

    res = ovvs_amd.Resources()
    t = time.perf_counter()
    index = ovvs_amd.neighbors.ivf_pq.build(base[:cfg.train_rows], metric=cfg.metric,
                                            nlist=cfg.nlist, pq_m=cfg.pq_m, pq_nbits=8,
                                            resources=res)
    index.extend(base[cfg.train_rows:])
    log(f"index built on the GPU in {time.perf_counter() - t:.1f} s")

    dev = torch.device("cuda:0")
    dq = torch.from_numpy(queries).to(dev)
    did = torch.empty((nq, k), dtype=torch.int64, device=dev)
    dd = torch.empty((nq, k), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()

    def step():
        index.search_device(dq.data_ptr(), nq, k, cfg.nprobe, krefine, did.data_ptr(),
                            dd.data_ptr(), lut_dtype=lut)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    log(f"{args.warmup} warmup steps done")
    if args.calibrate_copy_mb > 0:
        count = args.calibrate_copy_mb * (1 << 20) // 4
        src = torch.ones(count, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)                     # device-to-device copy kernel
        torch.mul(src, 2.0, out=dst)       # elementwise kernel: reads and writes count*4 bytes
        torch.cuda.synchronize()
        log(f"calibration copies of {args.calibrate_copy_mb} MiB done")
        del src, dst
    s0 = res.ivfpq_search_stats()
    h0 = res.ivfpq_table_queries()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    s1 = res.ivfpq_search_stats()
    table_queries = (res.ivfpq_table_queries() - h0) / args.steps
    elapsed = t1 - t0
    qps = nq * args.steps / elapsed
    log(f"{args.steps} timed steps: {elapsed * 1e3 / args.steps:.3f} ms/step, {qps:,.0f} QPS, "
        f"{table_queries:.0f} queries per step handed to the full-table scan")

    # Smaller batches of the same queries (the config's other batch sizes; reported
    # beside `value`, which is the whole batch).
    small = {}
    for b in (() if args.no_small_batches else (1, 100)):
        if b >= nq:
            continue
        for _ in range(3):
            index.search_device(dq[:b].data_ptr(), b, k, cfg.nprobe, krefine, did[:b].data_ptr(),
                                dd[:b].data_ptr(), lut_dtype=lut)
        torch.cuda.synchronize()
        reps = 50
        tb = time.perf_counter()
        for _ in range(reps):
            index.search_device(dq[:b].data_ptr(), b, k, cfg.nprobe, krefine, did[:b].data_ptr(),
                                dd[:b].data_ptr(), lut_dtype=lut)
        torch.cuda.synchronize()
        small[str(b)] = {"queries_per_s": b * reps / (time.perf_counter() - tb),
                         "ms_per_batch": (time.perf_counter() - tb) * 1e3 / reps}
    if small:
        log("smaller batches: " + ", ".join(f"{b}: {v['queries_per_s']:,.0f} QPS" for b, v in small.items()))
    # The timed batch's results again (the small batches wrote into the output buffers).
    step()
    torch.cuda.synchronize()

    dsd = {key: s1[key] - s0[key] for key in s1 if isinstance(s1[key], int)}
    calls = dsd["successful_calls"]
    scan_s = dsd["adc_scan_select_ns"] / calls * 1e-9
    probe_s = dsd["coarse_pairwise_ns"] / calls * 1e-9
    code_bytes = dsd["candidate_rows"] / calls * cfg.pq_m
    stage_ms = {name: dsd[f"{name}_ns"] / calls * 1e-6
                for name in ("coarse_pairwise", "coarse_topk", "adc_scan_select",
                             "refine_distance", "total_wall")}
    gpu_ids = did.cpu().numpy()
    gpu_d = dd.cpu().numpy()

    # The host-pointer ABI over the same number of steps (PCIe copies of queries
    # and results included; reported beside `value`, never as it).
    host = None
    if not args.no_host_io:
        for _ in range(2):
            hids, hd = index.search_ex(queries, k, cfg.nprobe, krefine, lut_dtype=lut)
        t = time.perf_counter()
        for _ in range(args.steps):
            hids, hd = index.search_ex(queries, k, cfg.nprobe, krefine, lut_dtype=lut)
        dt = time.perf_counter() - t
        if not (np.array_equal(hids, gpu_ids) and np.array_equal(hd, gpu_d)):
            raise AssertionError("host-pointer and device-pointer searches disagree")
        host = {"queries_per_s": nq * args.steps / dt, "ms_per_step": dt * 1e3 / args.steps,
                "steps": args.steps}
        log(f"host-pointer ABI: {host['ms_per_step']:.3f} ms/step, {host['queries_per_s']:,.0f} QPS")

    truth = None
    rec = None
    if not args.no_recall:
        truth = exact_topk(torch.from_numpy(base).to(dev), dq, k, torch)
        rec = recall(gpu_ids, truth)
        log(f"recall@{k} vs exact = {rec:.4f}")

    extra = None
    if args.extra_krefine and args.extra_krefine != krefine:
        kr2 = max(args.extra_krefine, k)
        for _ in range(2):
            index.search_device(dq.data_ptr(), nq, k, cfg.nprobe, kr2, did.data_ptr(),
                                dd.data_ptr(), lut_dtype=lut)
        torch.cuda.synchronize()
        steps2 = max(1, args.steps // 2)
        t = time.perf_counter()
        for _ in range(steps2):
            index.search_device(dq.data_ptr(), nq, k, cfg.nprobe, kr2, did.data_ptr(),
                                dd.data_ptr(), lut_dtype=lut)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t
        extra = {"krefine": kr2, "queries_per_s": nq * steps2 / dt,
                 "ms_per_step": dt * 1e3 / steps2, "steps": steps2,
                 "recall_at_k": recall(did.cpu().numpy(), truth) if truth is not None else None}
        log(f"krefine {kr2}: {extra['ms_per_step']:.3f} ms/step, recall {extra['recall_at_k']}")

    peaks = None if args.no_peaks else measure_peaks(torch, dev)
    if peaks:
        log("measured peaks: " + ", ".join(f"{a} {b:,.1f}" for a, b in peaks.items()))

    # Roofline of the dominant kernel (the scan) from its committed counters.
    prof = f"k_scan_{cfg.name}" + ("_unclustered" if args.unclustered else "")
    valu, valu_src = profile_value(prof, "valu_insts_per_launch")
    traffic, traffic_src = profile_value(prof, "traffic_bytes_per_launch")
    roof = {
        "kernel": "k_scan (segment-bounded code scan + shortlist)",
        "bound": "valu",
        "unit": "G wave64 VALU instructions/s",
        "achieved": valu / scan_s / 1e9 if valu else None,
        "peak": VALU_PEAK_GINSTS,
        "frac": valu / scan_s / 1e9 / VALU_PEAK_GINSTS if valu else None,
        "valu_insts_per_launch": valu,
        "avg_launch_ms": scan_s * 1e3,
        "traffic": traffic,
        "hbm_GBps": traffic / scan_s / 1e9 if traffic else None,
        "hbm_frac": traffic / scan_s / 1e9 / HBM_PEAK_GBS if traffic else None,
        "counters_source": valu_src or traffic_src,
        "algorithmic_equivalent": {
            "note": "code bytes a full scan of every probed list reads (candidate_rows x "
                    "pq_dim, each (query, list) pair counted); the scan reads only rows its "
                    "lower bounds cannot rule out, so this rate is not an HBM figure",
            "bytes_per_launch": code_bytes,
            "GBps": code_bytes / scan_s / 1e9,
        },
    }
    if peaks and roof["achieved"]:
        roof["peak_measured"] = peaks["valu_G_wave64_insts_per_s"]
        roof["frac_measured"] = roof["achieved"] / peaks["valu_G_wave64_insts_per_s"]
    if peaks and roof["hbm_GBps"]:
        roof["hbm_frac_measured"] = roof["hbm_GBps"] / peaks["hbm_read_GBps"]
    gemm_flops = 2.0 * nq * cfg.nlist * cfg.dim
    bf16_flops, bf16_src = profile_value(f"k_probe_mfma_{cfg.name}", "bf16_flops_per_launch")
    probe = {
        "kernel": "k_probe_mfma (coarse probe on the matrix cores, exact by proof)",
        "bound": "mfma",
        "avg_launch_ms": probe_s * 1e3,
        "gemm_flops_per_launch": gemm_flops,
        "achieved_TFLOPs": gemm_flops / probe_s / 1e12,
        "frac_of_fp32_mfma_peak": gemm_flops / probe_s / 1e12 / MFMA_F32_PEAK_TFLOPS,
        "bf16_flops_executed_per_launch": bf16_flops,
        "bf16_TFLOPs": bf16_flops / probe_s / 1e12 if bf16_flops else None,
        "frac_of_bf16_mfma_peak": bf16_flops / probe_s / 1e12 / MFMA_BF16_PEAK_TFLOPS
        if bf16_flops else None,
        "counters_source": bf16_src,
    }

    cpu, parity = (None, None)
    if not args.no_cpu_baseline:
        kind = args.cpu_kind
        if kind == "auto":
            kind = "reference" if cfg.n * cfg.dim * 4 < (8 << 30) else "port"
        if kind == "reference":
            cpu, parity = cpu_baseline(index, queries, gpu_ids, gpu_d, k, cfg.nprobe, krefine,
                                       min(args.cpu_sample, nq), args.cpu_threads, cfg.lut_f16,
                                       ovvs_amd)
        else:
            cpu, parity = cpu_baseline_port(index, base, queries, gpu_ids, gpu_d, k, cfg.nprobe,
                                            krefine, min(args.cpu_sample, nq), args.cpu_threads)
        if cpu:
            log(f"cpu baseline {cpu['value']:,.1f} QPS; parity {parity}")

    line = {
        "metric": METRIC,
        "value": qps,
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": elapsed * 1e3 / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"ivfpq_{cfg.name}{'_unclustered' if args.unclustered else ''}_"
                        f"{cfg.n}x{cfg.dim}_nlist{cfg.nlist}_pq{cfg.pq_m}x8_"
                        f"nprobe{cfg.nprobe}_k{k}_nq{nq}_{'f16' if cfg.lut_f16 else 'f32'}lut",
            "lut_requested": "f16" if cfg.lut_f16 else "f32",
            "lut_computed": "f32",
            "n": cfg.n, "dim": cfg.dim, "nlist": cfg.nlist, "pq_dim": cfg.pq_m, "pq_bits": 8,
            "n_probes": cfg.nprobe, "k": k, "krefine": krefine, "batch": nq,
            "train_rows": cfg.train_rows, "parallelism": "single-gpu",
        },
        "roofline": roof,
        "probe": probe,
        "measured_peaks": peaks,
        "cpu_baseline": cpu,
        "stage_ms": stage_ms,
        "table_queries_per_step": table_queries,
        "smaller_batches": small,
        "host_io": host,
        "recall_at_k": rec,
        "krefine_32": extra,
        "recall_k": k,
        "parity_vs_reference": parity,
    }
    print(json.dumps(line), flush=True)
    index.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
