"""Seeded synthetic workloads for the IVF-PQ configurations (test and bench data).

Counter-based: every value is a pure function of (seed, stream, index), so any
row of any configuration can be regenerated independently (chunked generation of
large configs, CPU subsets of GPU workloads). A 64-bit SplitMix64 finalizer hashes
the counter; each normal draw takes one hash, splits it into two 32-bit uniforms
and applies Box-Muller in float64, then the row is formed in float32.

Configurations (BASELINE.json "configs"):
  c1  100k x 128, 1024 centers ~N(0,1), sigma 0.3, seed 0        (CPU-runnable)
  c2  1M x 96, 4096 centers ~N(0,1), sigma 0.25, seed 1          (headline)
  c3  10M x 128, 8192 centers ~U[0,255], sigma 12, rounded and clipped to [0,255], seed 2
  c4  1M x 768, 2048 centers ~N(0,1), x = normalize(center + 0.4 N), seed 3
  c5  100M x 96, 65536 centers ~N(0,1), sigma 0.25, seed 4
Queries are drawn from the same mixture on separate streams. Any configuration with
kind "iso" draws rows and queries from N(0, I) instead (no cluster structure: the
scan's lower bounds rule out little, its worst case).
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

STREAM_CENTERS = 1
STREAM_BASE_PICK = 2
STREAM_BASE_NOISE = 3
STREAM_QUERY_PICK = 4
STREAM_QUERY_NOISE = 5


def _mix64(z: np.ndarray) -> np.ndarray:
    z = z.copy()
    z ^= z >> np.uint64(30)
    z *= _M1
    z ^= z >> np.uint64(27)
    z *= _M2
    z ^= z >> np.uint64(31)
    return z


def _stream_key(seed: int, stream: int) -> np.uint64:
    base = np.array([(int(seed) * 0x100000001B3 + int(stream) * 0x9E3779B97F4A7C15)
                     & 0xFFFFFFFFFFFFFFFF], dtype=np.uint64)
    return _mix64(base)[0]


def hashes(seed: int, stream: int, start: int, count: int) -> np.ndarray:
    idx = np.arange(start, start + count, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix64(idx * _GOLDEN + _stream_key(seed, stream))


def uniform(seed: int, stream: int, start: int, count: int) -> np.ndarray:
    """float64 in (0, 1)."""
    h = hashes(seed, stream, start, count)
    return ((h >> np.uint64(11)).astype(np.float64) + 0.5) * (1.0 / 9007199254740992.0)


def normal(seed: int, stream: int, start: int, count: int) -> np.ndarray:
    """float64 standard normal draws."""
    h = hashes(seed, stream, start, count)
    u1 = ((h >> np.uint64(32)).astype(np.float64) + 0.5) * (1.0 / 4294967296.0)
    u2 = ((h & np.uint64(0xFFFFFFFF)).astype(np.float64) + 0.5) * (1.0 / 4294967296.0)
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


@dataclass(frozen=True)
class Config:
    name: str
    n: int
    dim: int
    ncenters: int
    sigma: float
    seed: int
    kind: str          # "gauss", "int255", "unit" or "iso" (isotropic N(0, I), no clusters)
    nq: int
    nlist: int
    pq_m: int
    nprobe: int
    k: int
    lut_f16: bool
    metric: int        # ovvsMetric
    train_rows: int    # rows the coarse/PQ quantizers are trained on (a prefix)


CONFIGS = {
    "c1": Config("c1", 100_000, 128, 1024, 0.3, 0, "gauss", 1_000, 256, 32, 16, 10, False, 0,
                 20_000),
    "c2": Config("c2", 1_000_000, 96, 4096, 0.25, 1, "gauss", 10_000, 4096, 48, 64, 10, False, 0,
                 262_144),
    "c3": Config("c3", 10_000_000, 128, 8192, 12.0, 2, "int255", 10_000, 16384, 64, 128, 100, True,
                 0, 1_048_576),
    "c4": Config("c4", 1_000_000, 768, 2048, 0.4, 3, "unit", 10_000, 2048, 96, 32, 10, True, 2,
                 262_144),
    "c5": Config("c5", 100_000_000, 96, 65536, 0.25, 4, "gauss", 10_000, 65536, 48, 256, 10, True,
                 0, 4_194_304),
}


def centers(cfg: Config) -> np.ndarray:
    count = cfg.ncenters * cfg.dim
    if cfg.kind == "int255":
        c = uniform(cfg.seed, STREAM_CENTERS, 0, count) * 255.0
    else:
        c = normal(cfg.seed, STREAM_CENTERS, 0, count)
    return c.astype(np.float32).reshape(cfg.ncenters, cfg.dim)


def _rows(cfg: Config, C: np.ndarray, start: int, count: int, pick_stream: int,
          noise_stream: int) -> np.ndarray:
    pick = np.minimum((uniform(cfg.seed, pick_stream, start, count) * cfg.ncenters).astype(np.int64),
                      cfg.ncenters - 1)
    noise = normal(cfg.seed, noise_stream, start * cfg.dim, count * cfg.dim).reshape(count, cfg.dim)
    if cfg.kind == "iso":
        return noise.astype(np.float32)
    base = C[pick]
    if cfg.kind == "int255":
        x = np.clip(np.rint(base.astype(np.float64) + cfg.sigma * noise), 0.0, 255.0)
        return x.astype(np.float32)
    if cfg.kind == "unit":
        x = base.astype(np.float64) + cfg.sigma * noise
        x /= np.linalg.norm(x, axis=1, keepdims=True)
        return x.astype(np.float32)
    return base + (cfg.sigma * noise).astype(np.float32)


def base_rows(cfg: Config, start: int, count: int, C: np.ndarray | None = None,
              chunk: int = 65536) -> np.ndarray:
    C = centers(cfg) if C is None else C
    out = np.empty((count, cfg.dim), dtype=np.float32)
    for s in range(0, count, chunk):
        m = min(chunk, count - s)
        out[s:s + m] = _rows(cfg, C, start + s, m, STREAM_BASE_PICK, STREAM_BASE_NOISE)
    return out


def query_rows(cfg: Config, start: int, count: int, C: np.ndarray | None = None) -> np.ndarray:
    C = centers(cfg) if C is None else C
    return _rows(cfg, C, start, count, STREAM_QUERY_PICK, STREAM_QUERY_NOISE)


def lcg_data(n: int, dim: int, seed: int) -> np.ndarray:
    """The reference tests' deterministic LCG inputs (reference tests/test_harness.hpp:71-79):
    s = s*1664525 + 1013904223 (mod 2^32), value = ((s >> 16) % 2000) / 1000 - 1 in float32."""
    out = np.empty(n * dim, dtype=np.float32)
    s = int(seed) & 0xFFFFFFFF
    vals = np.empty(n * dim, dtype=np.int64)
    for i in range(n * dim):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        vals[i] = (s >> 16) % 2000
    out[:] = vals.astype(np.float32) / np.float32(1000.0) - np.float32(1.0)
    return out.reshape(n, dim)
