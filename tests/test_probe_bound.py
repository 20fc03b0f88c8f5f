"""The matrix-core probe's candidate bound against an emulation of its arithmetic (CPU).

The probe (ovvs_amd/csrc/probe.hip) ranks centroids by an approximate score
a'(q,c) = |c'|^2 - 2 (q^ . c^) with q^, c^ the bf16 roundings of the centred
coordinates fl(x - mu), and proves that every centroid whose a' exceeds the
P-th smallest group minimum by more than 2E cannot be among the exact first P.
That rests on |a'(q,c) + |q - mu|^2 - s(q,c)| <= E for every pair, where s is the
reference's fp32 score (sequential sums, reference src/prim/mixer.cpp:177-198).

Here a' is emulated independently of the kernel (bf16 round-to-nearest-even of
each centred coordinate, products and sums in float64, rounded to fp32 once: one
particular order of the matrix core's accumulation), s is computed with the
reference's sequential fp32 loops, and the observed error is checked against E
on data shaped like every benchmark configuration, including integer data in
[0, 255] and data far from the origin, where the centring matters. A factor lost
from E (say the 2 of the cross term) makes these checks fail.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

U = 2.0 ** -23
UM = 2.0 ** -20


def candidate_bound_E(qn, qcn, cn_max, ccn_max, dim, ksteps):
    """E of candidate_bound (probe.hip), per query, before t + 2E is formed."""
    n = dim + 4.0
    g = n * U / (1.0 - n * U)
    qd = qn * (1.0 + 4.0 * n * U)
    cd = cn_max * (1.0 + 4.0 * n * U)
    S = np.sqrt(qd * cd) * (1.0 + 1e-6)
    e2 = (g + 3 * U) * (qd + cd) + 2 * (g + U) * S + U * (qd + cd + 2 * S)
    qc = qcn * (1.0 + 4.0 * n * U)
    cc = ccn_max * (1.0 + 4.0 * n * U)
    Sc = np.sqrt(qc * cc) * (1.0 + 1e-6)
    m = 33.0 * ksteps + 8.0
    gm = m * UM / (1.0 - m * UM)
    ep = 2.0 ** -7 + 2.0 ** -16 + 3 * U
    e1 = (g + 5 * U) * cc + 2 * (ep + 1.02 * gm + 1.02 * U) * Sc + \
        m * 1e-30 * (1 + np.sqrt(qc) + np.sqrt(cc) + np.sqrt(qd) + np.sqrt(cd))
    return 1.01 * (e1 + e2)


def bf16(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def seqsum_sq(x):
    """Row-wise left-to-right fp32 sums of squares from +0."""
    s = np.zeros(x.shape[0], dtype=np.float32)
    for t in range(x.shape[1]):
        s = (s + x[:, t] * x[:, t]).astype(np.float32)
    return s


def ref_scores(Q, C):
    """(qn + cn) - 2 * dot with sequential fp32 sums (the reference's coarse score)."""
    qn, cn = seqsum_sq(Q), seqsum_sq(C)
    dot = np.zeros((Q.shape[0], C.shape[0]), dtype=np.float32)
    for t in range(Q.shape[1]):
        dot = (dot + np.outer(Q[:, t], C[:, t]).astype(np.float32)).astype(np.float32)
    return ((qn[:, None] + cn[None, :]).astype(np.float32) - np.float32(2) * dot).astype(np.float32), qn, cn


def check(Q, C):
    Q = np.ascontiguousarray(Q, dtype=np.float32)
    C = np.ascontiguousarray(C, dtype=np.float32)
    dim = Q.shape[1]
    mu = C.astype(np.float64).mean(0).astype(np.float32)
    Qc = (Q - mu).astype(np.float32)
    Cc = (C - mu).astype(np.float32)
    cnc = seqsum_sq(Cc)
    qcn = seqsum_sq(Qc)
    D = (bf16(Qc).astype(np.float64) @ bf16(Cc).astype(np.float64).T).astype(np.float32)
    a = (cnc[None, :] - np.float32(2) * D).astype(np.float32)
    s, qn, cn = ref_scores(Q, C)
    qdev = np.sum((Q.astype(np.float64) - mu.astype(np.float64)) ** 2, axis=1)
    err = np.abs(a.astype(np.float64) + qdev[:, None] - s.astype(np.float64))
    E = candidate_bound_E(qn.astype(np.float64), qcn.astype(np.float64), float(cn.max()),
                          float(cnc.max()), dim, math.ceil(dim / 32))
    ratio = err / E[:, None]
    assert np.all(ratio <= 1.0), f"bound exceeded: max err/E {ratio.max():.3f}"
    return float(ratio.max())


def _mixture(rng, n, dim, centers, sigma):
    return centers[rng.integers(0, len(centers), n)] + sigma * rng.standard_normal((n, dim))


@pytest.mark.parametrize("kind,dim", [("gauss", 96), ("gauss", 128), ("int255", 128),
                                      ("unit", 768), ("far", 32), ("gauss", 8)])
def test_bound_covers_emulated_error(kind, dim):
    rng = np.random.default_rng(dim + len(kind))
    centers = rng.standard_normal((64, dim))
    if kind == "int255":
        centers = rng.uniform(0, 255, (64, dim))
        C = np.clip(np.rint(_mixture(rng, 512, dim, centers, 12.0)), 0, 255)
        Q = np.clip(np.rint(_mixture(rng, 64, dim, centers, 12.0)), 0, 255)
    elif kind == "unit":
        C = _mixture(rng, 256, dim, centers, 0.4)
        Q = _mixture(rng, 32, dim, centers, 0.4)
        C /= np.linalg.norm(C, axis=1, keepdims=True)
        Q /= np.linalg.norm(Q, axis=1, keepdims=True)
    elif kind == "far":
        C = 1000.0 + _mixture(rng, 512, dim, centers, 0.3)
        Q = 1000.0 + _mixture(rng, 64, dim, centers, 0.3)
    else:
        C = _mixture(rng, 512, dim, centers, 0.25)
        Q = _mixture(rng, 64, dim, centers, 0.25)
    worst = check(Q, C)
    # The bound is worst-case over signs and accumulation orders; typical errors sit
    # well inside it (a bound orders of magnitude too loose would admit far too many
    # candidates: the GPU tests count the fallbacks).
    assert worst > 1e-4, f"bound suspiciously loose: max err/E {worst:.2e}"


def _aligned_rounding(dim):
    """Coordinates of magnitude 1 + 3 * 2^-10, which bf16 rounds down to 1: every
    product's rounding error has the same sign, so the errors add up instead of
    cancelling (the case the worst-case bound is built for)."""
    v = np.float32(1.0 + 3.0 * 2.0 ** -10)
    C = np.full((256, dim), v, dtype=np.float32)  # half along +1, half along -1: mu = 0
    C[128:] = -v
    Q = np.full((32, dim), v, dtype=np.float32)
    Q[16:] = -v
    return Q, C


def test_bound_is_nearly_tight_for_aligned_rounding():
    worst = check(*_aligned_rounding(64))
    assert worst > 0.5, f"max err/E {worst:.3f}"


def test_a_lost_factor_is_caught():
    """A bound short by a factor of 2 (a plausible slip: the 2 of the cross term
    dropped) fails on data whose rounding errors all share a sign."""
    global candidate_bound_E
    orig = candidate_bound_E
    Q, C = _aligned_rounding(64)

    def halved(qn, qcn, cn_max, ccn_max, dim, ksteps):
        return orig(qn, qcn, cn_max, ccn_max, dim, ksteps) / 2.0

    candidate_bound_E = halved
    try:
        with pytest.raises(AssertionError):
            check(Q, C)
    finally:
        candidate_bound_E = orig
    check(Q, C)
