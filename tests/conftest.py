"""Shared pytest setup.

Markers: ``gpu`` tests need a HIP device and run on the MI355X box
(``pytest -m gpu``); everything else runs on the CPU (``pytest -m "not gpu"``).
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import pytest

try:
    # libovvs and torch-ROCm each bring a libamdhip64.so.7; the first one loaded
    # serves the whole process. Loading torch's first keeps torch usable in the
    # GPU tests that allocate device memory through it.
    import torch  # noqa: F401
except ImportError:
    pass

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) to run")


@pytest.fixture(scope="session")
def ovvs():
    import ovvs_amd

    return ovvs_amd


@pytest.fixture(scope="session")
def ref_cases():
    """Golden cases answered by the reference library (tests/golden/make_fixtures.py)."""
    manifest = json.loads((GOLDEN / "ref_cases.json").read_text())
    arrays = np.load(GOLDEN / "ref_cases.npz")
    return manifest, {k: arrays[k] for k in arrays.files}


def case_data(case, arrays, key="data"):
    from ovvs_amd.synth import lcg_data

    lcg = case.get(f"{key}_lcg")
    if lcg is not None:
        return lcg_data(*lcg)
    name = f"{case['name']}/{key}"
    return arrays[name] if name in arrays else None


def write_case_ipq1(case, arrays, tmp_path) -> Path:
    p = tmp_path / f"{case['name']}.ipq1"
    p.write_bytes(arrays[f"{case['name']}/ipq1"].tobytes())
    return p


def assert_results_match(ids, dists, exp_ids, exp_dists, rel=1e-4, label=""):
    """Ids identical; distances within rel * max(1, |d|); infinities identical."""
    ids = np.asarray(ids)
    exp_ids = np.asarray(exp_ids)
    assert ids.shape == exp_ids.shape, label
    bad = np.argwhere(ids != exp_ids)
    assert bad.size == 0, f"{label}: {len(bad)} id mismatches, first at {bad[:5].tolist()}: " \
                          f"got {ids[tuple(bad[0])]} expected {exp_ids[tuple(bad[0])]}"
    d = np.asarray(dists, dtype=np.float64)
    e = np.asarray(exp_dists, dtype=np.float64)
    inf = np.isinf(e)
    assert np.array_equal(np.isinf(d), inf), label
    assert np.array_equal(np.signbit(d[inf]), np.signbit(e[inf])), label
    fin = ~inf
    tol = rel * np.maximum(1.0, np.abs(e[fin]))
    err = np.abs(d[fin] - e[fin])
    assert np.all(err <= tol), f"{label}: max distance error {err.max()}"
