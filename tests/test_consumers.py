"""ABI consumers: a C program and a C++ program compiled against include/ovvs
and linked to libovvs.so, as the reference's own tests/consumer.c and
tests/consumer.cpp consume libovvs."""

from __future__ import annotations

import os
import subprocess

import pytest

from conftest import GOLDEN, ROOT

INC = ROOT / "include"
CONSUMERS = ROOT / "tests" / "consumer"


def _lib_dir(ovvs):
    return str(ovvs.library_path().parent)


def _build(compiler, src, out, ovvs, std):
    cmd = [compiler, std, "-Wall", "-Werror", f"-I{INC}", str(src), "-o", str(out),
           f"-L{_lib_dir(ovvs)}", "-lovvs", f"-Wl,-rpath,{_lib_dir(ovvs)}"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)


def test_c_consumer(ovvs, tmp_path):
    exe = tmp_path / "consumer"
    _build("gcc", CONSUMERS / "consumer.c", exe, ovvs, "-std=c11")
    out = tmp_path / "again.ipq1"
    r = subprocess.run([str(exe), str(GOLDEN / "legacy_ipq1_v1.bin"), str(out)],
                       capture_output=True, text=True)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    assert out.read_bytes() == (GOLDEN / "legacy_ipq1_v1.bin").read_bytes()


def test_cpp_consumer(ovvs, tmp_path):
    exe = tmp_path / "consumer_cpp"
    _build("g++", CONSUMERS / "consumer.cpp", exe, ovvs, "-std=c++17")
    r = subprocess.run([str(exe), str(GOLDEN / "legacy_ipq1_v1.bin")], capture_output=True,
                       text=True)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)


@pytest.mark.gpu
def test_cpp_consumer_searches_on_gpu(ovvs, tmp_path):
    exe = tmp_path / "consumer_cpp"
    _build("g++", CONSUMERS / "consumer.cpp", exe, ovvs, "-std=c++17")
    r = subprocess.run([str(exe), str(GOLDEN / "legacy_ipq1_v1.bin"), "search"],
                       capture_output=True, text=True, env=dict(os.environ))
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
