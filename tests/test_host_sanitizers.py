"""CPU: the library's host-only code under AddressSanitizer and
UndefinedBehaviorSanitizer.

tests/sanitize/host_checks.cpp is built with g++ -fsanitize=address,undefined
together with the host clustering engines (xspmm_amd/csrc/cluster.cpp), the
MatrixMarket reader (xspmm_amd/csrc/mtx.cpp) and the C oracle
(oracle/oracle.c); no GPU code is involved.  It compares the host clustering
(scan and index engines and the automatic choice, 1 and 4 threads, int32 and
int64) with the oracle's restatement of the reference greedy on 90 random
matrices (empty rows, unsorted and duplicated columns, thresholds 0 to 1,
block widths 1, 16, 64), runs the oracle's conversion, permutation and
products, and reads every MatrixMarket fixture plus malformed files.  Any
sanitizer report or mismatch fails the test.
"""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "xspmm_amd", "csrc")
SAN = "-fsanitize=address,undefined"


def _have(tool):
    return shutil.which(tool) is not None


@pytest.fixture(scope="module")
def host_checks(tmp_path_factory):
    if not (_have("g++") and _have("gcc")):
        pytest.skip("g++/gcc not available")
    if not os.path.isdir("/opt/rocm/include"):
        pytest.skip("HIP headers (/opt/rocm/include) not available")
    out = tmp_path_factory.mktemp("sanitize")
    oracle_o = str(out / "oracle.o")
    exe = str(out / "host_checks")
    cmds = [
        ["gcc", "-std=c11", "-O1", "-g", SAN, "-fno-sanitize-recover=undefined", "-fopenmp",
         "-c", os.path.join(ROOT, "oracle", "oracle.c"), "-o", oracle_o],
        ["g++", "-std=c++20", "-O1", "-g", SAN, "-fno-sanitize-recover=undefined", "-mpopcnt",
         "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", "-I" + os.path.join(ROOT, "include"),
         "-I" + CSRC, "-I" + os.path.join(ROOT, "oracle"),
         os.path.join(ROOT, "tests", "sanitize", "host_checks.cpp"),
         os.path.join(CSRC, "cluster.cpp"), os.path.join(CSRC, "mtx.cpp"), oracle_o,
         "-fopenmp", "-lpthread", "-o", exe],
    ]
    for c in cmds:
        r = subprocess.run(c, capture_output=True, text=True)
        assert r.returncode == 0, f"build failed: {' '.join(c)}\n{r.stderr[-4000:]}"
    return exe


def _malformed(tmp_path):
    files = {
        "empty.mtx": "",
        "header_only.mtx": "%%MatrixMarket matrix coordinate real general\n",
        "negative_dims.mtx": "%%MatrixMarket matrix coordinate real general\n-3 4 1\n1 1 1.0\n",
        "huge_dims.mtx": "%%MatrixMarket matrix coordinate real general\n99999999999 5 1\n1 1 2.0\n",
        "truncated.mtx": "%%MatrixMarket matrix coordinate real general\n4 4 3\n1 1 1.0\n2 2\n",
        "out_of_range.mtx": "%%MatrixMarket matrix coordinate real general\n3 3 4\n0 1 1.0\n4 1 2.0\n"
                            "1 9 3.0\n2 2 4.0\n",
        "garbage.mtx": "\x00\xff not a matrix \n 1 2 3 4 5 6 7 8 9\n",
        "long_line.mtx": "%%MatrixMarket matrix coordinate real general\n2 2 1\n1 1 " + "9" * 5000 + "\n",
    }
    paths = []
    for name, text in files.items():
        p = tmp_path / name
        p.write_bytes(text.encode("latin-1"))
        paths.append(str(p))
    paths.append(str(tmp_path / "missing.mtx"))
    return paths


def test_host_code_under_sanitizers(host_checks, tmp_path):
    golden = os.path.join(ROOT, "tests", "golden", "mtx")
    files = sorted(os.path.join(golden, f) for f in os.listdir(golden) if f.endswith(".mtx"))
    files += _malformed(tmp_path)
    env = dict(os.environ)
    env["ASAN_OPTIONS"] = "detect_leaks=1:verify_asan_link_order=0"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    env.pop("XSPMM_CLUSTER_ENGINE", None)
    r = subprocess.run([host_checks] + files, capture_output=True, text=True, env=env, timeout=600)
    tail = (r.stdout[-3000:] + "\n" + r.stderr[-6000:])
    assert r.returncode == 0, tail
    assert "host checks ok" in r.stdout, tail
    assert "runtime error" not in r.stderr, tail
    assert "ERROR: AddressSanitizer" not in r.stderr, tail
    lines = r.stdout.splitlines()
    # unreadable files raise; an empty file reads as an empty matrix (as the
    # comments-only fixture does), negative dimensions as a matrix without rows
    for name in ("missing.mtx", "garbage.mtx", "huge_dims.mtx"):
        assert all("error:" in l for l in lines if f"/{name} (" in l), name
    assert all("0 entries" in l for l in lines if "/negative_dims.mtx (" in l)
    # entries outside the matrix are dropped (one of the four is inside)
    assert all("3 x 3, 1 entries" in l for l in lines if "/out_of_range.mtx (" in l)
