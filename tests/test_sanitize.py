"""The CPW1 v4 parser, geometry check and writer (cpw4.c) under a host sanitizer build:
gcc -fsanitize=address,undefined of cpw4.c and a small driver (tests/v4_check_main.c), run on
the synthetic model file, on every malformed and geometry-mismatched variant of
tests/test_v4.py, and on a file the streaming writer produces. Any out-of-bounds access,
use-after-free, leak or undefined behaviour aborts the driver (no recovery), so the test
asserts a clean exit together with the expected codes (0 / -3)."""
import os
import shutil
import subprocess

import pytest

import cachepotato_amd as C
from cachepotato_amd import qwen3 as Q
from tests.conftest import ROOT
from tests.test_v4 import SMALL, GEOMETRY_CASES, _tables

pytestmark = pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not available")


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    d = tmp_path_factory.mktemp("asan")
    exe = d / "v4_check"
    cmd = ["gcc", "-std=c11", "-g", "-O1", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", "-fno-omit-frame-pointer",
           "-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(ROOT, "cachepotato_amd", "csrc"),
           os.path.join(ROOT, "tests", "v4_check_main.c"),
           os.path.join(ROOT, "cachepotato_amd", "csrc", "engine", "cpw4.c"), "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        pytest.skip("sanitizer build unavailable: " + r.stderr[-500:])
    return exe


def run(driver, *args):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([str(driver), *map(str, args)], capture_output=True, text=True, env=env,
                       timeout=120)
    assert r.returncode == 0, r.stderr[-3000:]
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr
    return [int(line.split()[0]) for line in r.stdout.strip().splitlines()]


def test_parser_on_good_and_malformed_files(driver, tmp_path):
    good = tmp_path / "small.v4"
    Q.write_synthetic(Q.bind(C.lib()), good, **SMALL)
    b, hdr, _, _ = _tables(good)
    files, want = [good], [0]
    for name, edit in sorted(GEOMETRY_CASES.items()):
        bb = bytearray(b)
        edit(bb, hdr)
        p = tmp_path / f"geometry_{name}.v4"
        p.write_bytes(bytes(bb))
        files.append(p)
        want.append(-3)
    for name, cut in (("truncated_header", 40), ("truncated_tables", hdr["off_d"] - 8),
                      ("truncated_payload", len(b) - 100)):
        p = tmp_path / f"{name}.v4"
        p.write_bytes(b[:cut])
        files.append(p)
        want.append(-3)
    bb = bytearray(b)
    bb[0] ^= 1
    p = tmp_path / "magic.v4"
    p.write_bytes(bytes(bb))
    files.append(p)
    want.append(-3)
    assert run(driver, *files) == want


def test_writer_output_parses(driver, tmp_path):
    p = tmp_path / "written.v4"
    assert run(driver, "--write", p) == [0]
