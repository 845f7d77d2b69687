"""The host code under AddressSanitizer and UndefinedBehaviorSanitizer (CPU):
the oracle (oracle/oracle.c) and the GGUF reader (bus-fill_amd/csrc/bf_gguf.cpp)
built with -fsanitize=address,undefined around tests/sanitize_main.cpp, then
run over the oracle's entry points and over GGUF files: a valid one, every
truncation of it, and random corruptions of its header.  Any sanitizer report
fails the test (halt on the first error)."""
import os
import random
import shutil
import subprocess

import pytest

from test_gguf import SAMPLE_KV, sample_tensors, write_gguf

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def sanitized(tmp_path_factory):
    gcc, gxx = shutil.which("gcc"), shutil.which("g++")
    if gcc is None or gxx is None:
        pytest.skip("gcc/g++ not available")
    d = tmp_path_factory.mktemp("sanitize")
    san = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]
    obj = str(d / "oracle.o")
    subprocess.run([gcc, *san, "-std=gnu11", "-fopenmp", "-ffp-contract=off", "-c",
                    os.path.join(ROOT, "oracle", "oracle.c"), "-o", obj], check=True)
    exe = str(d / "sanitize_main")
    subprocess.run([gxx, *san, "-std=c++17", "-fopenmp", "-I", os.path.join(ROOT, "include"),
                    "-I", os.path.join(ROOT, "bus-fill_amd", "csrc"), "-I", os.path.join(ROOT, "oracle"),
                    os.path.join(ROOT, "tests", "sanitize_main.cpp"),
                    os.path.join(ROOT, "bus-fill_amd", "csrc", "bf_gguf.cpp"), obj, "-o", exe], check=True)
    return exe


def run(exe, files):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1", UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1",
               OMP_NUM_THREADS="2")
    env.pop("LD_PRELOAD", None)
    r = subprocess.run([exe, *map(str, files)], capture_output=True, text=True, timeout=600, env=env)
    out = r.stdout + r.stderr
    assert r.returncode == 0 and "runtime error" not in out and "Sanitizer" not in out, out[-4000:]
    return r.stdout


def test_oracle_and_gguf_reader_under_sanitizers(sanitized, tmp_path):
    path = tmp_path / "sample.gguf"
    write_gguf(path, SAMPLE_KV, sample_tensors(), alignment=64)
    blob = path.read_bytes()
    files = [path]
    for cut in range(0, len(blob), max(1, len(blob) // 300)):
        p = tmp_path / f"trunc{cut}.gguf"
        p.write_bytes(blob[:cut])
        files.append(p)
    rng = random.Random(5)
    for i in range(200):
        b = bytearray(blob)
        for _ in range(rng.randint(1, 6)):
            b[rng.randrange(0, min(len(b), 700))] = rng.randrange(256)
        p = tmp_path / f"corrupt{i}.gguf"
        p.write_bytes(bytes(b))
        files.append(p)
    out = run(sanitized, files)
    assert "sanitized run ok" in out and f"{len(files)} files" in out, out
