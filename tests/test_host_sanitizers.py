"""Host-side sanitizer runs (CPU only; no device code is instrumented).

1. The device-buffer registry and pool (rpl_amd/csrc/host/rpl_runtime.c)
   under ThreadSanitizer and under AddressSanitizer + UBSan: eight threads
   create, upload, read, attach gradients to, fill, download and free
   tensors concurrently (tests/host/registry_stress.c, with host stand-ins
   for the rplhip_* device calls).
2. The rest of the CPU test suite against the sanitizer builds of the host
   layer (`make -C rpl_amd san` -> librpl_san.so) and of the oracle
   (`make -C oracle san` -> liboracle_san.so), with libasan preloaded into
   the Python process: ABI checks, error paths without a device, the seeded
   generator and every oracle pin run instrumented.  UBSan is built with
   -fno-sanitize-recover, so any report fails the run.
"""
import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
HOST = os.path.join(REPO, "rpl_amd", "csrc", "host")


def _gcc_lib(name):
    return subprocess.check_output(["gcc", f"-print-file-name={name}"], text=True).strip()


@pytest.mark.parametrize("sanitizer", ["thread", "address,undefined"])
def test_registry_stress(tmp_path, sanitizer):
    exe = tmp_path / "registry_stress"
    subprocess.check_call(["gcc", "-O1", "-g", "-std=gnu11", f"-fsanitize={sanitizer}", "-fno-sanitize-recover=all",
                           "-fno-omit-frame-pointer", "-I", os.path.join(REPO, "include"), "-I", HOST,
                           os.path.join(HOST, "rpl_runtime.c"), os.path.join(HERE, "host", "registry_stress.c"),
                           "-o", str(exe), "-lpthread", "-lm"])
    env = dict(os.environ, TSAN_OPTIONS="halt_on_error=1", ASAN_OPTIONS="detect_leaks=1")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "Sanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr
    assert "OK" in r.stdout


def test_cpu_suite_under_asan_ubsan():
    subprocess.check_call(["make", "-s", "-C", os.path.join(REPO, "rpl_amd"), "san"])
    subprocess.check_call(["make", "-s", "-C", os.path.join(REPO, "oracle"), "san"])
    env = dict(os.environ,
               LD_PRELOAD=f"{_gcc_lib('libasan.so')}:{_gcc_lib('libubsan.so')}",
               ASAN_OPTIONS="detect_leaks=0",  # the interpreter's own allocations
               RPL_LIB=os.path.join(REPO, "rpl_amd", "librpl_san.so"),
               RPL_ORACLE_LIB=os.path.join(REPO, "oracle", "liboracle_san.so"))
    r = subprocess.run([sys.executable, "-m", "pytest", HERE, "-q", "-x", "-s", "-m", "not gpu", "-p",
                        "no:cacheprovider", "--ignore", os.path.abspath(__file__)],
                       capture_output=True, text=True, timeout=900, env=env, cwd=REPO)
    out = r.stdout + r.stderr
    for built in (os.path.join(REPO, "rpl_amd", "librpl_san.so"), os.path.join(REPO, "oracle", "liboracle_san.so")):
        os.remove(built)  # test-only builds: keep them out of the tree that travels to the GPU box
    assert r.returncode == 0, out[-4000:]
    assert "runtime error" not in out and "AddressSanitizer" not in out, out[-4000:]
    assert " passed" in r.stdout
