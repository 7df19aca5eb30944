"""The library's host code (descriptor validation, the build plan, workspace layouts) under
AddressSanitizer and UndefinedBehaviorSanitizer: every source of dynamis_amd/csrc is
compiled with the sanitizers on its host side only (-Xarch_host; the device code is
built as usual but never launched) and linked with tests/host_sanitize_main.cpp, which
calls the host entry points on 20000 random and extreme descriptors (see its header).
Runs without a GPU; skipped where hipcc is absent."""
import os
import shutil
import subprocess
import sys
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path.insert(0, ROOT)


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc not available")
def test_host_code_under_asan_ubsan():
    from dynamis_amd import build as b

    with tempfile.TemporaryDirectory() as d:
        # every sanitizer flag is scoped to the host pass with -Xarch_host
        flags = [f for f in b.FLAGS if f not in ("-O3",)] + ["-O1", "-g", "-fno-omit-frame-pointer",
                                                          "-Xarch_host", "-fsanitize=address,undefined",
                                                          "-Xarch_host", "-fno-sanitize-recover=all"]
        objs = []
        for src in b.SOURCES:
            obj = os.path.join(d, src + ".o")
            # (the per-source scheduler flags are left out: device code is not run here)
            cmd = [b.HIPCC, *flags, "-c", os.path.join(b.CSRC, src), "-o", obj]
            r = subprocess.run(cmd, capture_output=True, text=True)
            assert r.returncode == 0, r.stdout + r.stderr
            objs.append(obj)
        main_o = os.path.join(d, "host_sanitize_main.o")
        cmd = [b.HIPCC, *flags, "-c", os.path.join(HERE, "host_sanitize_main.cpp"), "-o", main_o]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stdout + r.stderr
        exe = os.path.join(d, "host_sanitize")
        cmd = [b.HIPCC, f"--offload-arch={b.ARCH}", "-fsanitize=address,undefined", "-fno-gpu-sanitize",
               main_o, *objs, "-o", exe]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stdout + r.stderr
        env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0", UBSAN_OPTIONS="print_stacktrace=1")
        r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=300)
        assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
        assert "all checks passed" in r.stdout
        print(r.stdout)
