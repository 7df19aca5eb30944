"""The CPU oracle under AddressSanitizer and UndefinedBehaviorSanitizer: oracle/graph_oracle.c
and the driver tests/oracle_sanitize_main.c are compiled together with
-fsanitize=address,undefined (no recovery) and run; the driver exercises every oracle
entry point on edge cases and checks invariants the definition fixes (see its header).
Host code only; skipped where gcc cannot link the sanitizer runtimes."""
import os
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def test_oracle_under_asan_ubsan():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "oracle_sanitize")
        cmd = ["gcc", "-std=c11", "-O1", "-g", "-fno-omit-frame-pointer", "-ffp-contract=off",
               "-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fopenmp",
               os.path.join(ROOT, "oracle", "graph_oracle.c"), os.path.join(HERE, "oracle_sanitize_main.c"),
               "-o", exe, "-lm"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            if "asan" in r.stderr or "ubsan" in r.stderr:
                pytest.skip("sanitizer runtimes not available: " + r.stderr[-300:])
            raise AssertionError(r.stderr)
        env = dict(os.environ, OMP_NUM_THREADS="2", ASAN_OPTIONS="detect_leaks=1",
                   UBSAN_OPTIONS="print_stacktrace=1")
        r = subprocess.run([exe], capture_output=True, text=True, env=env, timeout=300)
        assert r.returncode == 0, r.stdout + r.stderr
        assert "all cases passed" in r.stdout
