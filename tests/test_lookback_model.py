"""The decoupled look-back of the single-pass compactions (dynamis_amd/csrc/dg_lookback.hpp),
run by a host-threaded model (tests/lookback_model.cpp, built here with g++ under
ThreadSanitizer): many threads take ticket-ordered tiles with random delays and publish
through relaxed atomics, exactly as the device workgroups do.  Every tile's exclusive
offset must equal the serial scan; with one tile that never publishes, the tiles before it
stay exact, the one behind it gives up after its bounded wait, and every thread ends
(the device kernel raises its error flag then).  Also unit cases of one window step."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("lb") / "lookback_model")
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-pthread", "-fsanitize=thread",
           os.path.join(HERE, "lookback_model.cpp"), "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:  # no TSan runtime: plain build
        cmd = [c for c in cmd if c != "-fsanitize=thread"]
        r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


@pytest.mark.parametrize("threads,tiles,seed", [(2, 3000, 1), (8, 20000, 2), (32, 20000, 3), (64, 5000, 4)])
def test_offsets_equal_serial_scan(model, threads, tiles, seed):
    r = subprocess.run([model, str(threads), str(tiles), str(seed), "0"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout + r.stderr


def test_silent_tile_bounded_wait(model):
    r = subprocess.run([model, "8", "4000", "5", "1"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout + r.stderr


def test_window_step_cases(tmp_path):
    src = tmp_path / "w.cpp"
    src.write_text(r'''
#include <cstdio>
#include "%s"
using namespace dg::lookback;
int main() {
  int64_t s = 0; bool d = false;
  uint64_t a[3] = {word(kAggregate, 5), word(kInclusive, 100), 0};      // agg, inclusive
  if (window_step(a, 3, &s, &d) != 2 || s != 105 || !d) return 1;
  s = 0; uint64_t b[2] = {word(kAggregate, 5), 0};                          // partial
  if (window_step(b, 2, &s, &d) != 1 || s != 5 || d) return 2;
  s = 0; uint64_t c[2] = {word(kAggregate, 5), word(kAggregate, 6)};        // no inclusive
  if (window_step(c, 2, &s, &d) != 2 || s != 11 || d) return 3;
  s = 0; uint64_t e[2] = {word(kInclusive, 7), 0};                          // stops at once
  if (window_step(e, 2, &s, &d) != 1 || s != 7 || !d) return 4;
  s = 0; uint64_t f[2] = {0, word(kInclusive, 7)};                          // nothing ready
  if (window_step(f, 2, &s, &d) != 0 || s != 0 || d) return 6;
  if (value_of(word(kInclusive, (1ll << 61) + 3)) != (1ll << 61) + 3) return 5;
  printf("ok\n"); return 0;
}''' % os.path.join(os.path.dirname(HERE), "dynamis_amd", "csrc", "dg_lookback.hpp"))
    exe = str(tmp_path / "w")
    subprocess.run(["g++", "-std=c++17", str(src), "-o", exe], check=True)
    r = subprocess.run([exe], capture_output=True, text=True)
    assert r.returncode == 0, r.returncode
