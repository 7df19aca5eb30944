"""Every hipcc command that a test builds keeps sanitizers off the device pass.

GPU AddressSanitizer builds cannot run on the target pool, so a hipcc line that asks for a
sanitizer must either scope each sanitizer flag to the host pass (the flag directly after
-Xarch_host) or carry -fno-gpu-sanitize on a line with no -Xarch_ option.  This scans the
source lines of tests/ and of the package that mention both hipcc (or HIPCC) and a
sanitizer flag.  CPU only."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SAN = re.compile(r"-fsanitize=")


def _files():
    for d in ("tests", "dynamis_amd", "oracle"):
        for dirpath, _, names in os.walk(os.path.join(ROOT, d)):
            for n in names:
                if n.endswith((".py", ".sh", ".mk")) or n == "Makefile":
                    yield os.path.join(dirpath, n)


def _bad_line(line):
    toks = re.findall(r"[\"']?(-[A-Za-z_][^\"'\s,]*)", line)
    if not any(SAN.match(t) for t in toks):
        return False
    if "-fno-gpu-sanitize" in toks and not any(t.startswith("-Xarch_") for t in toks):
        return False
    for i, t in enumerate(toks):
        if SAN.match(t) and (i == 0 or toks[i - 1] != "-Xarch_host"):
            return True
    return False


def test_no_device_sanitizer_in_hipcc_commands():
    bad = []
    for path in _files():
        if os.path.abspath(path) == os.path.abspath(__file__):
            continue
        with open(path, errors="replace") as f:
            text = f.read()
        if "hipcc" not in text.lower():
            continue
        for no, line in enumerate(text.splitlines(), 1):
            if _bad_line(line):
                bad.append(f"{os.path.relpath(path, ROOT)}:{no}: {line.strip()}")
    assert not bad, "sanitizer flags that reach the device pass:\n" + "\n".join(bad)


def test_checker_flags_the_bare_form():
    assert _bad_line('cmd = [HIPCC, "-fsanitize=address", main_o]')
    assert not _bad_line('cmd = [HIPCC, "-Xarch_host", "-fsanitize=address"]')
    assert not _bad_line('cmd = [HIPCC, "-fsanitize=address", "-fno-gpu-sanitize", main_o]')
