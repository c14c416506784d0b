"""The host code under AddressSanitizer + UndefinedBehaviorSanitizer (CPU only).

Runs the .focrq reader/writer tests — among them the 3000-blob differential
fuzz of the hand-written container parser against oracle/focrq_ref.py — the
ABI checks and the oracle tests in a child process against the host-sanitized
library and oracle, built here on demand (tests/sanitize.py); any sanitizer
report fails the child.
"""

from __future__ import annotations

import subprocess
import sys

from sanitize import DEFAULT_TESTS, ROOT, build_sanitized, sanitized_env


def test_host_code_clean_under_asan_and_ubsan():
    build_sanitized()
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", *DEFAULT_TESTS], cwd=ROOT,
                       env=sanitized_env(), capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, (r.stdout[-3000:], r.stderr[-3000:])
    assert "passed" in r.stdout and "AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr
