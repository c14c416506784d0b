"""The host code under AddressSanitizer + UndefinedBehaviorSanitizer (CPU only).

Runs the .focrq reader/writer tests — among them the 3000-blob differential
fuzz of the hand-written container parser against oracle/focrq_ref.py — the
ABI checks and the oracle tests in a child process against the host-sanitized
library and oracle (built by __graft_entry__.build(), see
franken_ocr_amd/sanitize.py); any sanitizer report fails the child.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def test_host_code_clean_under_asan_and_ubsan():
    from franken_ocr_amd import build as B
    from franken_ocr_amd import sanitize as S

    oracle_san = ROOT / "oracle" / "_san" / "liboracle_san.so"
    if not B.SAN_OUT.exists() or not oracle_san.exists():
        pytest.skip("sanitized builds absent (run __graft_entry__.build())")
    # a library older than its sources would test stale host code (and miss
    # entry points the ABI binds): rebuild it first
    newest = max(p.stat().st_mtime for p in B.sources() + list(B.CSRC.glob("*.hpp")))
    if B.SAN_OUT.stat().st_mtime < newest:
        B.build(sanitize=True)
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "san"], check=True)
    env = dict(os.environ)
    env.update({
        "LD_PRELOAD": S.asan_runtime(),
        "ASAN_OPTIONS": "detect_leaks=0:abort_on_error=1:halt_on_error=1:allocator_may_return_null=1",
        "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1",
        "FOCR_HIP_LIB": str(B.SAN_OUT),
        "FOCR_ORACLE_LIB": str(oracle_san),
        "PYTHONPATH": str(ROOT),
    })
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", *S.DEFAULT_TESTS], cwd=ROOT,
                       env=env, capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, (r.stdout[-3000:], r.stderr[-3000:])
    assert "passed" in r.stdout and "AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr
