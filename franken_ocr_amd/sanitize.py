"""Run the CPU-only checks of the host code under AddressSanitizer and
UndefinedBehaviorSanitizer (host code only; no GPU involved).

    python -m franken_ocr_amd.sanitize [pytest args...]

Builds the host-sanitized library (franken_ocr_amd/_build_san/, the gfx950
code unchanged) and the sanitized oracle (oracle/_san/), then runs pytest in
a child process that preloads clang's ASan runtime (the Python interpreter
itself is not instrumented) with both libraries selected through
FOCR_HIP_LIB / FOCR_ORACLE_LIB. Default selection: the .focrq reader/writer
tests (including the 3000-blob differential fuzz of the hand-written
container parser against oracle/focrq_ref.py), the ABI's load/export checks
and the oracle tests. Any sanitizer report aborts the child with a nonzero
status.
"""

from __future__ import annotations

import glob
import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
DEFAULT_TESTS = ["tests/test_focrq.py", "tests/test_abi.py", "tests/test_oracle.py", "-m", "not gpu"]


def asan_runtime() -> str:
    hits = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not hits:
        raise RuntimeError("clang's ASan runtime (libclang_rt.asan-x86_64.so) not found under /opt/rocm/llvm")
    return hits[-1]


def main(argv: list[str]) -> int:
    from franken_ocr_amd import build as B

    lib = B.build(verbose=True, sanitize=True)
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "san"], check=True)
    env = dict(os.environ)
    env.update({
        "LD_PRELOAD": asan_runtime(),
        # leaks of the uninstrumented interpreter are not ours; stop at the first report
        "ASAN_OPTIONS": "detect_leaks=0:abort_on_error=1:halt_on_error=1:allocator_may_return_null=1",
        "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1",
        "FOCR_HIP_LIB": str(lib),
        "FOCR_ORACLE_LIB": str(ROOT / "oracle" / "_san" / "liboracle_san.so"),
    })
    cmd = [sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", *(argv or DEFAULT_TESTS)]
    print("+", " ".join(cmd), file=sys.stderr, flush=True)
    return subprocess.run(cmd, cwd=ROOT, env=env).returncode


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
