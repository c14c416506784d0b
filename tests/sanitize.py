"""Run the CPU-only checks of the host code under AddressSanitizer and
UndefinedBehaviorSanitizer (host code only; no GPU involved). Test tooling:
nothing in the product package imports it.

    python tests/sanitize.py [pytest args...]

Builds the host-sanitized library (tests/_san/, the gfx950 code unchanged:
every -fsanitize= applies to the host pass only) and the sanitized oracle
(oracle/_san/), then runs pytest in a child process that preloads clang's
ASan runtime (the Python interpreter itself is not instrumented) with both
libraries selected through FOCR_HIP_LIB / FOCR_ORACLE_LIB. Default
selection: the .focrq reader/writer tests (including the 3000-blob
differential fuzz of the hand-written container parser against
oracle/focrq_ref.py), the ABI's load/export checks and the oracle tests. Any
sanitizer report aborts the child with a nonzero status.
"""

from __future__ import annotations

import glob
import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
DEFAULT_TESTS = ["tests/test_focrq.py", "tests/test_abi.py", "tests/test_oracle.py", "-m", "not gpu"]

# host-pass-only sanitizer flags for hipcc (each -fsanitize= right after -Xarch_host)
SANITIZE = ("-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer",
            "-Xarch_host", "-shared-libsan")
SAN_DIR = ROOT / "tests" / "_san"
SAN_LIB = SAN_DIR / "libfocr_hip_san.so"
SAN_ORACLE = ROOT / "oracle" / "_san" / "liboracle_san.so"


def asan_runtime() -> str:
    hits = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not hits:
        raise RuntimeError("clang's ASan runtime (libclang_rt.asan-x86_64.so) not found under /opt/rocm/llvm")
    return hits[-1]


def build_sanitized(force: bool = False) -> Path:
    """The host-sanitized library (rebuilt when older than any source) and
    the sanitized oracle."""
    from franken_ocr_amd import build as B

    newest = max(p.stat().st_mtime for p in B.sources() + list(B.CSRC.glob("*.hpp")))
    if force or not SAN_LIB.exists() or SAN_LIB.stat().st_mtime < newest:
        B.build(extra=SANITIZE, out=SAN_LIB, build_dir=SAN_DIR / "obj")
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "san"], check=True)
    return SAN_LIB


def sanitized_env() -> dict:
    env = dict(os.environ)
    env.update({
        "LD_PRELOAD": asan_runtime(),
        # leaks of the uninstrumented interpreter are not ours; stop at the first report
        "ASAN_OPTIONS": "detect_leaks=0:abort_on_error=1:halt_on_error=1:allocator_may_return_null=1",
        "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1",
        "FOCR_HIP_LIB": str(SAN_LIB),
        "FOCR_ORACLE_LIB": str(SAN_ORACLE),
        "PYTHONPATH": str(ROOT),
    })
    return env


def main(argv: list[str]) -> int:
    build_sanitized()
    cmd = [sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", *(argv or DEFAULT_TESTS)]
    print("+", " ".join(cmd), file=sys.stderr, flush=True)
    return subprocess.run(cmd, cwd=ROOT, env=sanitized_env()).returncode


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
