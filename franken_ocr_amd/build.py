"""Build recipe for libfocr_hip.so (gfx950 only) — run in-tree.

    python -m franken_ocr_amd.build        # or __graft_entry__.build()

Every .hip/.cpp under csrc/ is compiled with hipcc for --offload-arch=gfx950
and linked into franken_ocr_amd/libfocr_hip.so. Flags that matter for parity:

* -ffp-contract=off   no a*b+c -> FMA contraction: every f32 op rounds on its
                      own, as the reference's Rust code does, so dequant,
                      int4 group sums and the MoE combine are bit-reproducible.
* -Xclang -target-feature -Xclang -packed-fp32-ops
                      keep the compiler from emitting packed-FP32 VALU ops.
* -mllvm -amdgpu-mfma-vgpr-form
                      MFMA results land in arch VGPRs: the int4 kernels'
                      per-group f32 epilogue reads every MFMA output, and from
                      AGPRs each read would cost an extra v_accvgpr_read.
No -ffast-math: fp32 division and sqrt stay correctly rounded (the
quantizer's amax/127 and 1/a_scale must match the CPU bit for bit).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "libfocr_hip.so"
BUILD = PKG / "_build"

ARCH = "gfx950"
COMMON = [
    "-std=c++17",
    "-O3",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-ffp-contract=off",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-mllvm",
    "-amdgpu-mfma-vgpr-form",
    "-Wall",
    "-Wno-unused-result",
    "-Wno-unused-value",
    "-Wno-unused-function",
]


def hipcc() -> str:
    cand = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(cand).exists():
        raise RuntimeError("hipcc not found: the gfx950 library cannot be built")
    return cand


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _compile(src: Path, build_dir: Path, extra: tuple) -> Path:
    obj = build_dir / (src.stem + ".o")
    cmd = [hipcc(), *COMMON, *extra, "-x", "hip", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = False, extra: tuple = (), out: Path = OUT, build_dir: Path = BUILD) -> Path:
    """Compile every kernel/host source for gfx950 and link the shared
    library. `extra` flags go on every compile and the link (a variant build
    into its own `build_dir` / `out`, e.g. the host-sanitized copy the CPU
    sanitizer test makes)."""
    build_dir.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = min(8, len(srcs), os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda src: _compile(src, build_dir, tuple(extra)), srcs))
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", *extra, "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out} from {len(srcs)} sources", file=sys.stderr)
    return out


if __name__ == "__main__":
    build(verbose=True)
