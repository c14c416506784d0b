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


# Host-side sanitizers for the CPU-only checks of the host code (the .focrq
# parser, the ABI's argument checks): every -fsanitize= applies to the host
# pass only, the gfx950 code is built as usual. The result loads into a
# process that preloads the clang ASan runtime (franken_ocr_amd/sanitize.py).
SANITIZE = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer",
            "-Xarch_host", "-shared-libsan"]
SAN_BUILD = PKG / "_build_san"
SAN_OUT = SAN_BUILD / "libfocr_hip_san.so"


def _compile(src: Path, sanitize: bool = False) -> Path:
    obj = (SAN_BUILD if sanitize else BUILD) / (src.stem + ".o")
    cmd = [hipcc(), *COMMON, *(SANITIZE if sanitize else []), "-x", "hip", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = False, sanitize: bool = False) -> Path:
    """Compile every kernel/host source for gfx950 and link the shared library
    (with sanitize: the host-sanitized copy in _build_san/ instead)."""
    out_dir = SAN_BUILD if sanitize else BUILD
    out_dir.mkdir(exist_ok=True)
    out = SAN_OUT if sanitize else OUT
    srcs = sources()
    jobs = min(8, len(srcs), os.cpu_count() or 1)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda src: _compile(src, sanitize), srcs))
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", *(SANITIZE if sanitize else []), "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out} from {len(srcs)} sources", file=sys.stderr)
    return out


if __name__ == "__main__":
    build(verbose=True)
