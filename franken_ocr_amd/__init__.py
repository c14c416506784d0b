"""franken_ocr_amd — MI355X (gfx950) tier for franken_ocr's quantized decoder
hot path: the int8/int4 igemm tier, the 129280x1280 LM head + argmax, the
64-expert top-6 MoE decode layer and the R-SWA ring-buffer decode attention.

The compute lives in libfocr_hip.so (hand-written HIP for gfx950 behind the C
ABI in include/focr_hip.h). This package binds it with ctypes:

* ``franken_ocr_amd.simd``   — the reference's ``simd`` tier surface
  (igemm_s8s8 / igemm_u8s8 / int4 / caps / selftest) on the GPU,
* ``franken_ocr_amd.engine`` — device-resident engine ops (QInt8 upload,
  gemv_i8, lm_head_i8, MoeLayer, RingCache),
* ``franken_ocr_amd.device`` — contexts and device arrays,
* ``franken_ocr_amd.synth``  — seeded synthetic inputs for the configs.

There is no CPU fallback: without the built library every op raises
``ExtensionMissing``.
"""

from ._abi import (  # noqa: F401
    ContractViolation,
    ExtensionMissing,
    FocrHipError,
    NoDevice,
    RouteError,
    StateError,
)

__version__ = "0.1.0"


def library_path() -> str:
    from . import _abi

    return str(_abi.LIB_PATH)
