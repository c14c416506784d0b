// k_int4.hpp — in-register int4 nibble unpack shared by the int4 kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace focr {

// Sign-extend the nibble held in the low 4 bits of each byte (int4.rs:97-101):
// OR 0xF0 into the bytes whose bit 3 is set. (x >> 3) & 0x01010101 leaves a
// 0/1 per byte, and multiplying by 0xF0 cannot carry across bytes.
__device__ __forceinline__ uint32_t sext_nibbles(uint32_t x) {
    return x | (((x >> 3) & 0x01010101u) * 0xF0u);
}

// Four packed bytes b0..b3 -> eight int8 weights in k order (int4.rs:110-112,
// low nibble = even k): wlo = [lo(b0) hi(b0) lo(b1) hi(b1)],
// whi = [lo(b2) hi(b2) lo(b3) hi(b3)] (byte 0 = lowest address).
__device__ __forceinline__ void unpack8_i4(uint32_t packed, uint32_t& wlo, uint32_t& whi) {
    const uint32_t lo = packed & 0x0F0F0F0Fu;
    const uint32_t hi = (packed >> 4) & 0x0F0F0F0Fu;
    // v_perm_b32: selector bytes 0-3 pick bytes of the second operand (lo),
    // 4-7 bytes of the first (hi).
    wlo = sext_nibbles(__builtin_amdgcn_perm(hi, lo, 0x05010400u));
    whi = sext_nibbles(__builtin_amdgcn_perm(hi, lo, 0x07030602u));
}

}  // namespace focr
