// Shared helpers of the gfx950 kernels and the C ABI: error reporting, dtype codes, rounding primitives.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/weightferry.h"

namespace wf {

// thread-local last error (the ABI is called from several host threads: the copy issuer, the pin-ahead thread)
void set_error(const char* fmt, ...);

inline int hip_fail(hipError_t e, const char* what) {
    set_error("%s: %s", what, hipGetErrorString(e));
    return WF_EHIP;
}

#define WF_LAUNCH_CHECK(what)                                        \
    do {                                                             \
        hipError_t _e = hipGetLastError();                           \
        if (_e != hipSuccess) return ::wf::hip_fail(_e, what);       \
    } while (0)

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// ------------------------------------------------------------------------------------------- device primitives
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));

// little-endian f16 bits -> float (exact)
__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

// round to nearest even float16, kept as float32 (v_cvt_f16_f32, then back: exact)
__device__ __forceinline__ float round_f16(float x) { return (float)(_Float16)x; }

// round to nearest even bfloat16, kept as float32. For finite inputs this equals the reference's bit rule
// (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000 (enhancers/gguf_dequant.py:78-81): both are IEEE round to nearest
// even on the top 16 bits. v_cvt_pk_bf16_f32 on gfx950.
__device__ __forceinline__ float round_bf16(float x) {
    uint32_t b = __builtin_bit_cast(uint16_t, (__bf16)x);
    return __builtin_bit_cast(float, b << 16);
}

template <int D>
__device__ __forceinline__ float round_to(float x) {
    if constexpr (D == WF_F16) return round_f16(x);
    else if constexpr (D == WF_BF16) return round_bf16(x);
    else return x;
}

// two floats -> packed bf16 pair (low = a), one v_cvt_pk_bf16_f32
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
    bf2 r;
    r[0] = (__bf16)a;
    r[1] = (__bf16)b;
    return __builtin_bit_cast(uint32_t, r);
}

// two floats -> packed f16 pair (low = a)
__device__ __forceinline__ uint32_t pack_f16(float a, float b) {
    h2 r;
    r[0] = (_Float16)a;
    r[1] = (_Float16)b;
    return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ uint32_t h2_bits(h2 v) { return __builtin_bit_cast(uint32_t, v); }

// bytes [s, s+8) of the little-endian dword stream w0, w1, w2 where s is 0 or 2 (mod 4) bytes into w0
__device__ __forceinline__ uint2 funnel8(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t shift_bits) {
    uint2 r;
    r.x = __builtin_amdgcn_alignbit(w1, w0, shift_bits);
    r.y = __builtin_amdgcn_alignbit(w2, w1, shift_bits);
    return r;
}

}  // namespace wf
