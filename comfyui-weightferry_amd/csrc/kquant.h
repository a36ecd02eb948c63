// Device helpers shared by the dequantisation kernels and the fused dequant + GEMM kernel: quants to float16
// through the exponent trick, broadcasts of packed halves, and the K-quant 6-bit scale / min unpacking.
#pragma once

#include "wf_common.h"

namespace wf {

// bytes b0..b3 of w -> float16 pairs (1024 + b0, 1024 + b1), (1024 + b2, 1024 + b3)
__device__ __forceinline__ h2 biased_lo(uint32_t w) { return as_h2(__builtin_amdgcn_perm(0x64646464u, w, 0x04010400u)); }
__device__ __forceinline__ h2 biased_hi(uint32_t w) { return as_h2(__builtin_amdgcn_perm(0x64646464u, w, 0x04030402u)); }

__device__ __forceinline__ h2 h2s(float a) { h2 r; r[0] = (_Float16)a; r[1] = (_Float16)a; return r; }
__device__ __forceinline__ h2 lo2(h2 v) { h2 r; r[0] = v[0]; r[1] = v[0]; return r; }
__device__ __forceinline__ h2 hi2(h2 v) { h2 r; r[0] = v[1]; r[1] = v[1]; return r; }

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xffu; }

// get_scale_min of sub-block sub (0..7) from the scale bytes s0 = s[0..3], s1 = s[4..7], s2 = s[8..11]
// (enhancers/gguf_dequant.py:170-185)
__device__ __forceinline__ void scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int sub, uint32_t& sc,
                                          uint32_t& m) {
    const int j = sub & 3;
    const uint32_t a = byte_of(s0, j), b = byte_of(s1, j), c = byte_of(s2, j);
    if (sub < 4) {
        sc = a & 63u;
        m = b & 63u;
    } else {
        sc = (c & 0xfu) | ((a >> 2) & 0x30u);
        m = (c >> 4) | ((b >> 2) & 0x30u);
    }
}

// the same without a branch on sub (for a sub-block index that is uniform but unknown at compile time: a branch
// there would split the caller's straight-line code)
__device__ __forceinline__ void scale_min_nb(uint32_t s0, uint32_t s1, uint32_t s2, int sub, uint32_t& sc,
                                             uint32_t& m) {
    const int j = sub & 3;
    const uint32_t a = byte_of(s0, j), b = byte_of(s1, j), c = byte_of(s2, j);
    const uint32_t hi = 0u - (uint32_t)((sub >> 2) & 1);       // all ones for sub >= 4
    sc = ((a & 63u) & ~hi) | (((c & 0xfu) | ((a >> 2) & 0x30u)) & hi);
    m = ((b & 63u) & ~hi) | (((c >> 4) | ((b >> 2) & 0x30u)) & hi);
}

}  // namespace wf
