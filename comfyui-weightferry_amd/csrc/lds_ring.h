// Helpers of the GEMM kernels that stream operands global -> LDS with the load unit (buffer_load ... lds) through a
// ring of LDS stages: buffer resources with zero fill past the end, the 16-byte LDS DMA, the row swizzles, a barrier
// without the workgroup fence, the XCD-aware tile order and a compile-time loop.
#pragma once

#include <type_traits>
#include <utility>

#include "wf_common.h"

namespace wf {

// buffer resource over [base, base + bytes): loads past the end read as zeros, with no branch
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void* base, int64_t bytes) {
    const int32_t n = bytes > 0x7fffffff ? 0x7fffffff : (int32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, n, 0x00020000);
}

// chunk c (16 bytes) of a 64-byte LDS row r sits at slot c ^ ((r >> 2) & 3): the 16 lanes that read the same chunk
// of 16 consecutive rows hit 16 different 16-byte bank groups
__device__ __forceinline__ int swz4(int row, int chunk) { return chunk ^ ((row >> 2) & 3); }

// chunk c (16 bytes) of a 128-byte LDS row r sits at slot c ^ (((r >> 1) ^ ((r & 1) << 2)) & 7): conflict-free for
// the fragment reads of one chunk of consecutive rows and for whole-row writes
__device__ __forceinline__ int swz8(int row, int chunk) { return chunk ^ (((row >> 1) ^ ((row & 1) << 2)) & 7); }

// 16 bytes per lane from buffer r at voffset into LDS slot `lane` of the 1 KiB run at lds (wave-uniform); the byte
// offset is in voffset so that the buffer's range check covers it. The address-space cast is device code only; the
// host pass never sees it.
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voffset) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voffset, 0, 0, 0);
#endif
}

// s_barrier without the workgroup fence __syncthreads adds (that fence waits for every outstanding load, which
// would drain the ring); the memory clobber keeps the compiler from moving LDS accesses across it
__device__ __forceinline__ void wave_barrier_sync() { asm volatile("s_barrier" ::: "memory"); }

// 16-byte LDS write issued as inline assembly. The compiler's wait insertion treats any LDS store that follows an
// in-flight LDS DMA as a possible overlap and drains every load first; this write targets a ring slot that no DMA
// writes (the caller's contract). Invisible to the compiler's LDS counter, it can only make the compiler's own
// lgkmcnt waits stricter (LDS operations of a wave complete in order), never wrong.
__device__ __forceinline__ void lds_write16(void* p, uint4 v) {
#if defined(__HIP_DEVICE_COMPILE__)
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    const uint32_t a = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)p;
    const u32x4_t d = {v.x, v.y, v.z, v.w};
    asm volatile("ds_write_b128 %0, %1" ::"v"(a), "v"(d));
#endif
}

// the same for 8 bytes (ds_write_b64; p 8-byte aligned)
__device__ __forceinline__ void lds_write8(void* p, uint32_t lo, uint32_t hi) {
#if defined(__HIP_DEVICE_COMPILE__)
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    const uint32_t a = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)p;
    const u32x2_t d = {lo, hi};
    asm volatile("ds_write_b64 %0, %1" ::"v"(a), "v"(d));
#endif
}

// s_waitcnt vmcnt(N) alone (expcnt and lgkmcnt left at their maxima), N a compile-time count
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// tile index of workgroup w among T tiles: XCD-aware (workgroup w runs on XCD w % 8, so one XCD's workgroups take
// consecutive tiles and share their operand rows in its L2), then groups of 8 tile-rows, column by column
__device__ __forceinline__ void tile_order(int w, int T, int ntm, int ntn, int& tm, int& tn) {
    constexpr int kGroupRows = 8;
    int L = w;
    if ((T & 7) == 0) L = (w & 7) * (T >> 3) + (w >> 3);
    const int per_group = kGroupRows * ntn;
    const int group = L / per_group;
    const int first_m = group * kGroupRows;
    const int gm = min(ntm - first_m, kGroupRows);
    const int in = L - group * per_group;
    tm = first_m + in % gm;
    tn = in / gm;
}

// f(std::integral_constant<int, 0>{}), ..., f(std::integral_constant<int, N - 1>{}), unrolled at compile time
template <typename F, int... I>
__device__ __forceinline__ void static_for_seq(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_seq(f, std::make_integer_sequence<int, N>{});
}

}  // namespace wf
