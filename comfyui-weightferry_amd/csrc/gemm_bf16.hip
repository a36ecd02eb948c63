// Plain bf16 GEMM for gfx950: y[m, n] = bf16(sum_k x[m, k] * w[n, k] (+ bias[n])), float32 accumulation -- the
// second step of the two-step GGUF flow, in place of ComfyUI-GGUF's torch.nn.functional.linear on the weight that
// wf_dequant produced (enhancers/gguf_dequant.py:296-326 returns the weight to ComfyUI-GGUF, which multiplies).
//
// Both operands ([M, K] and [N, K], K-major) stream in whole 128-byte lines through two LDS stage buffers
// (wl_ring.h); VM x VN waves of WM x WN v_mfma_f32_32x32x16_bf16 tiles; the epilogue adds the bias, rounds once to
// bf16 and stores whole 16-byte row runs through the idle stage buffers.

#include <algorithm>

#include "wl_ring.h"

namespace wf {

typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));
typedef float f32x16v __attribute__((ext_vector_type(16)));

template <typename S, bool BIAS>
__global__ __launch_bounds__(S::NT) void gemm_bf16(const uint16_t* __restrict__ A, const uint16_t* __restrict__ B,
                                                   const uint16_t* __restrict__ bias, uint16_t* __restrict__ Y, int M,
                                                   int N, int K) {
    constexpr int WM = S::WM, WN = S::WN;
    __shared__ wl_frag sb0[S::SLOTS], sb1[S::SLOTS];
    const int ntm = (M + S::BM - 1) / S::BM, ntn = (N + S::BN - 1) / S::BN;
    int tm, tn;
    tile_order(blockIdx.x, ntm * ntn, ntm, ntn, tm, tn);
    // (the tile order's divisions run on the vector unit: back to scalar registers, so the buffer resources stay
    // scalar)
    const int m0 = __builtin_amdgcn_readfirstlane(tm * S::BM), n0 = __builtin_amdgcn_readfirstlane(tn * S::BN);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t KB = (uint32_t)K * 2u;
    const __amdgpu_buffer_rsrc_t ra = tile_rsrc(A + (int64_t)m0 * K, (int64_t)(M - m0) * K * 2);
    const __amdgpu_buffer_rsrc_t rb = tile_rsrc(B + (int64_t)n0 * K, (int64_t)(N - n0) * K * 2);
    f32x16v acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;
    wl_mainloop<S>(ra, rb, KB, (int)(KB / 128), wave, lane, sb0, sb1, acc,
                   [](const f32x16v& c, const wl_frag& a, const wl_frag& b) {
                       return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8v, a),
                                                                      __builtin_bit_cast(bf16x8v, b), c, 0, 0, 0);
                   });
    const int wm = wave / S::VN, wn = wave % S::VN;
    const int mw = m0 + wm * WM * 32, nw = n0 + wn * WN * 32;
    const int lr = lane & 31;
    float bn[WN];
#pragma unroll
    for (int j = 0; j < WN; j++) {
        const int n = nw + j * 32 + lr;
        bn[j] = BIAS && n < N ? __uint_as_float((uint32_t)bias[n] << 16) : 0.0f;
    }
    wl_store_tile<WM, WN>(wl_out_region<S>(sb0, sb1, wave), Y, M, N, mw, nw, lane, [&](int i, int j, int e) {
        float t = acc[i][j][e];
        if (BIAS) t = t + bn[j];
        return __builtin_bit_cast(uint16_t, (__bf16)t);
    });
}

template <int VM, int VN, int WM, int WN>
static void launch_bf16(const uint16_t* A, const uint16_t* B, const uint16_t* bias, uint16_t* Y, int M, int N, int K,
                        hipStream_t s) {
    using S = WlShape<VM, VN, WM, WN>;
    const int tiles = ((M + S::BM - 1) / S::BM) * ((N + S::BN - 1) / S::BN);
    if (bias) gemm_bf16<S, true><<<dim3(tiles), S::NT, 0, s>>>(A, B, bias, Y, M, N, K);
    else gemm_bf16<S, false><<<dim3(tiles), S::NT, 0, s>>>(A, B, bias, Y, M, N, K);
}

// modelled time of a tiling: whole rounds of 256 workgroups x tile area / relative efficiency (per mille)
static int64_t bf16_cost(int64_t M, int64_t N, int bm, int bn, int64_t eff) {
    const int64_t tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    return (tiles + 255) / 256 * bm * bn * 1000 / eff;
}

// 256 x 320 (8 waves of 2 x 5 MFMA tiles), 256 x 256 (8 waves of 4 x 2), 256 x 128 (4 waves of 4 x 2) or 128 x 160
// (4 waves of 1 x 5), by modelled time
static void run_bf16(const uint16_t* A, const uint16_t* B, const uint16_t* bias, uint16_t* Y, int M, int N, int K,
                     hipStream_t s) {
    const int64_t c320 = bf16_cost(M, N, 256, 320, 1000), c256 = bf16_cost(M, N, 256, 256, 900);
    const int64_t c128 = bf16_cost(M, N, 256, 128, 700), c160 = bf16_cost(M, N, 128, 160, 650);
    const int64_t best = std::min(std::min(c320, c256), std::min(c128, c160));
    const int form = best == c320 ? 0 : best == c256 ? 1 : best == c128 ? 2 : 3;
    switch (form) {
    case 0: launch_bf16<4, 2, 2, 5>(A, B, bias, Y, M, N, K, s); break;
    case 1: launch_bf16<2, 4, 4, 2>(A, B, bias, Y, M, N, K, s); break;
    case 2: launch_bf16<2, 2, 4, 2>(A, B, bias, Y, M, N, K, s); break;
    default: launch_bf16<4, 1, 1, 5>(A, B, bias, Y, M, N, K, s); break;
    }
}

}  // namespace wf

extern "C" int wf_linear_bf16(const void* x_bf16, const void* w_bf16, const void* bias_bf16, void* out_bf16,
                              int64_t M, int64_t N, int64_t K, void* stream) {
    using namespace wf;
    if (M < 0 || N < 0 || K <= 0) {
        set_error("wf_linear_bf16: M, N, K = %lld, %lld, %lld", (long long)M, (long long)N, (long long)K);
        return WF_EINVAL;
    }
    if (M == 0 || N == 0) return WF_OK;
    if (!x_bf16 || !w_bf16 || !out_bf16) { set_error("wf_linear_bf16: null pointer"); return WF_EINVAL; }
    if (K % 64 || !aligned(x_bf16, 16) || !aligned(w_bf16, 16) || (bias_bf16 && !aligned(bias_bf16, 2)) ||
        !aligned(out_bf16, 2)) {
        set_error("wf_linear_bf16: K %% 64 == 0 and 16-byte aligned operands are required");
        return WF_EUNSUPPORTED;
    }
    if (M >= (1LL << 31) || N >= (1LL << 31) || M * K * 2 >= (1LL << 31) || N * K * 2 >= (1LL << 31)) {
        set_error("wf_linear_bf16: operands beyond the buffer resources' 32-bit byte range");
        return WF_EUNSUPPORTED;
    }
    run_bf16(static_cast<const uint16_t*>(x_bf16), static_cast<const uint16_t*>(w_bf16),
             static_cast<const uint16_t*>(bias_bf16), static_cast<uint16_t*>(out_bf16), (int)M, (int)N, (int)K,
             static_cast<hipStream_t>(stream));
    WF_LAUNCH_CHECK("wf_linear_bf16 launch");
    return WF_OK;
}
