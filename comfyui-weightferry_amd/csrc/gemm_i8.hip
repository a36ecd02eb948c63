// Int8 W8A8 linear for gfx950: out[m, n] = OUT((float(acc) * xs[m]) * ws[n] (+ bias[n])), acc = sum_k xq[m, k] *
// wq[n, k] exactly in int32 -- the role of kitchen's cutlass_int8_dequant (enhancers/fused_int8.py:191-206).
//
// Tiling: a 256-thread workgroup computes a BM x BN tile with 2 x 2 waves; a wave owns WM x WN 32x32 tiles of
// v_mfma_i32_32x32x32_i8 (64 lanes x 16 int8 per operand, 16 int32 accumulators per lane). K advances in stages
// of 128 bytes: each stage of A (xq rows) and B (wq rows, K-major like A) is loaded from global memory into
// registers one stage ahead and written to a double-buffered LDS tile. Rows are 128 bytes = 8 chunks of 16 bytes;
// chunk c of row r sits at chunk slot c ^ ((r >> 1) & 7), so the 16 lanes of each quarter-wave hit 16 different
// 16-byte bank groups both when a stage is written and when 32 rows' fragments are read.
//
// Operand layout (both operands the same): lane l of a 32x32x32 fragment holds 16 bytes of row l % 32 at K offset
// 16 * (l / 32) of the 32-wide K step. Result layout: lane l, register i holds row 8 (i / 4) + 4 (l / 32) + i % 4,
// column l % 32 of the 32x32 tile.
//
// Tile order is XCD-aware: workgroup w runs on XCD w % 8, so consecutive tile indices are dealt to one XCD's
// workgroups and that XCD's L2 sees neighbouring tiles (they share A rows / B rows); within the order, tiles are
// grouped GROUP_M tile-rows at a time.

#include "wf_common.h"

namespace wf {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 128;        // K bytes per stage
constexpr int kGroupM = 8;      // tile-rows per group of the tile order

#ifndef GEMM_SWZ_NEW
#define GEMM_SWZ_NEW 1
#endif
__device__ __forceinline__ int swz(int row, int chunk) {
#if GEMM_SWZ_NEW
    return chunk ^ (((row >> 1) ^ ((row & 1) << 2)) & 7);
#else
    return chunk ^ ((row >> 1) & 7);
#endif
}

__device__ __forceinline__ float to_f32_out(const void* p, int64_t i, int dt) {
    if (dt == WF_BF16) return __uint_as_float((uint32_t)static_cast<const uint16_t*>(p)[i] << 16);
    if (dt == WF_F16) return (float)__builtin_bit_cast(_Float16, static_cast<const uint16_t*>(p)[i]);
    return static_cast<const float*>(p)[i];
}

// tile index of workgroup w among T tiles (XCD-aware), then grouped row-major order over (tm, tn)
__device__ __forceinline__ void tile_of(int w, int T, int ntm, int ntn, int& tm, int& tn) {
    int L = w;
    if ((T & 7) == 0) L = (w & 7) * (T >> 3) + (w >> 3);
    const int per_group = kGroupM * ntn;
    const int group = L / per_group;
    const int first_m = group * kGroupM;
    const int gm = min(ntm - first_m, kGroupM);
    const int in = L - group * per_group;
    tm = first_m + in % gm;
    tn = in / gm;
}

// Epilogue operands of the residual variant: out = OUT(resid + gate[m / rows_per_group] * t), t the plain epilogue
// value before rounding (the role of kitchen's cutlass_int8_dequant_residual, enhancers/fused_int8.py:212-268).
struct Residual {
    const uint16_t* gate;    // bf16 [groups, N]
    const uint16_t* resid;   // bf16 [M, N]
    int rows_per_group;
};

template <int WM, int WN, int OUT, bool BIAS, bool RESID = false>
__global__ __launch_bounds__(256) void gemm_i8(const int8_t* __restrict__ A, const int8_t* __restrict__ B,
                                               const float* __restrict__ xs, const float* __restrict__ ws,
                                               const void* __restrict__ bias, void* __restrict__ out,
                                               int M, int N, int K, Residual res = {}) {
    constexpr int BM = 2 * WM * 32, BN = 2 * WN * 32;
    constexpr int ACH = BM * 8 / 256, BCH = BN * 8 / 256;     // 16-byte chunks per thread per stage
    __shared__ uint4 lds[2][(BM + BN) * 8];
    const int ntm = (M + BM - 1) / BM, ntn = (N + BN - 1) / BN;
    int tm, tn;
    tile_of(blockIdx.x, ntm * ntn, ntm, ntn, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int nk = (K + kBK - 1) / kBK;

    uint4 ra[ACH], rb[BCH];
    auto gload = [&](int kt) {
        const int k0 = kt * kBK;
#pragma unroll
        for (int i = 0; i < ACH; i++) {
            const int idx = tid + 256 * i, r = idx >> 3, c = idx & 7;
            const int gm = m0 + r, gk = k0 + 16 * c;
            ra[i] = (gm < M && gk < K) ? *reinterpret_cast<const uint4*>(A + (int64_t)gm * K + gk)
                                       : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < BCH; i++) {
            const int idx = tid + 256 * i, r = idx >> 3, c = idx & 7;
            const int gn = n0 + r, gk = k0 + 16 * c;
            rb[i] = (gn < N && gk < K) ? *reinterpret_cast<const uint4*>(B + (int64_t)gn * K + gk)
                                       : make_uint4(0, 0, 0, 0);
        }
    };
    auto lstore = [&](int buf) {
        uint4* sa = lds[buf];
        uint4* sb = lds[buf] + BM * 8;
#pragma unroll
        for (int i = 0; i < ACH; i++) {
            const int idx = tid + 256 * i, r = idx >> 3, c = idx & 7;
            sa[r * 8 + swz(r, c)] = ra[i];
        }
#pragma unroll
        for (int i = 0; i < BCH; i++) {
            const int idx = tid + 256 * i, r = idx >> 3, c = idx & 7;
            sb[r * 8 + swz(r, c)] = rb[i];
        }
    };

    i32x16 acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0;

    gload(0);
    lstore(0);
    __syncthreads();
    const int lr = lane & 31, lk = lane >> 5;
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload(kt + 1);
        const uint4* sa = lds[cur];
        const uint4* sb = lds[cur] + BM * 8;
#pragma unroll
        for (int ks = 0; ks < kBK / 32; ks++) {
            const int ch = 2 * ks + lk;
            i32x4 af[WM], bf[WN];
#pragma unroll
            for (int i = 0; i < WM; i++) {
                const int r = wm * WM * 32 + i * 32 + lr;
                af[i] = __builtin_bit_cast(i32x4, sa[r * 8 + swz(r, ch)]);
            }
#pragma unroll
            for (int j = 0; j < WN; j++) {
                const int r = wn * WN * 32 + j * 32 + lr;
                bf[j] = __builtin_bit_cast(i32x4, sb[r * 8 + swz(r, ch)]);
            }
#pragma unroll
            for (int i = 0; i < WM; i++)
#pragma unroll
                for (int j = 0; j < WN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) lstore(cur ^ 1);
        __syncthreads();
    }

    // epilogue: (float(acc) * xs[m]) * ws[n] (+ bias[n]), rounded once to OUT
#pragma unroll
    for (int j = 0; j < WN; j++) {
        const int n = n0 + wn * WN * 32 + j * 32 + lr;
        if (n >= N) continue;
        const float wsn = ws[n];
        const float bn = BIAS ? to_f32_out(bias, n, OUT) : 0.0f;
#pragma unroll
        for (int i = 0; i < WM; i++) {
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int m = m0 + wm * WM * 32 + i * 32 + 8 * (e >> 2) + 4 * lk + (e & 3);
                if (m >= M) continue;
                float t = ((float)acc[i][j][e] * xs[m]) * wsn;
                if (BIAS) t = t + bn;
                const int64_t o = (int64_t)m * N + n;
                if constexpr (RESID) {
                    const float g = __uint_as_float((uint32_t)res.gate[(int64_t)(m / res.rows_per_group) * N + n] << 16);
                    const float r = __uint_as_float((uint32_t)res.resid[o] << 16);
                    t = r + g * t;
                }
                if constexpr (OUT == WF_BF16) {
                    static_cast<__bf16*>(out)[o] = (__bf16)t;
                } else {
                    static_cast<_Float16*>(out)[o] = (_Float16)t;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------------------- K % 128 == 0 path
// The same tiling with the main loop arranged for the MFMA pipe: A / B stages come in through buffer loads whose
// resource starts at the tile's first row and ends at the last valid row (rows past M or N read as zeros, with no
// branch), fragments are double-buffered in registers (the reads of K step ks + 1 are issued before the MFMAs of
// step ks), and the next stage's LDS writes follow the current stage's last fragment reads.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const int8_t* base, int64_t bytes) {
    const int32_t n = bytes > 0x7fffffff ? 0x7fffffff : (int32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(base), 0, n, 0x00020000);
}

#ifndef GEMM_I8_LSTORE_LATE
#define GEMM_I8_LSTORE_LATE 0
#endif

// VM x VN waves, each owning WM x WN 32x32 tiles: BM = 32 VM WM, BN = 32 VN WN, 64 VM VN threads.
template <int VM, int VN, int WM, int WN, int OUT, bool BIAS, bool RESID>
__global__ __launch_bounds__(64 * VM * VN) void gemm_i8_k128(const int8_t* __restrict__ A,
                                                             const int8_t* __restrict__ B,
                                                             const float* __restrict__ xs,
                                                             const float* __restrict__ ws,
                                                             const void* __restrict__ bias, void* __restrict__ out,
                                                             int M, int N, int K, Residual res) {
    constexpr int NT = 64 * VM * VN;
    constexpr int BM = VM * WM * 32, BN = VN * WN * 32;
    constexpr int ACH = BM * 8 / NT, BCH = BN * 8 / NT;
    constexpr int KS = kBK / 32;
    __shared__ uint4 lds[2][(BM + BN) * 8];
    const int ntm = (M + BM - 1) / BM, ntn = (N + BN - 1) / BN;
    int tm, tn;
    tile_of(blockIdx.x, ntm * ntn, ntm, ntn, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / VN, wn = wave % VN;
    const int nk = K / kBK;
    const __amdgpu_buffer_rsrc_t ra_rsrc = tile_rsrc(A + (int64_t)m0 * K, (int64_t)(M - m0) * K);
    const __amdgpu_buffer_rsrc_t rb_rsrc = tile_rsrc(B + (int64_t)n0 * K, (int64_t)(N - n0) * K);

    uint32_t aoff[ACH], boff[BCH];
    int aslot[ACH], bslot[BCH];
#pragma unroll
    for (int i = 0; i < ACH; i++) {
        const int idx = tid + NT * i, r = idx >> 3, c = idx & 7;
        aoff[i] = (uint32_t)(r * K + 16 * c);
        aslot[i] = r * 8 + swz(r, c);
    }
#pragma unroll
    for (int i = 0; i < BCH; i++) {
        const int idx = tid + NT * i, r = idx >> 3, c = idx & 7;
        boff[i] = (uint32_t)(r * K + 16 * c);
        bslot[i] = BM * 8 + r * 8 + swz(r, c);
    }
    i32x4 ra[ACH], rb[BCH];
    auto gload = [&](int kt) {
        const uint32_t k0 = (uint32_t)kt * kBK;
#pragma unroll
        for (int i = 0; i < ACH; i++) ra[i] = __builtin_amdgcn_raw_buffer_load_b128(ra_rsrc, aoff[i] + k0, 0, 0);
#pragma unroll
        for (int i = 0; i < BCH; i++) rb[i] = __builtin_amdgcn_raw_buffer_load_b128(rb_rsrc, boff[i] + k0, 0, 0);
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < ACH; i++) lds[buf][aslot[i]] = __builtin_bit_cast(uint4, ra[i]);
#pragma unroll
        for (int i = 0; i < BCH; i++) lds[buf][bslot[i]] = __builtin_bit_cast(uint4, rb[i]);
    };
    const int lr = lane & 31, lk = lane >> 5;
    int arow[WM], brow[WN];
#pragma unroll
    for (int i = 0; i < WM; i++) arow[i] = wm * WM * 32 + i * 32 + lr;
#pragma unroll
    for (int j = 0; j < WN; j++) brow[j] = BM + wn * WN * 32 + j * 32 + lr;
    i32x4 fa[2][WM], fb[2][WN];
    auto fread = [&](int buf, int ks, int set) {
        const int ch = 2 * ks + lk;
#pragma unroll
        for (int i = 0; i < WM; i++) fa[set][i] = __builtin_bit_cast(i32x4, lds[buf][arow[i] * 8 + swz(arow[i], ch)]);
#pragma unroll
        for (int j = 0; j < WN; j++) fb[set][j] = __builtin_bit_cast(i32x4, lds[buf][brow[j] * 8 + swz(brow[j], ch)]);
    };

    i32x16 acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0;

    gload(0);
    lstore(0);
    __syncthreads();
    fread(0, 0, 0);
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) gload(kt + 1);
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const int set = ks & 1;
            if (ks + 1 < KS) fread(cur, ks + 1, set ^ 1);
#pragma unroll
            for (int i = 0; i < WM; i++)
#pragma unroll
                for (int j = 0; j < WN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[set][i], fb[set][j], acc[i][j], 0, 0, 0);
            if (!GEMM_I8_LSTORE_LATE && ks == KS - 2 && more) lstore(cur ^ 1);
        }
        if (more) {
            if (GEMM_I8_LSTORE_LATE) lstore(cur ^ 1);     // the other buffer: nobody reads it in this stage
            __syncthreads();
            fread(cur ^ 1, 0, 0);
        }
    }

    // epilogue: (float(acc) * xs[m]) * ws[n] (+ bias[n]), rounded once to OUT
#pragma unroll
    for (int j = 0; j < WN; j++) {
        const int n = n0 + wn * WN * 32 + j * 32 + lr;
        if (n >= N) continue;
        const float wsn = ws[n];
        const float bn = BIAS ? to_f32_out(bias, n, OUT) : 0.0f;
#pragma unroll
        for (int i = 0; i < WM; i++) {
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int m = m0 + wm * WM * 32 + i * 32 + 8 * (e >> 2) + 4 * lk + (e & 3);
                if (m >= M) continue;
                float t = ((float)acc[i][j][e] * xs[m]) * wsn;
                if (BIAS) t = t + bn;
                const int64_t o = (int64_t)m * N + n;
                if constexpr (RESID) {
                    const float g = __uint_as_float((uint32_t)res.gate[(int64_t)(m / res.rows_per_group) * N + n] << 16);
                    const float r = __uint_as_float((uint32_t)res.resid[o] << 16);
                    t = r + g * t;
                }
                if constexpr (OUT == WF_BF16) {
                    static_cast<__bf16*>(out)[o] = (__bf16)t;
                } else {
                    static_cast<_Float16*>(out)[o] = (_Float16)t;
                }
            }
        }
    }
}

#ifndef GEMM_I8_SHAPE
#define GEMM_I8_SHAPE 2
#endif

// K % 128 == 0: the tile shape by output size. Shape 1: 4 waves of 4 x 4 tiles (256 x 256, one wave per SIMD);
// shape 2: 8 waves of 4 x 2 tiles (256 x 256, two waves per SIMD); small outputs: 4 waves of 2 x 2 (128 x 128).
template <int VM, int VN, int WM, int WN, int OUT>
static void launch_k128_shape(const int8_t* A, const int8_t* B, const float* xs, const float* ws, const void* bias,
                              void* out, int M, int N, int K, Residual r, bool resid, hipStream_t s) {
    constexpr int BM = VM * WM * 32, BN = VN * WN * 32, NT = 64 * VM * VN;
    const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    if (resid) gemm_i8_k128<VM, VN, WM, WN, OUT, false, true><<<dim3(tiles), NT, 0, s>>>(A, B, xs, ws, nullptr, out, M, N, K, r);
    else if (bias) gemm_i8_k128<VM, VN, WM, WN, OUT, true, false><<<dim3(tiles), NT, 0, s>>>(A, B, xs, ws, bias, out, M, N, K, r);
    else gemm_i8_k128<VM, VN, WM, WN, OUT, false, false><<<dim3(tiles), NT, 0, s>>>(A, B, xs, ws, bias, out, M, N, K, r);
}

template <int OUT>
static void launch_k128(const int8_t* A, const int8_t* B, const float* xs, const float* ws, const void* bias,
                        void* out, int M, int N, int K, Residual r, bool resid, hipStream_t s) {
    const int64_t big_tiles = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
    if (big_tiles < 512) launch_k128_shape<2, 2, 2, 2, OUT>(A, B, xs, ws, bias, out, M, N, K, r, resid, s);
    else if (GEMM_I8_SHAPE == 1) launch_k128_shape<2, 2, 4, 4, OUT>(A, B, xs, ws, bias, out, M, N, K, r, resid, s);
    else launch_k128_shape<2, 4, 4, 2, OUT>(A, B, xs, ws, bias, out, M, N, K, r, resid, s);
}

template <int WM, int WN, int OUT>
static void launch_gemm(const int8_t* A, const int8_t* B, const float* xs, const float* ws, const void* bias,
                        void* out, int M, int N, int K, hipStream_t s) {
    constexpr int BM = 2 * WM * 32, BN = 2 * WN * 32;
    const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    if (K % kBK == 0) {
        launch_k128<OUT>(A, B, xs, ws, bias, out, M, N, K, {}, false, s);
        return;
    }
    if (bias) gemm_i8<WM, WN, OUT, true><<<dim3(tiles), 256, 0, s>>>(A, B, xs, ws, bias, out, M, N, K);
    else gemm_i8<WM, WN, OUT, false><<<dim3(tiles), 256, 0, s>>>(A, B, xs, ws, bias, out, M, N, K);
}

template <int OUT>
static void dispatch(const int8_t* A, const int8_t* B, const float* xs, const float* ws, const void* bias,
                     void* out, int M, int N, int K, hipStream_t s) {
    // large outputs: 256 x 256 tiles (4 x 4 MFMA tiles per wave); small ones keep 128 x 128 to fill the chip
    const int64_t big_tiles = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
    if (big_tiles >= 512) launch_gemm<4, 4, OUT>(A, B, xs, ws, bias, out, M, N, K, s);
    else launch_gemm<2, 2, OUT>(A, B, xs, ws, bias, out, M, N, K, s);
}

template <int WM, int WN>
static void launch_resid(const int8_t* A, const int8_t* B, const float* xs, const float* ws, void* out, int M, int N,
                         int K, Residual r, hipStream_t s) {
    constexpr int BM = 2 * WM * 32, BN = 2 * WN * 32;
    const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    if (K % kBK == 0)
        launch_k128<WF_BF16>(A, B, xs, ws, nullptr, out, M, N, K, r, true, s);
    else
        gemm_i8<WM, WN, WF_BF16, false, true><<<dim3(tiles), 256, 0, s>>>(A, B, xs, ws, nullptr, out, M, N, K, r);
}

}  // namespace wf

extern "C" int wf_linear_i8_residual(const int8_t* xq, const int8_t* wq, const float* xs, const float* ws,
                                     const void* gate_bf16, const void* resid_bf16, void* out_bf16, int64_t M,
                                     int64_t N, int64_t K, int64_t rows_per_group, void* stream) {
    using namespace wf;
    if (M < 0 || N < 0 || K <= 0 || rows_per_group <= 0) { set_error("wf_linear_i8_residual: bad sizes"); return WF_EINVAL; }
    if (M == 0 || N == 0) return WF_OK;
    if (!xq || !wq || !xs || !ws || !gate_bf16 || !resid_bf16 || !out_bf16) { set_error("wf_linear_i8_residual: null pointer"); return WF_EINVAL; }
    if (K % 16 || !aligned(xq, 16) || !aligned(wq, 16)) {
        set_error("wf_linear_i8_residual: K %% 16 == 0 and 16-byte aligned operands are required");
        return WF_EUNSUPPORTED;
    }
    if (M % rows_per_group) { set_error("wf_linear_i8_residual: M is not a whole number of row groups"); return WF_EUNSUPPORTED; }
    if (M >= (1LL << 31) || N >= (1LL << 31) || K > 131071) { set_error("wf_linear_i8_residual: sizes too large"); return WF_EUNSUPPORTED; }
    Residual r{static_cast<const uint16_t*>(gate_bf16), static_cast<const uint16_t*>(resid_bf16), (int)rows_per_group};
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t big_tiles = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
    if (big_tiles >= 512) launch_resid<4, 4>(xq, wq, xs, ws, out_bf16, (int)M, (int)N, (int)K, r, s);
    else launch_resid<2, 2>(xq, wq, xs, ws, out_bf16, (int)M, (int)N, (int)K, r, s);
    WF_LAUNCH_CHECK("wf_linear_i8_residual launch");
    return WF_OK;
}

extern "C" int wf_linear_i8(const int8_t* xq, const int8_t* wq, const float* xs, const float* ws, const void* bias,
                            void* out, int out_dt, int64_t M, int64_t N, int64_t K, void* stream) {
    using namespace wf;
    if (M < 0 || N < 0 || K <= 0) { set_error("wf_linear_i8: M, N, K = %lld, %lld, %lld", (long long)M, (long long)N, (long long)K); return WF_EINVAL; }
    if (M == 0 || N == 0) return WF_OK;
    if (!xq || !wq || !xs || !ws || !out) { set_error("wf_linear_i8: null pointer"); return WF_EINVAL; }
    if (out_dt != WF_BF16 && out_dt != WF_F16) { set_error("wf_linear_i8: output dtype %d", out_dt); return WF_EUNSUPPORTED; }
    if (K % 16 || !aligned(xq, 16) || !aligned(wq, 16)) {
        set_error("wf_linear_i8: K %% 16 == 0 and 16-byte aligned operands are required");
        return WF_EUNSUPPORTED;
    }
    if (M >= (1LL << 31) || N >= (1LL << 31) || K >= (1LL << 31) || M * N >= (1LL << 62)) {
        set_error("wf_linear_i8: sizes beyond this build's 32-bit tile indices");
        return WF_EUNSUPPORTED;
    }
    // int32 accumulation is exact when K * 128 * 128 < 2^31
    if (K > 131071) { set_error("wf_linear_i8: K = %lld would overflow the int32 accumulator", (long long)K); return WF_EUNSUPPORTED; }
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (out_dt == WF_BF16) dispatch<WF_BF16>(xq, wq, xs, ws, bias, out, (int)M, (int)N, (int)K, s);
    else dispatch<WF_F16>(xq, wq, xs, ws, bias, out, (int)M, (int)N, (int)K, s);
    WF_LAUNCH_CHECK("wf_linear_i8 launch");
    return WF_OK;
}
