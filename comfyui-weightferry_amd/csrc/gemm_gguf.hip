// Fused K-quant dequantisation + bf16 GEMM for gfx950: y[m, n] = bf16(sum_k x[m, k] * W[n, k] (+ bias[n])), W the
// GGUF weight (Q4_K / Q5_K / Q6_K, [N, K] in 256-value super-blocks along K) dequantised inside the kernel with the
// reference's rounding chain (MID, then bf16 -- enhancers/gguf_dequant.py:195-224,250), float32 accumulation.
// The reference does the dequantisation into a bf16 weight in HBM and then ComfyUI-GGUF's F.linear; here the
// weight never leaves the chip in bf16.
//
// Tiling: a 256-thread workgroup computes a 256 x 256 tile with 2 x 2 waves of 128 x 128 (4 x 4 tiles of
// v_mfma_f32_32x32x16_bf16). K advances in stages of 64 (128 bytes of bf16 per row): the activation stage is
// loaded from global memory into registers one stage ahead; for the weight stage, thread t takes row n0 + t and
// dequantises its 64 values (one sub-block pair of the super-block) from the raw blocks, also one stage ahead.
// Both land in double-buffered LDS with the 16-byte chunk swizzle c ^ ((r >> 1) & 7) (conflict-free writes and
// fragment reads). Fragment layout: lane l holds 8 bf16 of row l % 32 at K offset 8 * (l / 32) of the 16-wide
// step; result layout: lane l, register i -> row 8 (i / 4) + 4 (l / 32) + i % 4, column l % 32.

#include "kquant.h"

namespace wf {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kGroupMG = 8;

__device__ __forceinline__ int swz8(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

__device__ __forceinline__ void tile_order(int w, int T, int ntm, int ntn, int& tm, int& tn) {
    int L = w;
    if ((T & 7) == 0) L = (w & 7) * (T >> 3) + (w >> 3);
    const int per_group = kGroupMG * ntn;
    const int group = L / per_group;
    const int first_m = group * kGroupMG;
    const int gm = min(ntm - first_m, kGroupMG);
    const int in = L - group * per_group;
    tm = first_m + in % gm;
    tn = in / gm;
}

// ND dwords of the bytes at p + o (an even address): loads the ND + 1 aligned dwords from a = (p + o) & ~3, i.e.
// [a, a + 4 ND + 4), which is [p + o - 2, p + o + 4 ND + 2) or [p + o, p + o + 4 ND + 4) -- callers keep both
// inside the super-block -- and shifts them into place.
template <int ND>
__device__ __forceinline__ void load_words(const uint8_t* p, uint32_t o, uint32_t (&w)[ND]) {
    const uintptr_t addr = reinterpret_cast<uintptr_t>(p + o);
    const uint32_t* d = reinterpret_cast<const uint32_t*>(addr & ~(uintptr_t)3);
    const uint32_t sh = (uint32_t)(addr & 3u) * 8u;
    uint32_t raw[ND + 1];
#pragma unroll
    for (int i = 0; i <= ND; i++) raw[i] = d[i];
#pragma unroll
    for (int i = 0; i < ND; i++) w[i] = __builtin_amdgcn_alignbit(raw[i + 1], raw[i], sh);
}

// raw bytes a thread needs for one row's 64 values of a stage
template <int QT>
struct StageRaw;
template <> struct StageRaw<12> { uint4 hdr; uint32_t q[8]; };
template <> struct StageRaw<13> { uint4 hdr; uint32_t q[8]; uint32_t qh[8]; };
template <> struct StageRaw<14> { uint32_t ql[16]; uint32_t qh[8]; uint32_t sc; uint32_t d; };

// Q4_K / Q5_K: pair p = sub-blocks 2p (low nibbles of qs[32p .. 32p + 32)) and 2p + 1 (high nibbles)
template <int QT>
__device__ __forceinline__ void raw_load(const uint8_t* sbp, int part, StageRaw<QT>& r) {
    if constexpr (QT == 12 || QT == 13) {
        constexpr int QS = QT == 12 ? 16 : 48;
        r.hdr = *reinterpret_cast<const uint4*>(sbp);
        const uint4 a = *reinterpret_cast<const uint4*>(sbp + QS + 32 * part);
        const uint4 b = *reinterpret_cast<const uint4*>(sbp + QS + 32 * part + 16);
        r.q[0] = a.x; r.q[1] = a.y; r.q[2] = a.z; r.q[3] = a.w;
        r.q[4] = b.x; r.q[5] = b.y; r.q[6] = b.z; r.q[7] = b.w;
        if constexpr (QT == 13) {
            const uint4 c = *reinterpret_cast<const uint4*>(sbp + 16);
            const uint4 e = *reinterpret_cast<const uint4*>(sbp + 32);
            r.qh[0] = c.x; r.qh[1] = c.y; r.qh[2] = c.z; r.qh[3] = c.w;
            r.qh[4] = e.x; r.qh[5] = e.y; r.qh[6] = e.z; r.qh[7] = e.w;
        }
    } else {
        // Q6_K values 64 part .. 64 part + 63: half h = part / 2; ql[64h .. +64), qh[32h .. +32), scales
        // 4 part .. 4 part + 3, d. The super-block may start 2 (mod 4) bytes into a dword.
        const int h = part >> 1;
        load_words<16>(sbp, 64 * h, r.ql);          // bytes [64h - 2, 64h + 68) at most: inside the 210
        load_words<8>(sbp, 128 + 32 * h, r.qh);     // bytes [126 + 32h, 164 + 32h) at most: inside
        const uint16_t* sc16 = reinterpret_cast<const uint16_t*>(sbp + 192 + 4 * part);
        r.sc = (uint32_t)sc16[0] | ((uint32_t)sc16[1] << 16);
        r.d = *reinterpret_cast<const uint16_t*>(sbp + 208);
    }
}

// 64 values of the row, as 32 packed bf16 pairs (values 2i, 2i + 1 in o[i])
template <int QT, int MID>
__device__ __forceinline__ void raw_dequant(const StageRaw<QT>& r, int part, uint32_t (&o)[32]) {
    if constexpr (QT == 12 || QT == 13) {
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            lo[i] = r.q[i] & 0x0f0f0f0fu;
            hi[i] = (r.q[i] >> 4) & 0x0f0f0f0fu;
            if constexpr (QT == 13) {
                lo[i] |= ((r.qh[i] >> (2 * part)) & 0x01010101u) << 4;
                hi[i] |= ((r.qh[i] >> (2 * part + 1)) & 0x01010101u) << 4;
            }
        }
        uint32_t scA, mA, scB, mB;
        scale_min(r.hdr.y, r.hdr.z, r.hdr.w, 2 * part, scA, mA);
        scale_min(r.hdr.y, r.hdr.z, r.hdr.w, 2 * part + 1, scB, mB);
        if constexpr (MID == WF_F16) {
            const h2 dd = as_h2(r.hdr.x);
            const h2 off = h2s(-1024.0f);
            const h2 pA = dd * (as_h2(scA | (mA << 16) | 0x64006400u) + off);
            const h2 pB = dd * (as_h2(scB | (mB << 16) | 0x64006400u) + off);
            const h2 dsA = lo2(pA), dmA = hi2(pA), dsB = lo2(pB), dmB = hi2(pB);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const h2 a0 = dsA * (biased_lo(lo[i]) + off) - dmA, a1 = dsA * (biased_hi(lo[i]) + off) - dmA;
                const h2 b0 = dsB * (biased_lo(hi[i]) + off) - dmB, b1 = dsB * (biased_hi(hi[i]) + off) - dmB;
                o[2 * i] = pack_bf16((float)a0[0], (float)a0[1]);
                o[2 * i + 1] = pack_bf16((float)a1[0], (float)a1[1]);
                o[16 + 2 * i] = pack_bf16((float)b0[0], (float)b0[1]);
                o[16 + 2 * i + 1] = pack_bf16((float)b1[0], (float)b1[1]);
            }
        } else {
            const float d = round_to<MID>(f16_bits_to_f32(r.hdr.x & 0xffffu));
            const float dmin = round_to<MID>(f16_bits_to_f32(r.hdr.x >> 16));
            const float dsA = round_to<MID>(d * (float)scA), dmA = round_to<MID>(dmin * (float)mA);
            const float dsB = round_to<MID>(d * (float)scB), dmB = round_to<MID>(dmin * (float)mB);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float a[4], b[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    a[e] = round_to<MID>(round_to<MID>(dsA * (float)byte_of(lo[i], e)) - dmA);
                    b[e] = round_to<MID>(round_to<MID>(dsB * (float)byte_of(hi[i], e)) - dmB);
                }
                o[2 * i] = pack_bf16(a[0], a[1]);
                o[2 * i + 1] = pack_bf16(a[2], a[3]);
                o[16 + 2 * i] = pack_bf16(b[0], b[1]);
                o[16 + 2 * i + 1] = pack_bf16(b[2], b[3]);
            }
        }
    } else {
        // value l (0..63): low bits nibble (part & 1) of ql[l]; high bits of qh[l % 32] at shift 2 (2 (part & 1) +
        // l / 32); scale byte l / 16 of r.sc
        const uint32_t ns = 4u * (uint32_t)(part & 1);
        const uint32_t s0 = 2u * (2u * (uint32_t)(part & 1)), s1 = s0 + 2u;
        uint32_t code[16];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t hsh = i < 8 ? s0 : s1;
            code[i] = ((r.ql[i] >> ns) & 0x0f0f0f0fu) | (((r.qh[i & 7] >> hsh) & 0x03030303u) << 4);
        }
        if constexpr (MID == WF_F16) {
            const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)r.d);
            const h2 off = h2s(-1056.0f);
#pragma unroll
            for (int g = 0; g < 4; g++) {                 // scale g covers values 16g .. 16g + 15 = code[4g .. 4g + 3]
                h2 dsc;
                dsc[0] = (_Float16)(float)(int8_t)byte_of(r.sc, g);
                dsc[1] = dsc[0];
                h2 dd; dd[0] = d; dd[1] = d;
                const h2 ds = dd * dsc;
#pragma unroll
                for (int i = 4 * g; i < 4 * g + 4; i++) {
                    const h2 v0 = ds * (biased_lo(code[i]) + off), v1 = ds * (biased_hi(code[i]) + off);
                    o[2 * i] = pack_bf16((float)v0[0], (float)v0[1]);
                    o[2 * i + 1] = pack_bf16((float)v1[0], (float)v1[1]);
                }
            }
        } else {
            const float d = round_to<MID>(f16_bits_to_f32(r.d));
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const float ds = round_to<MID>(d * (float)(int8_t)byte_of(r.sc, g));
#pragma unroll
                for (int i = 4 * g; i < 4 * g + 4; i++) {
                    float v[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) v[e] = round_to<MID>(ds * (float)((int)byte_of(code[i], e) - 32));
                    o[2 * i] = pack_bf16(v[0], v[1]);
                    o[2 * i + 1] = pack_bf16(v[2], v[3]);
                }
            }
        }
    }
}

template <int QT>
struct GGUFTs { static constexpr int TS = QT == 12 ? 144 : QT == 13 ? 176 : 210; };

template <int QT, int MID, bool BIAS>
__global__ __launch_bounds__(256) void gemm_gguf(const uint16_t* __restrict__ X, const uint8_t* __restrict__ W,
                                                 const uint16_t* __restrict__ bias, uint16_t* __restrict__ Y,
                                                 int M, int N, int K) {
    constexpr int BM = 256, BN = 256, WT = 4;          // 4 x 4 MFMA tiles of 32 x 32 per wave
    constexpr int TS = GGUFTs<QT>::TS;
    constexpr int ACH = BM * 8 / 256;                  // 16-byte activation chunks per thread per stage
    __shared__ uint4 lds[2][(BM + BN) * 8];
    const int ntm = (M + BM - 1) / BM, ntn = (N + BN - 1) / BN;
    int tm, tn;
    tile_order(blockIdx.x, ntm * ntn, ntm, ntn, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int nk = K / 64;
    const int sbs_per_row = K / 256;
    const int wrow = n0 + tid;                         // this thread's weight row
    const bool wlive = wrow < N;
    const uint8_t* wrow_p = W + (int64_t)(wlive ? wrow : 0) * sbs_per_row * TS;

    uint4 ra[ACH];
    StageRaw<QT> rw;
    auto gload = [&](int kt) {
        const int k0 = kt * 64;
#pragma unroll
        for (int i = 0; i < ACH; i++) {
            const int idx = tid + 256 * i, r = idx >> 3, c = idx & 7;
            const int gm = m0 + r;
            ra[i] = gm < M ? *reinterpret_cast<const uint4*>(X + (int64_t)gm * K + k0 + 8 * c) : make_uint4(0, 0, 0, 0);
        }
        if (wlive) raw_load<QT>(wrow_p + (kt >> 2) * TS, kt & 3, rw);
    };
    auto lstore = [&](int buf, int kt) {
        uint4* sa = lds[buf];
        uint4* sb = lds[buf] + BM * 8;
#pragma unroll
        for (int i = 0; i < ACH; i++) {
            const int idx = tid + 256 * i, r = idx >> 3, c = idx & 7;
            sa[r * 8 + swz8(r, c)] = ra[i];
        }
        uint32_t o[32];
        if (wlive) {
            raw_dequant<QT, MID>(rw, kt & 3, o);
        } else {
#pragma unroll
            for (int i = 0; i < 32; i++) o[i] = 0;
        }
#pragma unroll
        for (int c = 0; c < 8; c++) sb[tid * 8 + swz8(tid, c)] = make_uint4(o[4 * c], o[4 * c + 1], o[4 * c + 2], o[4 * c + 3]);
    };

    f32x16 acc[WT][WT];
#pragma unroll
    for (int i = 0; i < WT; i++)
#pragma unroll
        for (int j = 0; j < WT; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

    gload(0);
    lstore(0, 0);
    __syncthreads();
    const int lr = lane & 31, lk = lane >> 5;
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload(kt + 1);
        const uint4* sa = lds[cur];
        const uint4* sb = lds[cur] + BM * 8;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const int ch = 2 * ks + lk;
            bf16x8 af[WT], bf[WT];
#pragma unroll
            for (int i = 0; i < WT; i++) {
                const int r = wm * WT * 32 + i * 32 + lr;
                af[i] = __builtin_bit_cast(bf16x8, sa[r * 8 + swz8(r, ch)]);
            }
#pragma unroll
            for (int j = 0; j < WT; j++) {
                const int r = wn * WT * 32 + j * 32 + lr;
                bf[j] = __builtin_bit_cast(bf16x8, sb[r * 8 + swz8(r, ch)]);
            }
#pragma unroll
            for (int i = 0; i < WT; i++)
#pragma unroll
                for (int j = 0; j < WT; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) lstore(cur ^ 1, kt + 1);
        __syncthreads();
    }

#pragma unroll
    for (int j = 0; j < WT; j++) {
        const int n = n0 + wn * WT * 32 + j * 32 + lr;
        if (n >= N) continue;
        const float bn = BIAS ? __uint_as_float((uint32_t)bias[n] << 16) : 0.0f;
#pragma unroll
        for (int i = 0; i < WT; i++) {
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int m = m0 + wm * WT * 32 + i * 32 + 8 * (e >> 2) + 4 * lk + (e & 3);
                if (m >= M) continue;
                float t = acc[i][j][e];
                if (BIAS) t = t + bn;
                Y[(int64_t)m * N + n] = __builtin_bit_cast(uint16_t, (__bf16)t);
            }
        }
    }
}

template <int QT, int MID>
static void launch(const uint16_t* X, const uint8_t* W, const uint16_t* bias, uint16_t* Y, int M, int N, int K,
                   hipStream_t s) {
    const int tiles = ((M + 255) / 256) * ((N + 255) / 256);
    if (bias) gemm_gguf<QT, MID, true><<<dim3(tiles), 256, 0, s>>>(X, W, bias, Y, M, N, K);
    else gemm_gguf<QT, MID, false><<<dim3(tiles), 256, 0, s>>>(X, W, bias, Y, M, N, K);
}

template <int QT>
static void launch_mid(int mid, const uint16_t* X, const uint8_t* W, const uint16_t* bias, uint16_t* Y, int M,
                       int N, int K, hipStream_t s) {
    if (mid == WF_F16) launch<QT, WF_F16>(X, W, bias, Y, M, N, K, s);
    else if (mid == WF_BF16) launch<QT, WF_BF16>(X, W, bias, Y, M, N, K, s);
    else launch<QT, WF_F32>(X, W, bias, Y, M, N, K, s);
}

}  // namespace wf

extern "C" int wf_linear_gguf(const void* x_bf16, int64_t M, int64_t K, const void* wq, int64_t wq_bytes,
                              int qtype, int64_t N, const void* bias_bf16, void* out_bf16, int mid_dt,
                              void* stream) {
    using namespace wf;
    if (qtype != 12 && qtype != 13 && qtype != 14) {
        set_error("wf_linear_gguf: GGML type %d is not handled (Q4_K, Q5_K, Q6_K)", qtype);
        return WF_EUNSUPPORTED;
    }
    if (mid_dt < 0 || mid_dt > 2) { set_error("wf_linear_gguf: dequant dtype %d", mid_dt); return WF_EUNSUPPORTED; }
    if (M < 0 || N < 0 || K <= 0) { set_error("wf_linear_gguf: M, N, K = %lld, %lld, %lld", (long long)M, (long long)N, (long long)K); return WF_EINVAL; }
    if (K % 256) { set_error("wf_linear_gguf: K = %lld is not a multiple of 256", (long long)K); return WF_EUNSUPPORTED; }
    const int ts = qtype == 12 ? 144 : qtype == 13 ? 176 : 210;
    if (wq_bytes != N * (K / 256) * ts) {
        set_error("wf_linear_gguf: %lld weight bytes for [%lld, %lld]", (long long)wq_bytes, (long long)N, (long long)K);
        return WF_EUNSUPPORTED;
    }
    if (M == 0 || N == 0) return WF_OK;
    if (!x_bf16 || !wq || !out_bf16) { set_error("wf_linear_gguf: null pointer"); return WF_EINVAL; }
    if (!aligned(x_bf16, 16) || !aligned(wq, 16) || !aligned(out_bf16, 2) || (bias_bf16 && !aligned(bias_bf16, 2))) {
        set_error("wf_linear_gguf: x and the weight blocks must be 16-byte aligned");
        return WF_EUNSUPPORTED;
    }
    if (M >= (1LL << 31) || N >= (1LL << 31) || K >= (1LL << 31)) { set_error("wf_linear_gguf: sizes too large"); return WF_EUNSUPPORTED; }
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint16_t* X = static_cast<const uint16_t*>(x_bf16);
    const uint8_t* W = static_cast<const uint8_t*>(wq);
    const uint16_t* B = static_cast<const uint16_t*>(bias_bf16);
    uint16_t* Y = static_cast<uint16_t*>(out_bf16);
    if (qtype == 12) launch_mid<12>(mid_dt, X, W, B, Y, (int)M, (int)N, (int)K, s);
    else if (qtype == 13) launch_mid<13>(mid_dt, X, W, B, Y, (int)M, (int)N, (int)K, s);
    else launch_mid<14>(mid_dt, X, W, B, Y, (int)M, (int)N, (int)K, s);
    WF_LAUNCH_CHECK("wf_linear_gguf launch");
    return WF_OK;
}
