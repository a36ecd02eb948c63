// Fused K-quant dequantisation + bf16 GEMM for gfx950: y[m, n] = bf16(sum_k x[m, k] * W[n, k] (+ bias[n])), W the
// GGUF weight (Q4_K / Q5_K / Q6_K, [N, K] in 256-value super-blocks along K) dequantised inside the kernel with the
// reference's rounding chain (MID, then bf16 -- enhancers/gguf_dequant.py:195-224,250), float32 accumulation.
// The reference does the dequantisation into a bf16 weight in HBM and then ComfyUI-GGUF's F.linear; here the
// weight never leaves the chip in bf16.
//
// Tiling: a 256-thread workgroup computes a 256 x 128 tile with 2 x 2 waves of 128 x 64 (4 x 2 tiles of
// v_mfma_f32_32x32x16_bf16), and two workgroups share a CU (48 KB of LDS and at most 256 registers per lane each),
// so one workgroup's barrier waits, dequantisation and LDS writes run while the other's MFMAs do. K advances in
// stages of 64 (128 bytes of bf16 per row): the next stage's activations (buffer loads; rows past M read as zeros)
// and raw weight blocks come into registers while the current stage's MFMAs run; after a barrier the stage is
// written to the single LDS tile -- threads 2r and 2r + 1 take the two halves of weight row n0 + r (for Q4_K / Q5_K
// exactly one 32-value sub-block each) and dequantise them on the way -- and a second barrier publishes it. A
// 16-byte chunk swizzle keeps the LDS writes and fragment reads conflict-free. Fragment layout: lane l holds 8 bf16
// of row l % 32 at K offset 8 * (l / 32) of the 16-wide step; result layout: lane l, register i -> row
// 8 (i / 4) + 4 (l / 32) + i % 4, column l % 32.

#include "kquant.h"

namespace wf {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kGroupMG = 8;

__device__ __forceinline__ int swz8(int row, int chunk) { return chunk ^ (((row >> 1) ^ ((row & 1) << 2)) & 7); }

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

// Raw bytes a thread needs for its 32 values of a stage: half h (0 / 1) of the stage's 64-value slice `part`
// (0..3) of one super-block.
template <int QT>
struct HalfRaw;
template <> struct HalfRaw<12> { uint4 hdr; uint32_t q[8]; };
template <> struct HalfRaw<13> { uint4 hdr; uint32_t q[8]; uint32_t qh[8]; };
template <> struct HalfRaw<14> { uint32_t ql[8]; uint32_t qh[8]; uint32_t sc; uint32_t d; };

template <int QT>
__device__ __forceinline__ void half_load(const uint8_t* sbp, int part, int h, HalfRaw<QT>& r) {
    if constexpr (QT == 12 || QT == 13) {
        // Q4_K / Q5_K: sub-block 2 part + h = nibble h of qs[32 part .. 32 part + 32); Q5_K bit (2 part + h) of qh
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
        // Q6_K values 64 part + 32 h + i: ql[64 (part / 2) + 32 h + i] nibble (part & 1); qh[32 (part / 2) + i] at
        // shift 2 (2 (part & 1) + h); scales 4 part + 2 h + i / 16; d. Reads stay inside the 210-byte block.
        const int hh = part >> 1;
        load_words<8>(sbp, 64 * hh + 32 * h, r.ql);       // bytes up to 96 + 36 = 132
        load_words<8>(sbp, 128 + 32 * hh, r.qh);          // bytes up to 160 + 36 = 196
        r.sc = *reinterpret_cast<const uint16_t*>(sbp + 192 + 4 * part + 2 * h);
        r.d = *reinterpret_cast<const uint16_t*>(sbp + 208);
    }
}

// 32 values as 16 packed bf16 pairs (values 2i, 2i + 1 in o[i])
template <int QT, int MID>
__device__ __forceinline__ void half_dequant(const HalfRaw<QT>& r, int part, int h, uint32_t (&o)[16]) {
    if constexpr (QT == 12 || QT == 13) {
        const int sub = 2 * part + h;
        const uint32_t ns = 4u * (uint32_t)h;
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            q[i] = (r.q[i] >> ns) & 0x0f0f0f0fu;
            if constexpr (QT == 13) q[i] |= ((r.qh[i] >> sub) & 0x01010101u) << 4;
        }
        uint32_t sc, m;
        scale_min(r.hdr.y, r.hdr.z, r.hdr.w, sub, sc, m);
        if constexpr (MID == WF_F16) {
            const h2 off = h2s(-1024.0f);
            const h2 pr = as_h2(r.hdr.x) * (as_h2(sc | (m << 16) | 0x64006400u) + off);   // (d * sc, dmin * m)
            const h2 ds = lo2(pr), dm = hi2(pr);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const h2 v0 = ds * (biased_lo(q[i]) + off) - dm, v1 = ds * (biased_hi(q[i]) + off) - dm;
                o[2 * i] = pack_bf16((float)v0[0], (float)v0[1]);
                o[2 * i + 1] = pack_bf16((float)v1[0], (float)v1[1]);
            }
        } else {
            const float d = round_to<MID>(f16_bits_to_f32(r.hdr.x & 0xffffu));
            const float dmin = round_to<MID>(f16_bits_to_f32(r.hdr.x >> 16));
            const float ds = round_to<MID>(d * (float)sc), dm = round_to<MID>(dmin * (float)m);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = round_to<MID>(round_to<MID>(ds * (float)byte_of(q[i], e)) - dm);
                o[2 * i] = pack_bf16(v[0], v[1]);
                o[2 * i + 1] = pack_bf16(v[2], v[3]);
            }
        }
    } else {
        const uint32_t ns = 4u * (uint32_t)(part & 1);
        const uint32_t hs = 2u * (2u * (uint32_t)(part & 1) + (uint32_t)h);
        uint32_t code[8];
#pragma unroll
        for (int i = 0; i < 8; i++)
            code[i] = ((r.ql[i] >> ns) & 0x0f0f0f0fu) | (((r.qh[i] >> hs) & 0x03030303u) << 4);
        if constexpr (MID == WF_F16) {
            const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)r.d);
            const h2 off = h2s(-1056.0f);
            h2 dd; dd[0] = d; dd[1] = d;
            h2 sc2;
            sc2[0] = (_Float16)(float)(int8_t)byte_of(r.sc, 0);
            sc2[1] = (_Float16)(float)(int8_t)byte_of(r.sc, 1);
            const h2 pd = dd * sc2;                       // (d * sc[first 16], d * sc[second 16]), rounded to f16
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const h2 ds = i < 4 ? lo2(pd) : hi2(pd);
                const h2 v0 = ds * (biased_lo(code[i]) + off), v1 = ds * (biased_hi(code[i]) + off);
                o[2 * i] = pack_bf16((float)v0[0], (float)v0[1]);
                o[2 * i + 1] = pack_bf16((float)v1[0], (float)v1[1]);
            }
        } else {
            const float d = round_to<MID>(f16_bits_to_f32(r.d));
            const float ds0 = round_to<MID>(d * (float)(int8_t)byte_of(r.sc, 0));
            const float ds1 = round_to<MID>(d * (float)(int8_t)byte_of(r.sc, 1));
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float ds = i < 4 ? ds0 : ds1;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = round_to<MID>(ds * (float)((int)byte_of(code[i], e) - 32));
                o[2 * i] = pack_bf16(v[0], v[1]);
                o[2 * i + 1] = pack_bf16(v[2], v[3]);
            }
        }
    }
}

template <int QT>
struct GGUFTs { static constexpr int TS = QT == 12 ? 144 : QT == 13 ? 176 : 210; };

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const void* base, int64_t bytes) {
    const int32_t n = bytes > 0x7fffffff ? 0x7fffffff : (int32_t)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, n, 0x00020000);
}

// VM x VN waves of WM x WN 32x32 tiles; 64 VM VN threads; stage = 64 K values. Thread t dequantises half h = t & 1
// of weight row t >> 1 of the stage (BN = 32 VN WN = NT / 2 rows). WPE workgroups' waves share each SIMD.
template <int VM, int VN, int WM, int WN, int QT, int MID, bool BIAS, int WPE>
__global__ __launch_bounds__(64 * VM * VN) __attribute__((amdgpu_waves_per_eu(WPE, WPE))) void gemm_gguf(const uint16_t* __restrict__ X, const uint8_t* __restrict__ W,
                                                          const uint16_t* __restrict__ bias, uint16_t* __restrict__ Y,
                                                          int M, int N, int K) {
    constexpr int NT = 64 * VM * VN;
    constexpr int BM = VM * WM * 32, BN = VN * WN * 32;
    static_assert(BN * 2 == NT, "two threads per weight row");
    constexpr int TS = GGUFTs<QT>::TS;
    constexpr int ACH = BM * 8 / NT;                   // 16-byte activation chunks per thread per stage
    __shared__ uint4 lds[(BM + BN) * 8];
    const int ntm = (M + BM - 1) / BM, ntn = (N + BN - 1) / BN;
    int tm, tn;
    tile_order(blockIdx.x, ntm * ntn, ntm, ntn, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / VN, wn = wave % VN;
    const int nk = K / 64;
    const int sbs_per_row = K / 256;
    const int wr = tid >> 1, wh = tid & 1;             // this thread's weight row in the tile, and its half
    const bool wlive = n0 + wr < N;
    const uint8_t* wrow_p = W + (int64_t)(wlive ? n0 + wr : 0) * sbs_per_row * TS;
    const __amdgpu_buffer_rsrc_t xr = rows_rsrc(X + (int64_t)m0 * K, (int64_t)(M - m0) * K * 2);

    uint32_t xoff[ACH];
    int xslot[ACH];
#pragma unroll
    for (int i = 0; i < ACH; i++) {
        const int idx = tid + NT * i, r = idx >> 3, c = idx & 7;
        xoff[i] = (uint32_t)(r * K + 8 * c) * 2u;
        xslot[i] = r * 8 + swz8(r, c);
    }
    uint4 ra[ACH];
    HalfRaw<QT> rw;
    auto gload = [&](int kt) {
        const uint32_t k0 = (uint32_t)kt * 128u;       // bytes of bf16
#pragma unroll
        for (int i = 0; i < ACH; i++)
            ra[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xr, xoff[i] + k0, 0, 0));
        if (wlive) half_load<QT>(wrow_p + (kt >> 2) * TS, kt & 3, wh, rw);
    };
    auto lstore = [&](int kt) {
#pragma unroll
        for (int i = 0; i < ACH; i++) lds[xslot[i]] = ra[i];
        uint32_t o[16];
        if (wlive) {
            half_dequant<QT, MID>(rw, kt & 3, wh, o);
        } else {
#pragma unroll
            for (int i = 0; i < 16; i++) o[i] = 0;
        }
        uint4* sb = lds + BM * 8 + wr * 8;
#pragma unroll
        for (int c = 0; c < 4; c++)
            sb[swz8(wr, 4 * wh + c)] = make_uint4(o[4 * c], o[4 * c + 1], o[4 * c + 2], o[4 * c + 3]);
    };
    const int lr = lane & 31, lk = lane >> 5;
    int arow[WM], brow[WN];
#pragma unroll
    for (int i = 0; i < WM; i++) arow[i] = wm * WM * 32 + i * 32 + lr;
#pragma unroll
    for (int j = 0; j < WN; j++) brow[j] = wn * WN * 32 + j * 32 + lr;
    bf16x8 fa[2][WM], fb[2][WN];
    auto fread = [&](int ks, int set) {
        const int ch = 2 * ks + lk;
        const uint4* sa = lds;
        const uint4* sb = lds + BM * 8;
#pragma unroll
        for (int i = 0; i < WM; i++) fa[set][i] = __builtin_bit_cast(bf16x8, sa[arow[i] * 8 + swz8(arow[i], ch)]);
#pragma unroll
        for (int j = 0; j < WN; j++) fb[set][j] = __builtin_bit_cast(bf16x8, sb[brow[j] * 8 + swz8(brow[j], ch)]);
    };

    f32x16 acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

    gload(0);
    lstore(0);
    __syncthreads();
    fread(0, 0);
    for (int kt = 0; kt < nk; kt++) {
        const bool more = kt + 1 < nk;
        if (more) gload(kt + 1);
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const int set = ks & 1;
            if (ks < 3) fread(ks + 1, set ^ 1);
#pragma unroll
            for (int i = 0; i < WM; i++)
#pragma unroll
                for (int j = 0; j < WN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[set][i], fb[set][j], acc[i][j], 0, 0, 0);
        }
        if (more) {
            __syncthreads();          // every wave is done reading this stage
            lstore(kt + 1);
            __syncthreads();
            fread(0, 0);
        }
    }

#pragma unroll
    for (int j = 0; j < WN; j++) {
        const int n = n0 + wn * WN * 32 + j * 32 + lr;
        if (n >= N) continue;
        const float bn = BIAS ? __uint_as_float((uint32_t)bias[n] << 16) : 0.0f;
#pragma unroll
        for (int i = 0; i < WM; i++) {
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int m = m0 + wm * WM * 32 + i * 32 + 8 * (e >> 2) + 4 * lk + (e & 3);
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
    // 4 waves (2 x 2) of 4 x 2 tiles: a 256 x 128 tile, two workgroups per CU
    const int tiles = ((M + 255) / 256) * ((N + 127) / 128);
    if (bias) gemm_gguf<2, 2, 4, 2, QT, MID, true, 2><<<dim3(tiles), 256, 0, s>>>(X, W, bias, Y, M, N, K);
    else gemm_gguf<2, 2, 4, 2, QT, MID, false, 2><<<dim3(tiles), 256, 0, s>>>(X, W, bias, Y, M, N, K);
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
