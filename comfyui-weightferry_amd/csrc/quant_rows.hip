// Per-row int8 quantisation of bf16 activations for gfx950: the role of the Triton `_quant_row` with PRE_NONE
// (enhancers/fused_kernels.py:137-174) and of kitchen's quantize_int8_rowwise_convrot64 (enhancers/fused_int8.py:
// 178-181).
//
// Per row r of K values x (bf16):
//   mode 1 (ConvRot): each 256-group goes through four radix-4 stages of stride 1, 4, 16, 64 -- (a, b, c, d) ->
//     (a+b+c-d, a+b-c+d, a-b+c+d, -a+b+c+d), every sum left to right in float32 -- then * 0.0625;
//   mode 0 (plain per-token): y = x.
//   amax = min(max |y|, 3.38953139e38); scale = max(amax / 127, 1e-30) (stored as float32);
//   q = clamp(rint(bf16(bf16(y) / bf16(scale))), -128, 127).
//
// A row is held in registers by one wave (rows up to 6144 values in ConvRot mode, 8192 plain; four rows per
// 256-thread workgroup) or by the four waves of a workgroup (wider rows, up to 32768 values; the waves' partial
// maxima meet in LDS -- the maximum does not depend on the order it is taken in, so the bits do not depend on the
// split). ConvRot: a lane loads 16 consecutive values of a 256-group (the two lowest radix-4 digits), runs stages 1
// and 4 on them, exchanges through LDS so that it then holds the 16 values that share its two lowest digits
// (stride 16), and runs stages 16 and 64. Groups are independent until the row maximum, so a wave may take any of
// them: pass p of wave w of a row takes groups 4 (p W + w) .. 4 (p W + w) + 3, W waves per row. The quotient y / s is computed with a
// correctly rounded reciprocal of s (one IEEE division per row) and one Markstein correction step -- mul, then two
// fma -- which is the correctly rounded IEEE quotient for every normal result (subnormal quotients round to 0 in the
// integer anyway). Built without contraction; the fma calls are explicit.
//
// ConvRot rows may first go through the operation the reference's quantiser applies before its rotation (PRE,
// enhancers/fused_kernels.py:14-18,143-163): GELU by table lookup (torch's GELU of every bf16 value), the
// scale-and-shift bf16(bf16(x * s1) + shift) of the row's group, or LayerNorm without affine, rounded to bf16, and
// then the scale-and-shift. The LayerNorm statistics follow the reference's Welford order (:97-136): 128 virtual
// threads, thread t updating (mean, sigma2, count) over the 4-value vectors t, t + 128, ... of the row, then
// shuffle-down merges within 32-thread warps (16, 8, 4, 2, 1) and across warps (2, 3 into 0, 1; 1 into 0). Lane l
// of the wave plays virtual threads l and l + 64. rstd = 1 / sqrt(var + eps) correctly rounded (the reference's
// rsqrt.approx.f32 is an NVIDIA approximation).

#include "wf_common.h"

namespace wf {

constexpr float kAmaxClamp = 3.38953139e38f;

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b16) { return __uint_as_float(b16 << 16); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// RN(y / s) for the row's finite scale s, given rs = RN(1 / s). An infinite y (a rotation that overflowed)
// gives y * rs = +-inf, which is the IEEE quotient; the correction step would turn it into NaN (inf - inf).
__device__ __forceinline__ float div_rn(float y, float s, float rs) {
    const float q = y * rs;
    const float rem = __builtin_fmaf(-q, s, y);
    const float r = __builtin_fmaf(rem, rs, q);
    return __builtin_isinf(q) ? q : r;
}

__device__ __forceinline__ int8_t quant1(float y, float sb, float rsb) {
    float v = __builtin_rintf(round_bf16(div_rn(round_bf16(y), sb, rsb)));
    v = fminf(fmaxf(v, -128.0f), 127.0f);
    return (int8_t)(int)v;
}

// the row's maximum over its W waves (W = 1: the wave's own); every lane of the W waves gets it. W > 1 needs the
// whole workgroup to be one row (no wave leaves early), since it takes a workgroup barrier.
template <int W>
__device__ __forceinline__ float row_max(float wave_amax, int wave) {
    if constexpr (W == 1) {
        return wave_amax;
    } else {
        __shared__ float part[W];
        if ((threadIdx.x & 63) == 0) part[wave] = wave_amax;
        __syncthreads();
        float m = part[0];
#pragma unroll
        for (int i = 1; i < W; i++) m = fmaxf(m, part[i]);
        return m;
    }
}

struct RowScale {
    float scale, sb, rsb;
};

__device__ __forceinline__ RowScale row_scale(float amax) {
    RowScale r;
    amax = fminf(amax, kAmaxClamp);
    r.scale = fmaxf(amax / 127.0f, 1.0e-30f);
    r.sb = round_bf16(r.scale);
    r.rsb = 1.0f / r.sb;
    return r;
}

// ----------------------------------------------------------------------------------------- operations (PRE)
struct PreArgs {
    const uint16_t* s;        // GELU: bf16 table [65536]; MOD / LNMOD: bf16 s1 = 1 + scale, [groups, K]
    const uint16_t* h;        // MOD / LNMOD: bf16 shift, [groups, K]
    int64_t rows_per_group;
    float eps;                // LNMOD
};

// PyTorch's cuWelfordCombine(dataB = own, dataA = other) as the reference restates it, with the contractions it
// makes explicit (enhancers/fused_kernels.py:84-94)
__device__ __forceinline__ void wcombine(float& m, float& s, float& c, float mo, float so, float co) {
    const float delta = m - mo;
    const float count = co + c;
    const float coef = 1.0f / count;
    const float na = co * coef, nb = c * coef;
    const float mean = __builtin_fmaf(na, mo, nb * m);
    const float sig = __builtin_fmaf((delta * delta) * co, nb, so + s);
    m = mean; s = sig; c = count;
}

// mean and sigma2 / K of one row (K % 512 == 0), every lane gets the result
__device__ __forceinline__ void ln_stats(const uint16_t* xr, int K, int lane, float& mu, float& var) {
    float m[2] = {0.0f, 0.0f}, sg[2] = {0.0f, 0.0f}, c[2] = {0.0f, 0.0f};
    for (int j = 0; j < (K >> 9); j++) {
#pragma unroll
        for (int vt = 0; vt < 2; vt++) {
            const int t = lane + 64 * vt;
            const uint2 w = *reinterpret_cast<const uint2*>(xr + 4 * (t + 128 * j));
            const float v4[4] = {bf16_bits_to_f32(w.x & 0xffffu), bf16_bits_to_f32(w.x >> 16),
                                 bf16_bits_to_f32(w.y & 0xffffu), bf16_bits_to_f32(w.y >> 16)};
#pragma unroll
            for (int ii = 0; ii < 4; ii++) {
                const float delta = v4[ii] - m[vt];
                c[vt] = c[vt] + 1.0f;
                m[vt] = __builtin_fmaf(delta, 1.0f / c[vt], m[vt]);
                sg[vt] = __builtin_fmaf(delta, v4[ii] - m[vt], sg[vt]);
            }
        }
    }
    // within each 32-thread virtual warp: lane i < o merges lane i + o
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) {
#pragma unroll
        for (int vt = 0; vt < 2; vt++) {
            const float mo = __shfl_down(m[vt], o, 32), so = __shfl_down(sg[vt], o, 32), co = __shfl_down(c[vt], o, 32);
            if ((lane & 31) < o) wcombine(m[vt], sg[vt], c[vt], mo, so, co);
        }
    }
    // warps 2, 3 (lanes 0, 32 of the second virtual thread) into warps 0, 1; then warp 1 (lane 32) into warp 0
    wcombine(m[0], sg[0], c[0], m[1], sg[1], c[1]);
    const float mo = __shfl(m[0], 32, 64), so = __shfl(sg[0], 32, 64), co = __shfl(c[0], 32, 64);
    wcombine(m[0], sg[0], c[0], mo, so, co);
    mu = __shfl(m[0], 0, 64);
    var = __shfl(sg[0], 0, 64) / (float)K;
}

// ------------------------------------------------------------------------------------------------ plain rows
// W waves per row, CPL chunks of 8 values per lane: chunk c = (i W + w) 64 + lane of the row for wave w, i < CPL.
// K <= 512 W CPL, K % 8 == 0. W = 1: four rows per workgroup; W = 4: one.
template <int CPL, int W>
__global__ __launch_bounds__(256) void quant_plain(const uint16_t* __restrict__ x, int64_t M, int K,
                                                   int8_t* __restrict__ xq, float* __restrict__ xs) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, w = wave % W;
    const int64_t row = (int64_t)blockIdx.x * (4 / W) + wave / W;
    if (W == 1 && row >= M) return;             // whole waves leave together; W = 1 takes no workgroup barrier
    const uint4* xr = reinterpret_cast<const uint4*>(x + row * K);
    const int nchunks = K >> 3;
    uint4 v[CPL];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; i++) {
        const int c = (i * W + w) * 64 + lane;
        v[i] = c < nchunks ? xr[c] : make_uint4(0, 0, 0, 0);
        const uint32_t u[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
        for (int h = 0; h < 4; h++) {
            amax = fmaxf(amax, fabsf(bf16_bits_to_f32(u[h] & 0xffffu)));
            amax = fmaxf(amax, fabsf(bf16_bits_to_f32(u[h] >> 16)));
        }
    }
    const RowScale rs = row_scale(row_max<W>(wave_max(amax), wave));
    if (lane == 0 && w == 0) xs[row] = rs.scale;
    uint2* qr = reinterpret_cast<uint2*>(xq + row * K);
#pragma unroll
    for (int i = 0; i < CPL; i++) {
        const int c = (i * W + w) * 64 + lane;
        if (c >= nchunks) continue;
        const uint32_t u[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
        uint32_t b[2] = {0, 0};
#pragma unroll
        for (int h = 0; h < 4; h++) {
            const uint32_t lo = (uint8_t)quant1(bf16_bits_to_f32(u[h] & 0xffffu), rs.sb, rs.rsb);
            const uint32_t hi = (uint8_t)quant1(bf16_bits_to_f32(u[h] >> 16), rs.sb, rs.rsb);
            b[h >> 1] |= (lo | (hi << 8)) << (16 * (h & 1));
        }
        qr[c] = make_uint2(b[0], b[1]);
    }
}

// --------------------------------------------------------------------------------------------- ConvRot rows
// radix-4 stage on 4 values (a, b, c, d) in place, sums left to right (enhancers/fused_kernels.py:65-81)
__device__ __forceinline__ void h4(float& a, float& b, float& c, float& d) {
    const float y0 = ((a + b) + c) - d;
    const float y1 = ((a + b) - c) + d;
    const float y2 = ((a - b) + c) + d;
    const float y3 = ((-a + b) + c) + d;
    a = y0; b = y1; c = y2; d = y3;
}

// LDS slot of element i (0..255) of group g of a wave's 4-group window: 17 floats per 16 elements (conflict-free
// for both the contiguous and the stride-16 access)
__device__ __forceinline__ int slot(int g, int i) { return g * 272 + i + (i >> 4); }

// W waves per row, NP passes of 4 groups (1024 values) per wave: K <= 1024 W NP, K % 256 == 0. Lane t of pass p
// of wave w owns group 4 (p W + w) + t / 16, position tl = t % 16. W = 1: four rows per workgroup; W = 4: one.
template <int NP, int PRE, int W>
__global__ __launch_bounds__(256) void quant_convrot(const uint16_t* __restrict__ x, int64_t M, int K,
                                                     int8_t* __restrict__ xq, float* __restrict__ xs, PreArgs pa) {
    __shared__ float stage[4][4 * 272];          // per wave: one 4-group window
    __shared__ uint32_t qbytes[4][256];          // per wave: the 1024 int8 values of one pass, 4 bytes a word
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, w = wave % W;
    const int64_t row = (int64_t)blockIdx.x * (4 / W) + wave / W;
    if (W == 1 && row >= M) return;              // whole waves leave together; W = 1 takes no workgroup barrier
    const int G = K >> 8;                        // groups in the row
    const int gl = lane >> 4, tl = lane & 15;
    float* st = stage[wave];
    float y[NP][16];
    float amax = 0.0f;
    float mu = 0.0f, rstd = 0.0f;
    const int64_t grp = PRE >= 2 ? row / pa.rows_per_group : 0;
    if constexpr (PRE == 3) {
        float var;
        ln_stats(x + row * K, K, lane, mu, var);
        rstd = (float)(1.0 / __builtin_sqrt((double)(var + pa.eps)));
    }
#pragma unroll
    for (int p = 0; p < NP; p++) {
        const int g = 4 * (p * W + w) + gl;
        const bool live = g < G;
        // 16 consecutive values [16 tl, 16 tl + 16) of group g: digits k0 (stride 1) and k1 (stride 4)
        float v[16];
        if (live) {
            const uint4* src = reinterpret_cast<const uint4*>(x + row * K + g * 256 + 16 * tl);
            const uint4 a = src[0], b = src[1];
            const uint32_t u[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int h = 0; h < 8; h++) {
                v[2 * h] = bf16_bits_to_f32(u[h] & 0xffffu);
                v[2 * h + 1] = bf16_bits_to_f32(u[h] >> 16);
            }
            if constexpr (PRE == 1) {
#pragma unroll
                for (int h = 0; h < 8; h++) {
                    v[2 * h] = bf16_bits_to_f32(pa.s[u[h] & 0xffffu]);
                    v[2 * h + 1] = bf16_bits_to_f32(pa.s[u[h] >> 16]);
                }
            } else if constexpr (PRE >= 2) {
                const int64_t o = grp * K + g * 256 + 16 * tl;
                const uint4* sp = reinterpret_cast<const uint4*>(pa.s + o);
                const uint4* hp = reinterpret_cast<const uint4*>(pa.h + o);
                const uint4 s0 = sp[0], s1 = sp[1], h0 = hp[0], h1 = hp[1];
                const uint32_t sw[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
                const uint32_t hw[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const float sc = bf16_bits_to_f32(i & 1 ? sw[i >> 1] >> 16 : sw[i >> 1] & 0xffffu);
                    const float sh = bf16_bits_to_f32(i & 1 ? hw[i >> 1] >> 16 : hw[i >> 1] & 0xffffu);
                    float t = v[i];
                    if constexpr (PRE == 3) t = round_bf16((t - mu) * rstd);
                    v[i] = round_bf16(round_bf16(t * sc) + sh);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < 16; i++) v[i] = 0.0f;
        }
#pragma unroll
        for (int q = 0; q < 4; q++) h4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);   // stride 1
#pragma unroll
        for (int q = 0; q < 4; q++) h4(v[q], v[q + 4], v[q + 8], v[q + 12]);                  // stride 4
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int i = 0; i < 16; i++) st[slot(gl, 16 * tl + i)] = v[i];
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_s_waitcnt(0);           // LDS writes of this wave done before the reads below
        __builtin_amdgcn_wave_barrier();
        // now the 16 values i = tl + 16 m (m = k2 + 4 k3) of group g
#pragma unroll
        for (int m = 0; m < 16; m++) v[m] = st[slot(gl, tl + 16 * m)];
#pragma unroll
        for (int q = 0; q < 4; q++) h4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);   // stride 16
#pragma unroll
        for (int q = 0; q < 4; q++) h4(v[q], v[q + 4], v[q + 8], v[q + 12]);                  // stride 64
#pragma unroll
        for (int m = 0; m < 16; m++) {
            y[p][m] = v[m] * 0.0625f;
            if (live) amax = fmaxf(amax, fabsf(y[p][m]));
        }
        __builtin_amdgcn_wave_barrier();
    }
    const RowScale rs = row_scale(row_max<W>(wave_max(amax), wave));
    if (lane == 0 && w == 0) xs[row] = rs.scale;
    // per pass: quantise into the wave's LDS words at the bytes' row positions, then store the pass's 1024 bytes
    // (four whole groups, contiguous in the row) with one 16-byte store per lane
    uint8_t* qb = reinterpret_cast<uint8_t*>(qbytes[wave]);
    const uint4* qs = reinterpret_cast<const uint4*>(qbytes[wave]);
    uint4* dst = reinterpret_cast<uint4*>(xq + row * K);
#pragma unroll
    for (int p = 0; p < NP; p++) {
        const int g0 = 4 * (p * W + w);
        if (g0 >= G) break;                      // the same for the whole wave
        if (g0 + gl < G) {
#pragma unroll
            for (int m = 0; m < 16; m++) qb[gl * 256 + tl + 16 * m] = (uint8_t)quant1(y[p][m], rs.sb, rs.rsb);
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_s_waitcnt(0);
        __builtin_amdgcn_wave_barrier();
        if (g0 + (lane >> 4) < G) dst[g0 * 16 + lane] = qs[lane];
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_s_waitcnt(0);           // the pass's LDS reads done before the next pass writes
        __builtin_amdgcn_wave_barrier();
    }
}

// widest rows taken: 32768 values (one workgroup of four waves per row)
constexpr int kMaxRowK = 32768;

template <int CPL, int W>
static void launch_plain(const uint16_t* x, int64_t M, int K, int8_t* xq, float* xs, hipStream_t s) {
    quant_plain<CPL, W><<<dim3((unsigned)((M + 4 / W - 1) / (4 / W))), 256, 0, s>>>(x, M, K, xq, xs);
}

static void launch_plain_rows(const uint16_t* x, int64_t M, int K, int8_t* xq, float* xs, hipStream_t s) {
    if (K <= 8192) {                                   // one wave per row
        const int cpl = (K + 511) / 512;
        if (cpl <= 2) launch_plain<2, 1>(x, M, K, xq, xs, s);
        else if (cpl <= 4) launch_plain<4, 1>(x, M, K, xq, xs, s);
        else if (cpl <= 8) launch_plain<8, 1>(x, M, K, xq, xs, s);
        else if (cpl <= 10) launch_plain<10, 1>(x, M, K, xq, xs, s);
        else launch_plain<16, 1>(x, M, K, xq, xs, s);
    } else {                                           // four waves per row: 2048 values per chunk step
        const int cpl = (K + 2047) / 2048;
        if (cpl <= 6) launch_plain<6, 4>(x, M, K, xq, xs, s);
        else if (cpl <= 8) launch_plain<8, 4>(x, M, K, xq, xs, s);
        else if (cpl <= 12) launch_plain<12, 4>(x, M, K, xq, xs, s);
        else launch_plain<16, 4>(x, M, K, xq, xs, s);
    }
}

template <int NP, int PRE, int W>
static void launch_convrot_pre(const uint16_t* x, int64_t M, int K, int8_t* xq, float* xs, const PreArgs& pa,
                               hipStream_t s) {
    quant_convrot<NP, PRE, W><<<dim3((unsigned)((M + 4 / W - 1) / (4 / W))), 256, 0, s>>>(x, M, K, xq, xs, pa);
}

template <int PRE>
static void launch_convrot(const uint16_t* x, int64_t M, int K, int8_t* xq, float* xs, const PreArgs& pa,
                           hipStream_t s) {
    if (K <= 6144) {                                   // one wave per row, 1024 values per pass
        const int np = (K + 1023) / 1024;
        if (np <= 1) launch_convrot_pre<1, PRE, 1>(x, M, K, xq, xs, pa, s);
        else if (np <= 2) launch_convrot_pre<2, PRE, 1>(x, M, K, xq, xs, pa, s);
        else if (np <= 3) launch_convrot_pre<3, PRE, 1>(x, M, K, xq, xs, pa, s);
        else if (np <= 4) launch_convrot_pre<4, PRE, 1>(x, M, K, xq, xs, pa, s);
        else if (np <= 5) launch_convrot_pre<5, PRE, 1>(x, M, K, xq, xs, pa, s);
        else launch_convrot_pre<6, PRE, 1>(x, M, K, xq, xs, pa, s);
    } else {                                           // four waves per row, 4096 values per pass
        const int np = (K + 4095) / 4096;
        if (np <= 2) launch_convrot_pre<2, PRE, 4>(x, M, K, xq, xs, pa, s);
        else if (np <= 3) launch_convrot_pre<3, PRE, 4>(x, M, K, xq, xs, pa, s);
        else if (np <= 4) launch_convrot_pre<4, PRE, 4>(x, M, K, xq, xs, pa, s);
        else if (np <= 5) launch_convrot_pre<5, PRE, 4>(x, M, K, xq, xs, pa, s);
        else if (np <= 6) launch_convrot_pre<6, PRE, 4>(x, M, K, xq, xs, pa, s);
        else launch_convrot_pre<8, PRE, 4>(x, M, K, xq, xs, pa, s);
    }
}

// the checks both entry points share
static int check_rows(const char* who, const void* x, int64_t M, int64_t K, const int8_t* xq, const float* xs) {
    if (M < 0 || K <= 0) { set_error("%s: M = %lld, K = %lld", who, (long long)M, (long long)K); return WF_EINVAL; }
    if (M == 0) return WF_OK;
    if (!x || !xq || !xs) { set_error("%s: null pointer", who); return WF_EINVAL; }
    if (!aligned(x, 16) || !aligned(xq, 16) || !aligned(xs, 4)) {
        set_error("%s: x and xq must be 16-byte aligned", who);
        return WF_EUNSUPPORTED;
    }
    if (M > ((int64_t)1 << 33)) { set_error("%s: M too large", who); return WF_EUNSUPPORTED; }
    return WF_OK;
}

}  // namespace wf

extern "C" int wf_quant_rows_i8(const void* x_bf16, int64_t M, int64_t K, int mode, int8_t* xq, float* xs,
                                void* stream) {
    using namespace wf;
    const int rc = check_rows("wf_quant_rows_i8", x_bf16, M, K, xq, xs);
    if (rc != WF_OK || M == 0) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint16_t* xp = static_cast<const uint16_t*>(x_bf16);
    const int k = (int)K;
    if (mode == 0) {
        if (K % 16 || K > kMaxRowK) {
            set_error("wf_quant_rows_i8: plain mode needs K %% 16 == 0 and K <= %d (K = %lld)", kMaxRowK,
                      (long long)K);
            return WF_EUNSUPPORTED;
        }
        launch_plain_rows(xp, M, k, xq, xs, s);
    } else if (mode == 1) {
        if (K % 256 || K > kMaxRowK) {
            set_error("wf_quant_rows_i8: ConvRot mode needs K %% 256 == 0 and K <= %d (K = %lld)", kMaxRowK,
                      (long long)K);
            return WF_EUNSUPPORTED;
        }
        launch_convrot<0>(xp, M, k, xq, xs, PreArgs{nullptr, nullptr, 1, 0.0f}, s);
    } else {
        set_error("wf_quant_rows_i8: mode %d", mode);
        return WF_EUNSUPPORTED;
    }
    WF_LAUNCH_CHECK("wf_quant_rows_i8 launch");
    return WF_OK;
}

extern "C" int wf_quant_rows_i8_pre(const void* x_bf16, int64_t M, int64_t K, int pre, const void* s_bf16,
                                    const void* shift_bf16, int64_t rows_per_group, float eps, int8_t* xq, float* xs,
                                    void* stream) {
    using namespace wf;
    const int rc = check_rows("wf_quant_rows_i8_pre", x_bf16, M, K, xq, xs);
    if (rc != WF_OK || M == 0) return rc;
    if (pre < 0 || pre > 3) { set_error("wf_quant_rows_i8_pre: operation %d", pre); return WF_EUNSUPPORTED; }
    if (K % 256 || K > kMaxRowK || (pre == 3 && K % 512)) {
        set_error("wf_quant_rows_i8_pre: K = %lld (K %% 256 == 0, K <= %d; LayerNorm K %% 512 == 0)", (long long)K,
                  kMaxRowK);
        return WF_EUNSUPPORTED;
    }
    if (pre >= 1 && !s_bf16) { set_error("wf_quant_rows_i8_pre: null pointer"); return WF_EINVAL; }
    if (pre >= 2) {
        if (!shift_bf16) { set_error("wf_quant_rows_i8_pre: null pointer"); return WF_EINVAL; }
        if (rows_per_group <= 0 || M % rows_per_group) {
            set_error("wf_quant_rows_i8_pre: M = %lld is not a whole number of %lld-row groups", (long long)M,
                      (long long)rows_per_group);
            return WF_EUNSUPPORTED;
        }
        if (!aligned(s_bf16, 16) || !aligned(shift_bf16, 16)) {
            set_error("wf_quant_rows_i8_pre: scale and shift must be 16-byte aligned");
            return WF_EUNSUPPORTED;
        }
    }
    if (pre == 1 && !aligned(s_bf16, 2)) { set_error("wf_quant_rows_i8_pre: table alignment"); return WF_EUNSUPPORTED; }
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint16_t* xp = static_cast<const uint16_t*>(x_bf16);
    const PreArgs pa{static_cast<const uint16_t*>(s_bf16), static_cast<const uint16_t*>(shift_bf16),
                     rows_per_group > 0 ? rows_per_group : 1, eps};
    const int k = (int)K;
    if (pre == 0) launch_convrot<0>(xp, M, k, xq, xs, pa, s);
    else if (pre == 1) launch_convrot<1>(xp, M, k, xq, xs, pa, s);
    else if (pre == 2) launch_convrot<2>(xp, M, k, xq, xs, pa, s);
    else launch_convrot<3>(xp, M, k, xq, xs, pa, s);
    WF_LAUNCH_CHECK("wf_quant_rows_i8_pre launch");
    return WF_OK;
}
