/*
 * ORACLE -- test infrastructure only.
 *
 * Scalar CPU restatement of the arithmetic of WeightFerry's quantized-weight hot path. Only the tests, the smoke
 * check and the CPU-baseline leg of the benchmark load this file (as a shared library); the product never does.
 *
 * Every function cites the reference lines it restates (paths relative to the reference checkout):
 *   - rounding helpers            enhancers/gguf_dequant.py:72-96
 *   - legacy 32-value blocks      enhancers/gguf_dequant.py:52-54,136-167
 *   - K-quant 256-value blocks    enhancers/gguf_dequant.py:56,170-256
 *   - LoRA add (_deq_add)         enhancers/gguf_dequant.py:99-133,387-409
 *   - int8 row quantiser          enhancers/fused_kernels.py:44-49,65-81,137-174
 *   - quantiser operations (PRE)  enhancers/fused_kernels.py:14-18,84-136,143-163; enhancers/fused_int8.py:28-39,94-105
 *   - int8 linear epilogue        enhancers/fused_int8.py:191-206 (the epilogue order is defined here)
 *
 * Build: gcc -O2 -fPIC -shared -ffp-contract=off -fno-fast-math (see oracle/Makefile). No FMA contraction: every
 * product and sum is rounded on its own, as the reference's kernels launched with enable_fp_fusion=False.
 *
 * Dtype codes (enhancers/gguf_dequant.py:58): 0 float16, 1 bfloat16, 2 float32.
 * GGML type ids (enhancers/gguf_dequant.py:52-56): 2 Q4_0, 3 Q4_1, 6 Q5_0, 7 Q5_1, 8 Q8_0,
 *                                                  10 Q2_K, 11 Q3_K, 12 Q4_K, 13 Q5_K, 14 Q6_K.
 */
#include <stdint.h>
#include <string.h>
#include <math.h>

static inline uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* IEEE-754 binary32 -> binary16, round to nearest, ties to even (textbook; subnormals and overflow to inf
 * included). NaN keeps its sign and top payload bits and is made quiet. */
uint16_t wfo_f32_to_f16_bits(float x) {
    uint32_t u = f2u(x);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) {                       /* inf / nan */
        if (a == 0x7f800000u) return sign | 0x7c00u;
        return sign | 0x7c00u | 0x0200u | (uint16_t)((a >> 13) & 0x3ffu);
    }
    int32_t fexp = (int32_t)(a >> 23);            /* biased binary32 exponent */
    if (fexp == 0) return sign;                   /* binary32 subnormal: far below half of 2^-24 */
    uint32_t mant = (a & 0x7fffffu) | 0x800000u;  /* 24-bit significand */
    int32_t e = fexp - 127 + 15;                  /* biased binary16 exponent */
    if (e >= 31) return sign | 0x7c00u;           /* >= 2^16: overflow */
    if (e >= 1) {                                 /* normal binary16 candidate */
        uint32_t h = ((uint32_t)e << 10) | ((mant >> 13) & 0x3ffu);
        uint32_t rb = mant & 0x1fffu;
        if (rb > 0x1000u || (rb == 0x1000u && (h & 1u))) h += 1u;   /* carry may reach inf: correct */
        return sign | (uint16_t)h;
    }
    /* binary16 subnormal: value / 2^-24 = mant * 2^(e - 1 - 13) -> shift right by 14 - e */
    int32_t shift = 14 - e;
    if (shift > 24) return sign;                  /* below 2^-25: rounds to zero */
    uint32_t h = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) h += 1u;
    return sign | (uint16_t)h;
}

/* binary16 bits -> binary32 (exact) */
float wfo_f16_bits_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0x1f) return u2f(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        if (m == 0) return u2f(sign);
        /* subnormal: m * 2^-24 (exact in binary32) */
        float v = (float)m * u2f(0x33800000u);    /* 2^-24 */
        return sign ? -v : v;
    }
    return u2f(sign | ((e - 15 + 127) << 23) | (m << 13));
}

/* the bf16 rounding of the reference: (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000 on the bits
 * (enhancers/gguf_dequant.py:78-81; enhancers/fused_kernels.py:44-49) */
static inline uint32_t bf16_trick(uint32_t u) { return (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u; }

/* _round(x, D) of enhancers/gguf_dequant.py:72-83: the nearest value of dtype D, kept as float32 */
float wfo_round(float x, int D) {
    if (D == 0) return wfo_f16_bits_to_f32(wfo_f32_to_f16_bits(x));
    if (D == 1) return u2f(bf16_trick(f2u(x)));
    return x;
}

/* store of an already-rounded value in dtype D at element i of dst */
static inline void store_dt(void* dst, int64_t i, float x, int D) {
    if (D == 0) ((uint16_t*)dst)[i] = wfo_f32_to_f16_bits(x);
    else if (D == 1) ((uint16_t*)dst)[i] = (uint16_t)(bf16_trick(f2u(x)) >> 16);
    else ((float*)dst)[i] = x;
}

/* _f16 of enhancers/gguf_dequant.py:86-90: little-endian float16 at byte offset off */
static inline float ld_f16(const uint8_t* p) { return wfo_f16_bits_to_f32((uint16_t)(p[0] | (p[1] << 8))); }

/* legacy format table, enhancers/gguf_dequant.py:52-54: block bytes, has m, qh offset, qs offset, sub, int8 */
typedef struct { int ts, has_m, qh, qs, sub, is_q8; } legacy_fmt;
static int legacy(int q, legacy_fmt* f) {
    switch (q) {
    case 2: *f = (legacy_fmt){18, 0, -1, 2, 8, 0}; return 1;    /* Q4_0 */
    case 3: *f = (legacy_fmt){20, 1, -1, 4, 0, 0}; return 1;    /* Q4_1 */
    case 6: *f = (legacy_fmt){22, 0, 2, 6, 16, 0}; return 1;    /* Q5_0 */
    case 7: *f = (legacy_fmt){24, 1, 4, 8, 0, 0}; return 1;     /* Q5_1 */
    case 8: *f = (legacy_fmt){34, 0, -1, 2, 0, 1}; return 1;    /* Q8_0 */
    default: return 0;
    }
}

/* bytes per 256-value super-block, enhancers/gguf_dequant.py:56 */
int wfo_kquant_bytes(int q) {
    switch (q) { case 10: return 84; case 11: return 110; case 12: return 144; case 13: return 176;
                 case 14: return 210; default: return 0; }
}

/* one value of a legacy block: _deq, enhancers/gguf_dequant.py:136-167 */
static float deq_legacy(const uint8_t* b, const legacy_fmt* f, int v, int MID, int OUT) {
    float d = wfo_round(ld_f16(b), MID);
    float q;
    if (f->is_q8) {
        q = (float)(int8_t)b[f->qs + v];
    } else {
        int nib = (b[f->qs + (v % 16)] >> ((v / 16) * 4)) & 0xF;
        if (f->qh >= 0) nib |= ((b[f->qh + v / 8] >> (v % 8)) & 1) << 4;
        q = (float)(nib - f->sub);
    }
    float x = wfo_round(d * q, MID);
    if (f->has_m) x = wfo_round(x + wfo_round(ld_f16(b + 2), MID), MID);
    return wfo_round(x, OUT);
}

/* get_scale_min of sub-block sub (0..7) from the 12 scale bytes s: _sc / _mn, enhancers/gguf_dequant.py:170-185 */
void wfo_scale_min(const uint8_t* s, int sub, int* sc, int* m) {
    if (sub < 4) {
        *sc = s[sub] & 63;
        *m = s[sub + 4] & 63;
    } else {
        int j = sub - 4;
        *sc = (s[j + 8] & 0xF) | ((s[j] >> 2) & 0x30);
        *m = (s[j + 8] >> 4) | ((s[j + 4] >> 2) & 0x30);
    }
}

/* one value v (0..255) of a K-quant super-block b: _deq_k, enhancers/gguf_dequant.py:188-250 */
static float deq_k(const uint8_t* b, int fmt, int v, int MID, int OUT) {
    float x;
    if (fmt == 12 || fmt == 13) {                               /* :195-212 */
        int qs_off = fmt == 12 ? 16 : 48;
        int sub = v / 32;
        int q = (b[qs_off + (sub / 2) * 32 + v % 32] >> ((sub % 2) * 4)) & 0xF;
        if (fmt == 13) q |= ((b[16 + v % 32] >> sub) & 1) << 4;
        int sc, mn;
        wfo_scale_min(b + 4, sub, &sc, &mn);
        float d = wfo_round(ld_f16(b), MID);
        float dmin = wfo_round(ld_f16(b + 2), MID);
        float ds = wfo_round(d * (float)sc, MID);
        float dm = wfo_round(dmin * (float)mn, MID);
        x = wfo_round(wfo_round(ds * (float)q, MID) - dm, MID);
    } else if (fmt == 14) {                                     /* :213-224 */
        int h = v / 128, r = v % 128;
        int lo = (b[h * 64 + r % 64] >> ((r / 64) * 4)) & 0xF;
        int hi = (b[128 + h * 32 + r % 32] >> ((r / 32) * 2)) & 3;
        int q = (lo | (hi << 4)) - 32;
        float sc = (float)(int8_t)b[192 + v / 16];
        float d = wfo_round(wfo_round(ld_f16(b + 208), MID) * sc, MID);
        x = wfo_round(d * (float)q, MID);
    } else if (fmt == 11) {                                     /* :225-240 */
        int i = v / 16;
        int ls = (b[96 + i % 8] >> ((i / 8) * 4)) & 0xF;
        int hs = (b[104 + i % 4] >> ((i / 4) * 2)) & 3;
        int sc = (ls | (hs << 4)) - 32;
        float d = wfo_round(wfo_round(ld_f16(b + 108), MID) * (float)sc, MID);
        int r = v % 128;
        int ql = (b[32 + (v / 128) * 32 + r % 32] >> ((r / 32) * 2)) & 3;
        int hb = ((b[v % 32] >> (v / 32)) & 1) ^ 1;
        int q = ql - (hb << 2);
        x = wfo_round(d * (float)q, MID);
    } else {                                                    /* Q2_K :241-249 */
        int sb = b[v / 16];
        float dl = wfo_round(wfo_round(ld_f16(b + 80), MID) * (float)(sb & 0xF), MID);
        float ml = wfo_round(wfo_round(ld_f16(b + 82), MID) * (float)(sb >> 4), MID);
        int r = v % 128;
        int q = (b[16 + (v / 128) * 32 + r % 32] >> ((r / 32) * 2)) & 3;
        x = wfo_round(wfo_round(dl * (float)q, MID) - ml, MID);
    }
    return wfo_round(x, OUT);                                   /* :250 */
}

/* dequantize(data, qtype, oshape, mid, out) of enhancers/gguf_dequant.py:277-326 on a flat weight of n values.
 * Returns 0, or -1 when the byte count does not match n (the reference returns None there). */
int wfo_dequant(const uint8_t* src, int64_t nbytes, int qtype, int MID, int OUT, void* dst, int64_t n) {
    legacy_fmt f;
    if (MID < 0 || MID > 2 || OUT < 0 || OUT > 2) return -1;
    if (legacy(qtype, &f)) {
        if (nbytes % f.ts || (nbytes / f.ts) * 32 != n) return -1;
        for (int64_t blk = 0; blk < n / 32; blk++)
            for (int v = 0; v < 32; v++)
                store_dt(dst, blk * 32 + v, deq_legacy(src + blk * f.ts, &f, v, MID, OUT), OUT);
        return 0;
    }
    int ts = wfo_kquant_bytes(qtype);
    if (!ts || nbytes % ts || (nbytes / ts) * 256 != n) return -1;
    for (int64_t blk = 0; blk < n / 256; blk++)
        for (int v = 0; v < 256; v++)
            store_dt(dst, blk * 256 + v, deq_k(src + blk * ts, qtype, v, MID, OUT), OUT);
    return 0;
}

/* ---------------------------------------------------------------------------------------------- LoRA add */

/* value i of dtype D at dst, widened exactly to float32 */
static inline float load_dt(const void* dst, int64_t i, int D) {
    if (D == 0) return wfo_f16_bits_to_f32(((const uint16_t*)dst)[i]);
    if (D == 1) return u2f((uint32_t)((const uint16_t*)dst)[i] << 16);
    return ((const float*)dst)[i];
}

/* _deq_add of enhancers/gguf_dequant.py:99-133 on a flat weight of n values, as _add_loras launches it (:387-409):
 * w = the dequantised value (the chain of wfo_dequant, rounded to OUT) when src is not NULL (DEQ), else the OUT
 * value already in dst; then dst = R_OUT(w + R_OUT(diff * sa)) -- the product, its rounding, the sum and its
 * rounding each on their own (:127). Returns 0, or -1 when the blocks do not hold n values. */
int wfo_dequant_add(const uint8_t* src, int64_t nbytes, int qtype, int MID, int OUT, const float* diff, float sa,
                    void* dst, int64_t n) {
    if (OUT < 0 || OUT > 2) return -1;
    if (src && wfo_dequant(src, nbytes, qtype, MID, OUT, dst, n)) return -1;
    for (int64_t i = 0; i < n; i++) {
        const float w = load_dt(dst, i, OUT);
        const float p = diff[i] * sa;
        store_dt(dst, i, wfo_round(w + wfo_round(p, OUT), OUT), OUT);
    }
    return 0;
}

/* ---------------------------------------------------------------------------------------------- int8 quantiser */

/* one radix-4 stage of stride S on a 256-group: (a, b, c, d) -> (a+b+c-d, a+b-c+d, a-b+c+d, -a+b+c+d), each sum
 * left to right (enhancers/fused_kernels.py:65-81) */
static void h4_stage(float* y, int S) {
    for (int blk = 0; blk < 256; blk += 4 * S)
        for (int s = 0; s < S; s++) {
            float a = y[blk + s], b = y[blk + S + s], c = y[blk + 2 * S + s], d = y[blk + 3 * S + s];
            y[blk + s] = ((a + b) + c) - d;
            y[blk + S + s] = ((a + b) - c) + d;
            y[blk + 2 * S + s] = ((a - b) + c) + d;
            y[blk + 3 * S + s] = ((-a + b) + c) + d;
        }
}

/* per-row int8 quantisation, _quant_row with PRE_NONE (enhancers/fused_kernels.py:137-174).
 * mode 1: ConvRot (256-groups, stages of stride 1, 4, 16, 64, then * 0.0625); mode 0: plain per-token (no
 * rotation). x: bf16 bits [M, K]; xq: int8 [M, K]; xs: float32 [M]. IEEE division (the reference relies on
 * Triton's default division on its GPU; see the header of the build's design notes). */
int wfo_quant_rows(const uint16_t* x, int64_t M, int64_t K, int mode, int8_t* xq, float* xs, float* work) {
    if (mode == 1 && K % 256) return -1;
    for (int64_t r = 0; r < M; r++) {
        float* y = work;
        for (int64_t k = 0; k < K; k++) y[k] = u2f((uint32_t)x[r * K + k] << 16);
        if (mode == 1) {
            for (int64_t g = 0; g < K; g += 256) {
                h4_stage(y + g, 1); h4_stage(y + g, 4); h4_stage(y + g, 16); h4_stage(y + g, 64);
            }
            for (int64_t k = 0; k < K; k++) y[k] = y[k] * 0.0625f;
        }
        float amax = 0.0f;
        for (int64_t k = 0; k < K; k++) { float a = fabsf(y[k]); if (a > amax) amax = a; }
        amax = fminf(amax, 3.38953139e38f);
        float scale = fmaxf(amax / 127.0f, 1.0e-30f);
        xs[r] = scale;
        float sb = wfo_round(scale, 1);
        for (int64_t k = 0; k < K; k++) {
            float v = rintf(wfo_round(wfo_round(y[k], 1) / sb, 1));
            v = fminf(fmaxf(v, -128.0f), 127.0f);
            xq[r * K + k] = (int8_t)v;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------------------------------ int8 linear */

/* out[m, n] = R_OUT((f32(acc[m, n]) * xs[m]) * ws[n] (+ bias[n])), acc = sum_k xq[m, k] * wq[n, k] exactly in
 * int32 (the role of kitchen's cutlass_int8_dequant, enhancers/fused_int8.py:191-206; the epilogue order is this
 * build's definition). bias: optional, in the output dtype. */
int wfo_linear_i8(const int8_t* xq, const int8_t* wq, const float* xs, const float* ws, const void* bias,
                  void* out, int OUT, int64_t M, int64_t N, int64_t K, int32_t* acc_out) {
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            int64_t acc = 0;
            const int8_t* a = xq + m * K;
            const int8_t* b = wq + n * K;
            for (int64_t k = 0; k < K; k++) acc += (int32_t)a[k] * (int32_t)b[k];
            if (acc > INT32_MAX || acc < INT32_MIN) return -2;
            if (acc_out) acc_out[m * N + n] = (int32_t)acc;
            float t = ((float)(int32_t)acc * xs[m]) * ws[n];
            if (bias) {
                float bv = OUT == 2 ? ((const float*)bias)[n]
                         : OUT == 1 ? u2f((uint32_t)((const uint16_t*)bias)[n] << 16)
                                    : wfo_f16_bits_to_f32(((const uint16_t*)bias)[n]);
                t = t + bv;
            }
            store_dt(out, m * N + n, wfo_round(t, OUT), OUT);
        }
    return 0;
}

/* out = bf16(f32(resid) + f32(gate) * bf16((f32(acc) * xs[m]) * ws[n])): the plain linear's bf16 output, then
 * torch.addcmul(resid, gate, out) on bf16 tensors (the product of two bf16 values is exact in float32; the sum is
 * rounded once to float32). The role of kitchen's cutlass_int8_dequant_residual, whose bits the reference states
 * equal that addcmul (enhancers/fused_int8.py:212-268; enhancers/fused_block.py:24-26); gate [groups, N], row m in
 * group m / rows_per_group. bf16 operands only. */
int wfo_linear_i8_residual(const int8_t* xq, const int8_t* wq, const float* xs, const float* ws,
                           const uint16_t* gate, const uint16_t* resid, uint16_t* out,
                           int64_t M, int64_t N, int64_t K, int64_t rows_per_group) {
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++) {
            int64_t acc = 0;
            for (int64_t k = 0; k < K; k++) acc += (int32_t)xq[m * K + k] * (int32_t)wq[n * K + k];
            float t = ((float)(int32_t)acc * xs[m]) * ws[n];
            float g = u2f((uint32_t)gate[(m / rows_per_group) * N + n] << 16);
            float rv = u2f((uint32_t)resid[m * N + n] << 16);
            float o = rv + g * u2f(bf16_trick(f2u(t)));     /* addcmul on the bf16 GEMM output */
            out[m * N + n] = (uint16_t)(bf16_trick(f2u(o)) >> 16);
        }
    return 0;
}

/* ------------------------------------------------------------------------------------------- array helpers */

/* n float32 values -> their binary16 bits (textbook RNE above), for exhaustive checks over bit patterns */
/* ----------------------------------------------------------------------------------- quantiser operations */

/* cuWelfordCombine(dataB = own, dataA = other) as the reference restates it, contractions explicit
 * (enhancers/fused_kernels.py:84-94) */
static void wcombine(float* m, float* s, float* c, float mo, float so, float co) {
    const float delta = *m - mo;
    const float count = co + *c;
    const float coef = 1.0f / count;
    const float na = co * coef, nb = *c * coef;
    const float mean = fmaf(na, mo, nb * *m);
    const float sig = fmaf((delta * delta) * co, nb, so + *s);
    *m = mean; *s = sig; *c = count;
}

/* _ln_stats of enhancers/fused_kernels.py:108-136 on one bf16 row of K values (K % 512 == 0): 128 threads, thread t
 * updating (mean, sigma2, count) over values (t + 128 j) * 4 + ii, j-major; then the shuffle-down merges of [4, 32]
 * (N = 32 .. 2) and of the 4 warps (2, 3 into 0, 1; 1 into 0). Returns mean and sigma2 / K. */
void wfo_ln_stats(const uint16_t* xr, int64_t K, float* mu, float* var) {
    float m[128], sg[128], c[128];
    for (int t = 0; t < 128; t++) {
        m[t] = 0.0f; sg[t] = 0.0f; c[t] = 0.0f;
        for (int64_t j = 0; j < K / 512; j++)
            for (int ii = 0; ii < 4; ii++) {
                const float v = u2f((uint32_t)xr[(t + j * 128) * 4 + ii] << 16);
                const float delta = v - m[t];
                c[t] = c[t] + 1.0f;
                m[t] = fmaf(delta, 1.0f / c[t], m[t]);
                sg[t] = fmaf(delta, v - m[t], sg[t]);
            }
    }
    for (int N = 32; N >= 2; N /= 2)
        for (int w = 0; w < 4; w++)
            for (int t = 0; t < N / 2; t++) {
                const int a = 32 * w + t, b = 32 * w + t + N / 2;
                wcombine(&m[a], &sg[a], &c[a], m[b], sg[b], c[b]);
            }
    wcombine(&m[0], &sg[0], &c[0], m[64], sg[64], c[64]);      /* warp 2 into warp 0 */
    wcombine(&m[32], &sg[32], &c[32], m[96], sg[96], c[96]);   /* warp 3 into warp 1 */
    wcombine(&m[0], &sg[0], &c[0], m[32], sg[32], c[32]);      /* warp 1 into warp 0 */
    *mu = m[0];
    *var = sg[0] / (float)K;
}

/* _quant_row with an operation before the rotation (enhancers/fused_kernels.py:137-174), ConvRot mode:
 * pre 0 none; 1 GELU: y = table[bits(x)] (table: bf16 bits [65536]); 2 MOD: y = R16(R16(x * s1[g]) + h[g]);
 * 3 LNMOD: y = R16((x - mu) * rstd), then MOD; g = row / rows_per_group, s1 and h bf16 [groups, K].
 * rstd = RN(1 / sqrt(var + eps)) (the reference's rsqrt.approx.f32 is an NVIDIA approximation). */
int wfo_quant_rows_pre(const uint16_t* x, int64_t M, int64_t K, int pre, const uint16_t* s, const uint16_t* h,
                       int64_t rows_per_group, float eps, int8_t* xq, float* xs, float* work, uint16_t* rowbuf) {
    if (K % 256 || pre < 0 || pre > 3 || (pre == 3 && K % 512)) return -1;
    if (pre >= 2 && (rows_per_group <= 0 || M % rows_per_group)) return -1;
    for (int64_t r = 0; r < M; r++) {
        const uint16_t* xr = x + r * K;
        float mu = 0.0f, rstd = 0.0f;
        if (pre == 3) {
            float var;
            wfo_ln_stats(xr, K, &mu, &var);
            rstd = (float)(1.0 / sqrt((double)(var + eps)));
        }
        const int64_t g = pre >= 2 ? r / rows_per_group : 0;
        for (int64_t k = 0; k < K; k++) {
            float v = u2f((uint32_t)xr[k] << 16);
            if (pre == 1) {
                v = u2f((uint32_t)s[xr[k]] << 16);
            } else if (pre >= 2) {
                if (pre == 3) v = wfo_round((v - mu) * rstd, 1);
                const float sc = u2f((uint32_t)s[g * K + k] << 16), sh = u2f((uint32_t)h[g * K + k] << 16);
                v = wfo_round(wfo_round(v * sc, 1) + sh, 1);
            }
            rowbuf[k] = (uint16_t)(f2u(v) >> 16);      /* every value here is a bf16 value */
        }
        if (wfo_quant_rows(rowbuf, 1, K, 1, xq + r * K, xs + r, work)) return -1;
    }
    return 0;
}

void wfo_f32_to_f16_array(const float* x, uint16_t* h, int64_t n) {
    for (int64_t i = 0; i < n; i++) h[i] = wfo_f32_to_f16_bits(x[i]);
}

/* n float32 values -> _round(x, D) as float32 */
void wfo_round_array(const float* x, float* y, int64_t n, int D) {
    for (int64_t i = 0; i < n; i++) y[i] = wfo_round(x[i], D);
}
