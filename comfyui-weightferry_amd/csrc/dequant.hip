// GGUF block dequantisation for gfx950: the role of the Triton kernels `_deq` / `_deq_k` of the reference
// (enhancers/gguf_dequant.py:136-256), with the same rounding chain -- every product and sum rounded to the dequant
// dtype MID, then the cast to OUT -- and no FMA contraction (built with -ffp-contract=off).
//
// Layout of the work: each lane owns whole 16-byte output chunks (8 values of a 2-byte OUT), so a wave's store is
// 1 KiB of contiguous output. K-quant super-blocks (256 values) are handled by 16 lanes; the 16-byte header of a
// Q4_K / Q5_K super-block (d, dmin, 12 scale bytes) is one 128-bit load per lane, the quants one 64-bit load.
// Q8_0 (34 B) and Q6_K (210 B) blocks are not dword-aligned: their quants are read as aligned dwords and shifted
// into place with v_alignbit (funnel8), every load inside the block's own bytes.
//
// MID = float16 runs on packed half math. That gives the reference's bits exactly: each product d*q, d*sc is
// exact in float32 (at most 11 + 8 significant bits), so rounding it to float16 is what v_pk_mul_f16 computes;
// each sum of two float16 values rounded to float32 and then to float16 equals the directly rounded sum, because
// float32 carries 24 >= 2 * 11 + 2 bits (double rounding is innocuous then). The quants enter as float16 through
// the exponent trick: the bits 0x6400 | b are the float16 1024 + b exactly for a byte b, and subtracting 1024 (or
// 1024 + bias) is exact.
//
// MID = bfloat16 / float32 run on float32 math with explicit rounding (round_to<MID>). No value on these paths is
// a float32 subnormal (every non-zero value is at least 2^-24 in magnitude), so the hardware's round-to-nearest-even
// conversions equal the reference's bit rule for every finite value.

#include "kquant.h"

// Launch shape of the streaming kernels: each thread handles DEQ_ITEMS lane-items with every load issued before any
// arithmetic; DEQ_NT_STORE writes the output with non-temporal stores (it is read by a later kernel, not this one).
// Measured on MI355X: 1 item per thread and non-temporal stores are the fastest (a persistent, grid-capped launch
// and more items per thread were slower).
#ifndef DEQ_ITEMS
#define DEQ_ITEMS 1
#endif
#ifndef DEQ_NT_STORE
#define DEQ_NT_STORE 1
#endif

namespace wf {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void st(uint4* p, const uint4& v) {
#if DEQ_NT_STORE
    u32x4 w = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(p));
#else
    *p = v;
#endif
}

// ------------------------------------------------------------------------------------------------- stores
template <int OUT>
__device__ __forceinline__ void store8(void* out, int64_t e0, const float (&v)[8]) {  // e0: element index
    if constexpr (OUT == WF_F32) {
        uint4* o = reinterpret_cast<uint4*>(static_cast<float*>(out) + e0);
        st(o, make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])));
        st(o + 1, make_uint4(__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]), __float_as_uint(v[7])));
    } else {
        uint4 r;
        if constexpr (OUT == WF_BF16) {
            r.x = pack_bf16(v[0], v[1]); r.y = pack_bf16(v[2], v[3]);
            r.z = pack_bf16(v[4], v[5]); r.w = pack_bf16(v[6], v[7]);
        } else {
            r.x = pack_f16(v[0], v[1]); r.y = pack_f16(v[2], v[3]);
            r.z = pack_f16(v[4], v[5]); r.w = pack_f16(v[6], v[7]);
        }
        st(reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + e0), r);
    }
}

// 8 float16 values (MID = f16) -> OUT
template <int OUT>
__device__ __forceinline__ void store8h(void* out, int64_t e0, const h2 (&v)[4]) {
    if constexpr (OUT == WF_F16) {
        uint4 r = {h2_bits(v[0]), h2_bits(v[1]), h2_bits(v[2]), h2_bits(v[3])};
        st(reinterpret_cast<uint4*>(static_cast<uint16_t*>(out) + e0), r);
    } else {
        float f[8];
#pragma unroll
        for (int i = 0; i < 4; i++) { f[2 * i] = (float)v[i][0]; f[2 * i + 1] = (float)v[i][1]; }
        store8<OUT>(out, e0, f);
    }
}

// Where a lane-item's 8 values (MID values held in float32, or float16 pairs for MID = f16) go. ToOut: cast to OUT
// and stored -- the dequantisation. AddDiff: the LoRA add of the reference's _deq_add (enhancers/gguf_dequant.py:
// 99-133) fused behind it: w = OUT(x), then out = OUT(w + OUT(diff * sa)), each product and sum rounded on its own.
struct ToOut {
    void* out;
    template <int OUT>
    __device__ __forceinline__ void put(int64_t e0, const float (&v)[8]) const { store8<OUT>(out, e0, v); }
    template <int OUT>
    __device__ __forceinline__ void puth(int64_t e0, const h2 (&v)[4]) const { store8h<OUT>(out, e0, v); }
};

template <int OUT>
__device__ __forceinline__ void add_scaled(float (&w)[8], const float* diff, float sa) {
    const float4 d0 = *reinterpret_cast<const float4*>(diff), d1 = *reinterpret_cast<const float4*>(diff + 4);
    const float d[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
#pragma unroll
    for (int i = 0; i < 8; i++) w[i] = round_to<OUT>(w[i] + round_to<OUT>(d[i] * sa));
}

struct AddDiff {
    void* out;
    const float* diff;
    float sa;
    template <int OUT>
    __device__ __forceinline__ void put(int64_t e0, const float (&v)[8]) const {
        float w[8];
#pragma unroll
        for (int i = 0; i < 8; i++) w[i] = round_to<OUT>(v[i]);
        add_scaled<OUT>(w, diff + e0, sa);
        store8<OUT>(out, e0, w);
    }
    template <int OUT>
    __device__ __forceinline__ void puth(int64_t e0, const h2 (&v)[4]) const {
        float f[8];
#pragma unroll
        for (int i = 0; i < 4; i++) { f[2 * i] = (float)v[i][0]; f[2 * i + 1] = (float)v[i][1]; }
        put<OUT>(e0, f);
    }
};

// Every fast kernel is a Format with load(src, t) -> Raw (only global loads) and emit(sink, t, Raw) (arithmetic and
// stores) for lane-item t of one workgroup's tile; the driver issues the loads of DEQ_ITEMS items before emitting
// any of them. A tile is DEQ_ITEMS * 256 lane-items = whole blocks, so the workgroup's block and output bases are
// scalar and each lane works with 32-bit offsets. The grid covers every lane-item (no loop).
template <typename F, bool ADD>
__global__ __launch_bounds__(256) void deq_items(const uint8_t* __restrict__ src, void* __restrict__ out,
                                                 int64_t nlanes, const float* __restrict__ diff, float sa) {
    constexpr int U = DEQ_ITEMS;
    constexpr int TILE_BLOCKS = U * 256 / F::LANES_PER_BLOCK;
    const int64_t t0 = (int64_t)blockIdx.x * (U * 256);
    const uint8_t* tsrc = src + (int64_t)blockIdx.x * TILE_BLOCKS * F::TS;
    const int64_t tval = (int64_t)blockIdx.x * TILE_BLOCKS * F::PER;     // first value of the tile
    void* tout = static_cast<char*>(out) + tval * F::OUT_BYTES;
    typename F::Raw r[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const uint32_t t = threadIdx.x + 256u * u;
        if (t0 + t < nlanes) r[u] = F::load(tsrc, t);
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
        const uint32_t t = threadIdx.x + 256u * u;
        if (t0 + t < nlanes) {
            if constexpr (ADD) F::emit(AddDiff{tout, diff + tval, sa}, t, r[u]);
            else F::emit(ToOut{tout}, t, r[u]);
        }
    }
}

// ------------------------------------------------------------------------------------------------- Q8_0
// 34-byte blocks of 32 values: d (f16) at 0, int8 quants at 2. Lane-item = 8 values (4 per block).
// x = OUT(MID(MID(d) * q)), enhancers/gguf_dequant.py:145-160.
template <int MID, int OUT>
struct Q8_0 {
    static constexpr int LANES_PER_BLOCK = 4, TS = 34, PER = 32, OUT_BYTES = OUT == WF_F32 ? 4 : 2;
    struct Raw { uint32_t d; uint2 q; };
    static __device__ __forceinline__ Raw load(const uint8_t* src, uint32_t t) {
        const uint32_t blk = t >> 2;
        const uint32_t c = t & 3;
        Raw r;
        r.d = *reinterpret_cast<const uint16_t*>(src + blk * 34);
        const uint32_t o = blk * 34 + 2 + 8 * c;              // first quant byte of this lane
        const uint32_t a = o & ~3u;
        const uint32_t sh = (uint32_t)(o & 3) * 8u;           // 0 or 16
        const uint32_t* wp = reinterpret_cast<const uint32_t*>(src + a);
        const uint32_t w0 = wp[0], w1 = wp[1];
        const uint32_t w2 = *reinterpret_cast<const uint16_t*>(src + a + (sh ? 8 : 6));  // inside [o, o + 8)
        r.q = funnel8(w0, w1, w2, sh);
        return r;
    }
    template <class S>
    static __device__ __forceinline__ void emit(const S& o, uint32_t t, const Raw& r) {
        const uint32_t e0 = t * 8;
        if constexpr (MID == WF_F16) {
            const h2 d2 = as_h2(r.d | (r.d << 16));
            const h2 bias = h2s(-1152.0f);                     // 1024 + 128: int8 as unsigned byte ^ 0x80
            const uint32_t u0 = r.q.x ^ 0x80808080u, u1 = r.q.y ^ 0x80808080u;
            h2 v[4];
            v[0] = d2 * (biased_lo(u0) + bias);
            v[1] = d2 * (biased_hi(u0) + bias);
            v[2] = d2 * (biased_lo(u1) + bias);
            v[3] = d2 * (biased_hi(u1) + bias);
            o.template puth<OUT>(e0, v);
        } else {
            const float d = round_to<MID>(f16_bits_to_f32(r.d));
            float v[8];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v[i] = round_to<MID>(d * (float)(int8_t)byte_of(r.q.x, i));
                v[4 + i] = round_to<MID>(d * (float)(int8_t)byte_of(r.q.y, i));
            }
            o.template put<OUT>(e0, v);
        }
    }
};

// ------------------------------------------------------------------------------------------ Q4_K / Q5_K
// Q4_K (144 B): d @0, dmin @2, scales[12] @4, qs[128] @16. Q5_K (176 B): the same plus qh[32] @16, qs @48.
// Lane-item j (16 per super-block) writes values [8j, 8j + 8) and [128 + 8j, 128 + 8j + 8), so each of its two
// store instructions covers whole 256-byte runs of output. With g = j / 4 and c = j % 4, those are sub-blocks g
// and 4 + g; their quants are nibble g % 2 of qs bytes [32(g / 2) + 8c, +8) and [64 + 32(g / 2) + 8c, +8), and Q5_K
// adds bit g / 4 + g of qh[8c + i] as bit 4. x = MID(MID(MID(d * sc) * q) - MID(dmin * m)), :195-212; sc / m of
// sub-block g (< 4) and 4 + g from scale bytes g, g + 4, g + 8 (get_scale_min, :170-185).
template <int QT, int MID, int OUT>
struct Q45_K {
    static constexpr int LANES_PER_BLOCK = 16, PER = 256, OUT_BYTES = OUT == WF_F32 ? 4 : 2;
    static constexpr int TS = QT == 12 ? 144 : 176;
    static constexpr int QS = QT == 12 ? 16 : 48;
    struct Raw { uint4 hdr; uint2 q1, q2, qh; };
    static __device__ __forceinline__ Raw load(const uint8_t* src, uint32_t t) {
        const uint32_t sb = t >> 4;
        const int j = (int)(t & 15), g = j >> 2, c = j & 3;
        const uint8_t* base = src + sb * TS;
        const int o = QS + 32 * (g >> 1) + 8 * c;
        Raw r;
        r.hdr = *reinterpret_cast<const uint4*>(base);
        r.q1 = *reinterpret_cast<const uint2*>(base + o);
        r.q2 = *reinterpret_cast<const uint2*>(base + o + 64);
        if constexpr (QT == 13) r.qh = *reinterpret_cast<const uint2*>(base + 16 + 8 * c);
        return r;
    }
    template <class S>
    static __device__ __forceinline__ void emit(const S& o, uint32_t t, const Raw& r) {
        const uint32_t sb = t >> 4;
        const int j = (int)(t & 15), g = j >> 2;
        const uint32_t ns = 4u * (uint32_t)(g & 1);
        uint32_t n1[2], n2[2];
        n1[0] = (r.q1.x >> ns) & 0x0f0f0f0fu; n1[1] = (r.q1.y >> ns) & 0x0f0f0f0fu;
        n2[0] = (r.q2.x >> ns) & 0x0f0f0f0fu; n2[1] = (r.q2.y >> ns) & 0x0f0f0f0fu;
        if constexpr (QT == 13) {
            n1[0] |= ((r.qh.x >> g) & 0x01010101u) << 4;
            n1[1] |= ((r.qh.y >> g) & 0x01010101u) << 4;
            n2[0] |= ((r.qh.x >> (g + 4)) & 0x01010101u) << 4;
            n2[1] |= ((r.qh.y >> (g + 4)) & 0x01010101u) << 4;
        }
        const uint32_t a = byte_of(r.hdr.y, g), b = byte_of(r.hdr.z, g), cc = byte_of(r.hdr.w, g);
        const uint32_t sc1 = a & 63u, m1 = b & 63u;                                   // sub-block g
        const uint32_t sc2 = (cc & 0xfu) | ((a >> 2) & 0x30u), m2 = (cc >> 4) | ((b >> 2) & 0x30u);  // 4 + g
        const uint32_t e1 = sb * 256 + 8 * j, e2 = e1 + 128;
        if constexpr (MID == WF_F16) {
            const h2 dd = as_h2(r.hdr.x);                       // (d, dmin)
            const h2 off = h2s(-1024.0f);
            // (sc, m) as float16 pairs through the exponent trick, then (d * sc, dmin * m) rounded to f16
            const h2 p1 = dd * (as_h2(sc1 | (m1 << 16) | 0x64006400u) + off);
            const h2 p2 = dd * (as_h2(sc2 | (m2 << 16) | 0x64006400u) + off);
            const h2 ds1 = lo2(p1), dm1 = hi2(p1), ds2 = lo2(p2), dm2 = hi2(p2);
            h2 v1[4], v2[4];
#pragma unroll
            for (int w = 0; w < 2; w++) {
                v1[2 * w] = ds1 * (biased_lo(n1[w]) + off) - dm1;
                v1[2 * w + 1] = ds1 * (biased_hi(n1[w]) + off) - dm1;
                v2[2 * w] = ds2 * (biased_lo(n2[w]) + off) - dm2;
                v2[2 * w + 1] = ds2 * (biased_hi(n2[w]) + off) - dm2;
            }
            o.template puth<OUT>(e1, v1);
            o.template puth<OUT>(e2, v2);
        } else {
            const float d = round_to<MID>(f16_bits_to_f32(r.hdr.x & 0xffffu));
            const float dmin = round_to<MID>(f16_bits_to_f32(r.hdr.x >> 16));
            const float ds1 = round_to<MID>(d * (float)sc1), dm1 = round_to<MID>(dmin * (float)m1);
            const float ds2 = round_to<MID>(d * (float)sc2), dm2 = round_to<MID>(dmin * (float)m2);
            float v1[8], v2[8];
#pragma unroll
            for (int w = 0; w < 2; w++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    v1[4 * w + i] = round_to<MID>(round_to<MID>(ds1 * (float)byte_of(n1[w], i)) - dm1);
                    v2[4 * w + i] = round_to<MID>(round_to<MID>(ds2 * (float)byte_of(n2[w], i)) - dm2);
                }
            o.template put<OUT>(e1, v1);
            o.template put<OUT>(e2, v2);
        }
    }
};

// ------------------------------------------------------------------------------------------------- Q6_K
// 210 B: ql[128] @0, qh[64] @128, int8 scales[16] @192, d @208. Lane-item j (16 per super-block): half h = j / 8,
// chunk c = j % 8 -> ql bytes [64h + 8c, +8): low nibbles are values 128h + 8c + i, high nibbles
// 128h + 64 + 8c + i; their 2 high bits come from qh[32h + 8(c % 4) + i] at shift 2(c / 4) and 2(2 + c / 4);
// scales 8h + c / 2 and 8h + 4 + c / 2. x = MID(MID(MID(d) * sc) * q), q = (lo | hi << 4) - 32, :213-224.
__device__ __forceinline__ uint2 load8_a2(const uint8_t* base, uint32_t o) {
    // 8 bytes at byte offset o (o even): reads [o, o + 8) plus, when o is 2 (mod 4), the 2 bytes before o (the
    // end of the previous block, or of this block's earlier field; never before the buffer, since block 0 starts
    // dword-aligned)
    const uint32_t a = o & ~3u;
    const uint32_t sh = (o & 3) * 8u;
    const uint32_t* wp = reinterpret_cast<const uint32_t*>(base + a);
    const uint32_t w0 = wp[0], w1 = wp[1];
    const uint32_t w2 = *reinterpret_cast<const uint16_t*>(base + a + (sh ? 8 : 6));
    return funnel8(w0, w1, w2, sh);
}

template <int MID, int OUT>
struct Q6_K {
    static constexpr int LANES_PER_BLOCK = 16, TS = 210, PER = 256, OUT_BYTES = OUT == WF_F32 ? 4 : 2;
    struct Raw { uint2 ql, qh; uint32_t sl, sh, d; };
    static __device__ __forceinline__ Raw load(const uint8_t* src, uint32_t t) {
        const uint32_t sb = t >> 4;
        const int j = (int)(t & 15), h = j >> 3, c = j & 7;
        const uint32_t b0 = sb * 210;
        Raw r;
        r.ql = load8_a2(src, b0 + 64 * h + 8 * c);
        r.qh = load8_a2(src, b0 + 128 + 32 * h + 8 * (c & 3));
        r.sl = src[b0 + 192 + 8 * h + (c >> 1)];
        r.sh = src[b0 + 192 + 8 * h + 4 + (c >> 1)];
        r.d = *reinterpret_cast<const uint16_t*>(src + b0 + 208);
        return r;
    }
    template <class S>
    static __device__ __forceinline__ void emit(const S& o, uint32_t t, const Raw& r) {
        const uint32_t sb = t >> 4;
        const int j = (int)(t & 15), h = j >> 3, c = j & 7;
        const uint32_t s1 = 2u * (uint32_t)(c >> 2), s2 = s1 + 4u;
        uint32_t lo[2], hi[2];   // 6-bit codes 0..63, one per byte
        lo[0] = (r.ql.x & 0x0f0f0f0fu) | (((r.qh.x >> s1) & 0x03030303u) << 4);
        hi[0] = ((r.ql.x >> 4) & 0x0f0f0f0fu) | (((r.qh.x >> s2) & 0x03030303u) << 4);
        lo[1] = (r.ql.y & 0x0f0f0f0fu) | (((r.qh.y >> s1) & 0x03030303u) << 4);
        hi[1] = ((r.ql.y >> 4) & 0x0f0f0f0fu) | (((r.qh.y >> s2) & 0x03030303u) << 4);
        const uint32_t eA = sb * 256 + 128 * h + 8 * c, eB = eA + 64;
        if constexpr (MID == WF_F16) {
            const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)r.d);
            h2 dsc;
            dsc[0] = (_Float16)(float)(int8_t)r.sl;
            dsc[1] = (_Float16)(float)(int8_t)r.sh;
            h2 dd; dd[0] = d; dd[1] = d;
            const h2 pd = dd * dsc;                              // (d * sc_lo, d * sc_hi), rounded to f16
            const h2 dA = lo2(pd), dB = hi2(pd);
            const h2 bias = h2s(-1056.0f);                       // 1024 + 32
            h2 va[4], vb[4];
#pragma unroll
            for (int w = 0; w < 2; w++) {
                va[2 * w] = dA * (biased_lo(lo[w]) + bias);
                va[2 * w + 1] = dA * (biased_hi(lo[w]) + bias);
                vb[2 * w] = dB * (biased_lo(hi[w]) + bias);
                vb[2 * w + 1] = dB * (biased_hi(hi[w]) + bias);
            }
            o.template puth<OUT>(eA, va);
            o.template puth<OUT>(eB, vb);
        } else {
            const float d = round_to<MID>(f16_bits_to_f32(r.d));
            const float dA = round_to<MID>(d * (float)(int8_t)r.sl), dB = round_to<MID>(d * (float)(int8_t)r.sh);
            float va[8], vb[8];
#pragma unroll
            for (int w = 0; w < 2; w++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    va[4 * w + i] = round_to<MID>(dA * (float)((int)byte_of(lo[w], i) - 32));
                    vb[4 * w + i] = round_to<MID>(dB * (float)((int)byte_of(hi[w], i) - 32));
                }
            o.template put<OUT>(eA, va);
            o.template put<OUT>(eB, vb);
        }
    }
};

// ------------------------------------------------------------------------------------ format constants
// Legacy formats: block bytes TS, quant bytes at QS, high bits at QH (Q5_x), min at 2 (HAS_M), quant offset SUB
// (enhancers/gguf_dequant.py:52-56).
template <int QT>
struct Fmt;
template <> struct Fmt<2> { static constexpr int TS = 18, PER = 32, HAS_M = 0, QH = -1, QS = 2, SUB = 8; };
template <> struct Fmt<3> { static constexpr int TS = 20, PER = 32, HAS_M = 1, QH = -1, QS = 4, SUB = 0; };
template <> struct Fmt<6> { static constexpr int TS = 22, PER = 32, HAS_M = 0, QH = 2, QS = 6, SUB = 16; };
template <> struct Fmt<7> { static constexpr int TS = 24, PER = 32, HAS_M = 1, QH = 4, QS = 8, SUB = 0; };

// ------------------------------------------------------------------------- Q4_0 / Q4_1 / Q5_0 / Q5_1 (tiled)
// Q4_0 (18 B): d @0, qs[16] @2. Q4_1 (20 B): d @0, m @2, qs @4. Q5_0 (22 B): d @0, qh[4] @2, qs @6. Q5_1 (24 B):
// d @0, m @2, qh[4] @4, qs @8. Value v of a block is nibble v / 16 of qs[v % 16]; Q5_x adds bit v of qh (read as a
// little-endian dword) as bit 4; q = nib - SUB (Q4_0: 8, Q5_0: 16, else 0). x = MID(MID(d) * q), then
// x = MID(x + MID(m)) for Q4_1 / Q5_1 (enhancers/gguf_dequant.py:145-160). Lane-item c (4 per block) writes values
// [8c, 8c + 8): nibble c / 2 of qs bytes [8(c % 2), +8) and the high bits of qh byte c, so a wave's store is 16 whole
// blocks of output (1 KiB for a 2-byte OUT). Blocks of 18 and 22 bytes are only 2-byte aligned: their quants are
// read as aligned dwords and funnel-shifted (load8_a2); Q4_1's are dword-aligned and Q5_1's 8-byte aligned.
template <int QT, int MID, int OUT>
struct Legacy {
    using F = Fmt<QT>;
    static constexpr int LANES_PER_BLOCK = 4, TS = F::TS, PER = 32, OUT_BYTES = OUT == WF_F32 ? 4 : 2;
    struct Raw { uint32_t dm, qh; uint2 q; };
    static __device__ __forceinline__ Raw load(const uint8_t* src, uint32_t t) {
        const uint32_t blk = t >> 2, c = t & 3;
        const uint32_t b = blk * TS;
        const uint32_t o = b + F::QS + 8 * (c & 1);
        Raw r;
        if constexpr (F::HAS_M) r.dm = *reinterpret_cast<const uint32_t*>(src + b);     // TS 20 / 24: aligned
        else r.dm = *reinterpret_cast<const uint16_t*>(src + b);
        if constexpr (F::QH >= 0) r.qh = src[b + F::QH + c];
        else r.qh = 0;
        if constexpr (TS % 8 == 0) {
            r.q = *reinterpret_cast<const uint2*>(src + o);
        } else if constexpr (TS % 4 == 0) {
            const uint32_t* p = reinterpret_cast<const uint32_t*>(src + o);
            r.q = make_uint2(p[0], p[1]);
        } else {
            r.q = load8_a2(src, o);
        }
        return r;
    }
    template <class S>
    static __device__ __forceinline__ void emit(const S& o, uint32_t t, const Raw& r) {
        const uint32_t c = t & 3;
        const uint32_t ns = 4u * (c >> 1);
        uint32_t n[2];
        n[0] = (r.q.x >> ns) & 0x0f0f0f0fu;
        n[1] = (r.q.y >> ns) & 0x0f0f0f0fu;
        if constexpr (F::QH >= 0) {
            // bit i of the qh byte -> bit 4 of byte i: the four shifted copies of a 4-bit value x in
            // x * (1 + 2^7 + 2^14 + 2^21) do not overlap, so bit i lands alone on bit 8i
            n[0] |= (((r.qh & 0xfu) * 0x00204081u) & 0x01010101u) << 4;
            n[1] |= (((r.qh >> 4) * 0x00204081u) & 0x01010101u) << 4;
        }
        const uint32_t e0 = t * 8;
        if constexpr (MID == WF_F16) {
            const uint32_t dbits = r.dm & 0xffffu;
            const h2 d2 = as_h2(dbits | (dbits << 16));
            const h2 bias = h2s(-1024.0f - (float)F::SUB);
            h2 v[4];
#pragma unroll
            for (int w = 0; w < 2; w++) {
                v[2 * w] = d2 * (biased_lo(n[w]) + bias);
                v[2 * w + 1] = d2 * (biased_hi(n[w]) + bias);
            }
            if constexpr (F::HAS_M) {
                const uint32_t mbits = r.dm >> 16;
                const h2 m2 = as_h2(mbits | (mbits << 16));
#pragma unroll
                for (int i = 0; i < 4; i++) v[i] = v[i] + m2;
            }
            o.template puth<OUT>(e0, v);
        } else {
            const float d = round_to<MID>(f16_bits_to_f32(r.dm & 0xffffu));
            float v[8];
#pragma unroll
            for (int w = 0; w < 2; w++)
#pragma unroll
                for (int i = 0; i < 4; i++)
                    v[4 * w + i] = round_to<MID>(d * (float)((int)byte_of(n[w], i) - F::SUB));
            if constexpr (F::HAS_M) {
                const float m = round_to<MID>(f16_bits_to_f32(r.dm >> 16));
#pragma unroll
                for (int i = 0; i < 8; i++) v[i] = round_to<MID>(v[i] + m);
            }
            o.template put<OUT>(e0, v);
        }
    }
};

// ------------------------------------------------------------------------------------------------- Q2_K
// 84 B: scales[16] @0 (low nibble: scale, high nibble: min of 16-value sub-block i), qs[64] @16, d @80, dmin @82.
// Value v: q = (qs[32(v / 128) + v % 32] >> 2((v % 128) / 32)) & 3, dl = MID(MID(d) * (s[v / 16] & 15)),
// ml = MID(MID(dmin) * (s[v / 16] >> 4)), x = MID(MID(dl * q) - ml) (enhancers/gguf_dequant.py:237-246).
// Lane-item j (16 per super-block) writes values [8j, 8j + 8) and [128 + 8j, +8): qs bytes [8(j % 4), +8) and
// [32 + 8(j % 4), +8) at shift 2(j / 4), scale bytes j / 2 and 8 + j / 2.
template <int MID, int OUT>
struct Q2_K {
    static constexpr int LANES_PER_BLOCK = 16, TS = 84, PER = 256, OUT_BYTES = OUT == WF_F32 ? 4 : 2;
    struct Raw { uint2 q1, q2; uint32_t dd, s1, s2; };
    static __device__ __forceinline__ Raw load(const uint8_t* src, uint32_t t) {
        const uint32_t sb = t >> 4, j = t & 15;
        const uint32_t b0 = sb * 84;                           // dword-aligned
        const uint32_t* q = reinterpret_cast<const uint32_t*>(src + b0 + 16 + 8 * (j & 3));
        Raw r;
        r.q1 = make_uint2(q[0], q[1]);
        r.q2 = make_uint2(q[8], q[9]);
        r.dd = *reinterpret_cast<const uint32_t*>(src + b0 + 80);
        r.s1 = src[b0 + (j >> 1)];
        r.s2 = src[b0 + 8 + (j >> 1)];
        return r;
    }
    template <class S>
    static __device__ __forceinline__ void emit(const S& o, uint32_t t, const Raw& r) {
        const uint32_t sb = t >> 4, j = t & 15;
        const uint32_t sh = 2u * (j >> 2);
        uint32_t n1[2], n2[2];
        n1[0] = (r.q1.x >> sh) & 0x03030303u; n1[1] = (r.q1.y >> sh) & 0x03030303u;
        n2[0] = (r.q2.x >> sh) & 0x03030303u; n2[1] = (r.q2.y >> sh) & 0x03030303u;
        const uint32_t e1 = sb * 256 + 8 * j, e2 = e1 + 128;
        if constexpr (MID == WF_F16) {
            const h2 dd = as_h2(r.dd);                          // (d, dmin)
            const h2 off = h2s(-1024.0f);
            // (scale, min) as float16 pairs through the exponent trick, then (d * scale, dmin * min) rounded to f16
            const h2 p1 = dd * (as_h2((r.s1 & 15u) | ((r.s1 >> 4) << 16) | 0x64006400u) + off);
            const h2 p2 = dd * (as_h2((r.s2 & 15u) | ((r.s2 >> 4) << 16) | 0x64006400u) + off);
            const h2 dl1 = lo2(p1), ml1 = hi2(p1), dl2 = lo2(p2), ml2 = hi2(p2);
            h2 v1[4], v2[4];
#pragma unroll
            for (int w = 0; w < 2; w++) {
                v1[2 * w] = dl1 * (biased_lo(n1[w]) + off) - ml1;
                v1[2 * w + 1] = dl1 * (biased_hi(n1[w]) + off) - ml1;
                v2[2 * w] = dl2 * (biased_lo(n2[w]) + off) - ml2;
                v2[2 * w + 1] = dl2 * (biased_hi(n2[w]) + off) - ml2;
            }
            o.template puth<OUT>(e1, v1);
            o.template puth<OUT>(e2, v2);
        } else {
            const float d = round_to<MID>(f16_bits_to_f32(r.dd & 0xffffu));
            const float dmin = round_to<MID>(f16_bits_to_f32(r.dd >> 16));
            const float dl1 = round_to<MID>(d * (float)(r.s1 & 15u)), ml1 = round_to<MID>(dmin * (float)(r.s1 >> 4));
            const float dl2 = round_to<MID>(d * (float)(r.s2 & 15u)), ml2 = round_to<MID>(dmin * (float)(r.s2 >> 4));
            float v1[8], v2[8];
#pragma unroll
            for (int w = 0; w < 2; w++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    v1[4 * w + i] = round_to<MID>(round_to<MID>(dl1 * (float)byte_of(n1[w], i)) - ml1);
                    v2[4 * w + i] = round_to<MID>(round_to<MID>(dl2 * (float)byte_of(n2[w], i)) - ml2);
                }
            o.template put<OUT>(e1, v1);
            o.template put<OUT>(e2, v2);
        }
    }
};

// ------------------------------------------------------------------------------------------------- Q3_K
// 110 B: hmask[32] @0, qs[64] @32, scales[12] @96, d @108. Value v, sub-block i = v / 16: sc = (low 4 bits from
// scale byte i % 8 at nibble i / 8) | (2 high bits from byte 8 + i % 4 at shift 2(i / 4)) << 4, minus 32;
// d' = MID(MID(d) * sc); q = ((qs[32(v / 128) + v % 32] >> 2((v % 128) / 32)) & 3) - 4 * (1 - bit v / 32 of
// hmask[v % 32]); x = MID(d' * q) (enhancers/gguf_dequant.py:225-236). Lane-item j (16 per super-block) writes values
// [8j, 8j + 8) and [128 + 8j, +8): hmask and qs bytes [8(j % 4), +8) (qs also [32 + 8(j % 4), +8)) at shift
// 2(j / 4) (hmask bits j / 4 and 4 + j / 4), sub-blocks j / 2 and 8 + j / 2. The 3-bit code (ql | hbit << 2) enters
// float16 as 1024 + code, and 1028 is subtracted.
template <int MID, int OUT>
struct Q3_K {
    static constexpr int LANES_PER_BLOCK = 16, TS = 110, PER = 256, OUT_BYTES = OUT == WF_F32 ? 4 : 2;
    struct Raw { uint2 hm, q1, q2; uint32_t ls, hs, d; };
    static __device__ __forceinline__ Raw load(const uint8_t* src, uint32_t t) {
        const uint32_t sb = t >> 4, j = t & 15;
        const uint32_t b0 = sb * 110;                          // 2-byte aligned
        const uint32_t c = 8 * (j & 3);
        Raw r;
        r.hm = load8_a2(src, b0 + c);
        r.q1 = load8_a2(src, b0 + 32 + c);
        r.q2 = load8_a2(src, b0 + 64 + c);
        r.ls = src[b0 + 96 + (j >> 1)];
        r.hs = src[b0 + 104 + ((j >> 1) & 3)];
        r.d = *reinterpret_cast<const uint16_t*>(src + b0 + 108);
        return r;
    }
    template <class S>
    static __device__ __forceinline__ void emit(const S& o, uint32_t t, const Raw& r) {
        const uint32_t sb = t >> 4, j = t & 15;
        const uint32_t sh = 2u * (j >> 2), hb = j >> 2;
        const uint32_t hsh = 2u * ((j >> 1) >> 2);             // 2 * (sub-block / 4) for sub-block j / 2
        // sub-block j / 2: low nibble of ls, bits hsh of hs; sub-block 8 + j / 2: high nibble, bits hsh + 4
        const int sc1 = (int)((r.ls & 15u) | (((r.hs >> hsh) & 3u) << 4)) - 32;
        const int sc2 = (int)((r.ls >> 4) | (((r.hs >> (hsh + 4)) & 3u) << 4)) - 32;
        uint32_t c1[2], c2[2];
#pragma unroll
        for (int w = 0; w < 2; w++) {
            const uint32_t hm = w ? r.hm.y : r.hm.x;
            const uint32_t qa = w ? r.q1.y : r.q1.x, qb = w ? r.q2.y : r.q2.x;
            c1[w] = ((qa >> sh) & 0x03030303u) | (((hm >> hb) & 0x01010101u) << 2);
            c2[w] = ((qb >> sh) & 0x03030303u) | (((hm >> (hb + 4)) & 0x01010101u) << 2);
        }
        const uint32_t e1 = sb * 256 + 8 * j, e2 = e1 + 128;
        if constexpr (MID == WF_F16) {
            const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)r.d);
            h2 dd; dd[0] = d; dd[1] = d;
            h2 sc; sc[0] = (_Float16)(float)sc1; sc[1] = (_Float16)(float)sc2;
            const h2 pd = dd * sc;                               // (d * sc1, d * sc2), rounded to f16
            const h2 dA = lo2(pd), dB = hi2(pd);
            const h2 bias = h2s(-1028.0f);                       // 1024 + 4
            h2 v1[4], v2[4];
#pragma unroll
            for (int w = 0; w < 2; w++) {
                v1[2 * w] = dA * (biased_lo(c1[w]) + bias);
                v1[2 * w + 1] = dA * (biased_hi(c1[w]) + bias);
                v2[2 * w] = dB * (biased_lo(c2[w]) + bias);
                v2[2 * w + 1] = dB * (biased_hi(c2[w]) + bias);
            }
            o.template puth<OUT>(e1, v1);
            o.template puth<OUT>(e2, v2);
        } else {
            const float d = round_to<MID>(f16_bits_to_f32(r.d));
            const float dA = round_to<MID>(d * (float)sc1), dB = round_to<MID>(d * (float)sc2);
            float v1[8], v2[8];
#pragma unroll
            for (int w = 0; w < 2; w++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    v1[4 * w + i] = round_to<MID>(dA * (float)((int)byte_of(c1[w], i) - 4));
                    v2[4 * w + i] = round_to<MID>(dB * (float)((int)byte_of(c2[w], i) - 4));
                }
            o.template put<OUT>(e1, v1);
            o.template put<OUT>(e2, v2);
        }
    }
};

// out = OUT(out + OUT(diff * sa)) on n values already in out: the reference's _deq_add with DEQ off (a K-quant
// dequantised by its own kernel first, or the second and later LoRAs, enhancers/gguf_dequant.py:387-409). Lane t
// takes values [8t, 8t + 8); the last lane of a count that is not a multiple of 8 goes value by value.
template <int OUT>
__global__ __launch_bounds__(256) void add_diff(void* __restrict__ out, const float* __restrict__ diff, float sa,
                                                int64_t n) {
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t * 8 < n; t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t e0 = t * 8;
        if (e0 + 8 <= n) {
            float w[8];
            if constexpr (OUT == WF_F32) {
                const float4 a = *reinterpret_cast<const float4*>(static_cast<float*>(out) + e0);
                const float4 b = *reinterpret_cast<const float4*>(static_cast<float*>(out) + e0 + 4);
                w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w; w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
            } else {
                const uint4 a = *reinterpret_cast<const uint4*>(static_cast<uint16_t*>(out) + e0);
                const uint32_t u[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    if constexpr (OUT == WF_BF16) {
                        w[2 * i] = __uint_as_float(u[i] << 16);
                        w[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
                    } else {
                        w[2 * i] = f16_bits_to_f32(u[i] & 0xffffu);
                        w[2 * i + 1] = f16_bits_to_f32(u[i] >> 16);
                    }
                }
            }
            add_scaled<OUT>(w, diff + e0, sa);
            store8<OUT>(out, e0, w);
        } else {
            for (int64_t e = e0; e < n; e++) {
                float w;
                if constexpr (OUT == WF_F32) w = static_cast<float*>(out)[e];
                else if constexpr (OUT == WF_BF16) w = __uint_as_float((uint32_t)static_cast<uint16_t*>(out)[e] << 16);
                else w = f16_bits_to_f32(static_cast<uint16_t*>(out)[e]);
                w = round_to<OUT>(w + round_to<OUT>(diff[e] * sa));
                if constexpr (OUT == WF_F32) static_cast<float*>(out)[e] = w;
                else if constexpr (OUT == WF_BF16) static_cast<uint16_t*>(out)[e] = __builtin_bit_cast(uint16_t, (__bf16)w);
                else static_cast<uint16_t*>(out)[e] = __builtin_bit_cast(uint16_t, (_Float16)w);
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------- launch
struct Launch {
    int64_t nlanes;
    dim3 grid;
};

// grid of the grid-stride add kernel (at most 2^20 workgroups)
static Launch plan(int64_t nlanes) {
    int64_t wgs = (nlanes + 255) / 256;
    if (wgs > (1 << 20)) wgs = 1 << 20;
    if (wgs < 1) wgs = 1;
    return {nlanes, dim3((unsigned)wgs)};
}

// grid of the tiled kernels: one workgroup per tile of DEQ_ITEMS * 256 lane-items, every tile launched (no loop);
// wf_dequant bounds the value count so that this fits gridDim.x
template <typename F, bool ADD>
static void launch_items(const uint8_t* src, void* out, int64_t nblocks, const float* diff, float sa, hipStream_t s) {
    const int64_t nlanes = nblocks * F::LANES_PER_BLOCK;
    const int64_t wgs = (nlanes + 256LL * DEQ_ITEMS - 1) / (256LL * DEQ_ITEMS);
    deq_items<F, ADD><<<dim3((unsigned)wgs), 256, 0, s>>>(src, out, nlanes, diff, sa);
}

template <int MID, int OUT, bool ADD>
static void launch_fmt(int qtype, const uint8_t* src, void* out, int64_t nblocks, const float* diff, float sa,
                       hipStream_t s) {
    switch (qtype) {
    case 8: launch_items<Q8_0<MID, OUT>, ADD>(src, out, nblocks, diff, sa, s); break;
    case 12: launch_items<Q45_K<12, MID, OUT>, ADD>(src, out, nblocks, diff, sa, s); break;
    case 13: launch_items<Q45_K<13, MID, OUT>, ADD>(src, out, nblocks, diff, sa, s); break;
    case 14: launch_items<Q6_K<MID, OUT>, ADD>(src, out, nblocks, diff, sa, s); break;
    case 2: launch_items<Legacy<2, MID, OUT>, ADD>(src, out, nblocks, diff, sa, s); break;
    case 3: launch_items<Legacy<3, MID, OUT>, ADD>(src, out, nblocks, diff, sa, s); break;
    case 6: launch_items<Legacy<6, MID, OUT>, ADD>(src, out, nblocks, diff, sa, s); break;
    case 7: launch_items<Legacy<7, MID, OUT>, ADD>(src, out, nblocks, diff, sa, s); break;
    case 10: launch_items<Q2_K<MID, OUT>, ADD>(src, out, nblocks, diff, sa, s); break;
    case 11: launch_items<Q3_K<MID, OUT>, ADD>(src, out, nblocks, diff, sa, s); break;
    default: break;
    }
}

template <int MID, bool ADD>
static void launch_mid(int out_dt, int qtype, const uint8_t* src, void* out, int64_t nblocks, const float* diff,
                       float sa, hipStream_t s) {
    if (out_dt == WF_F16) launch_fmt<MID, WF_F16, ADD>(qtype, src, out, nblocks, diff, sa, s);
    else if (out_dt == WF_BF16) launch_fmt<MID, WF_BF16, ADD>(qtype, src, out, nblocks, diff, sa, s);
    else launch_fmt<MID, WF_F32, ADD>(qtype, src, out, nblocks, diff, sa, s);
}

template <bool ADD>
static void launch_all(int mid_dt, int out_dt, int qtype, const uint8_t* src, void* out, int64_t nblocks,
                       const float* diff, float sa, hipStream_t s) {
    if (mid_dt == WF_F16) launch_mid<WF_F16, ADD>(out_dt, qtype, src, out, nblocks, diff, sa, s);
    else if (mid_dt == WF_BF16) launch_mid<WF_BF16, ADD>(out_dt, qtype, src, out, nblocks, diff, sa, s);
    else launch_mid<WF_F32, ADD>(out_dt, qtype, src, out, nblocks, diff, sa, s);
}

// bytes per block and values per block of a supported GGML type (0 when unsupported)
int block_bytes(int qtype, int* per) {
    switch (qtype) {
    case 2: *per = 32; return 18;
    case 3: *per = 32; return 20;
    case 6: *per = 32; return 22;
    case 7: *per = 32; return 24;
    case 8: *per = 32; return 34;
    case 10: *per = 256; return 84;
    case 11: *per = 256; return 110;
    case 12: *per = 256; return 144;
    case 13: *per = 256; return 176;
    case 14: *per = 256; return 210;
    default: *per = 0; return 0;
    }
}

}  // namespace wf

namespace wf {
// the checks wf_dequant and wf_dequant_add share; returns WF_OK and the block count, or the error code
static int check_blocks(const char* who, const void* src, int64_t src_bytes, int qtype, int mid_dt, int out_dt,
                        const void* out, int64_t n_values, int64_t* nblocks) {
    int per = 0;
    const int ts = block_bytes(qtype, &per);
    if (!ts) { set_error("%s: GGML type %d is not handled", who, qtype); return WF_EUNSUPPORTED; }
    if (mid_dt < 0 || mid_dt > 2 || out_dt < 0 || out_dt > 2) {
        set_error("%s: dtype codes %d / %d", who, mid_dt, out_dt);
        return WF_EUNSUPPORTED;
    }
    if (src_bytes < 0 || n_values < 0 || src_bytes % ts) {
        set_error("%s: %lld bytes is not a whole number of %d-byte blocks", who, (long long)src_bytes, ts);
        return WF_EUNSUPPORTED;
    }
    *nblocks = src_bytes / ts;
    if (*nblocks * per != n_values) {
        set_error("%s: %lld blocks hold %lld values, not %lld", who, (long long)*nblocks,
                  (long long)(*nblocks * per), (long long)n_values);
        return WF_EUNSUPPORTED;
    }
    if (n_values > (int64_t)1 << 40) {   // keeps every tiled launch under 2^31 workgroups
        set_error("%s: %lld values is beyond the kernels' limit of 2^40", who, (long long)n_values);
        return WF_EUNSUPPORTED;
    }
    if (n_values && (!src || !out)) { set_error("%s: null pointer", who); return WF_EINVAL; }
    if (!aligned(src, 16) || !aligned(out, 16)) {
        set_error("%s: src and out must be 16-byte aligned", who);
        return WF_EUNSUPPORTED;
    }
    return WF_OK;
}
}  // namespace wf

extern "C" int wf_dequant(const void* src, int64_t src_bytes, int qtype, int mid_dt, int out_dt, void* out,
                          int64_t n_values, void* stream) {
    using namespace wf;
    int64_t nblocks = 0;
    const int rc = check_blocks("wf_dequant", src, src_bytes, qtype, mid_dt, out_dt, out, n_values, &nblocks);
    if (rc != WF_OK || n_values == 0) return rc;
    launch_all<false>(mid_dt, out_dt, qtype, static_cast<const uint8_t*>(src), out, nblocks, nullptr, 0.0f,
                      static_cast<hipStream_t>(stream));
    WF_LAUNCH_CHECK("wf_dequant launch");
    return WF_OK;
}

extern "C" int wf_dequant_add(const void* src, int64_t src_bytes, int qtype, int mid_dt, int out_dt,
                              const float* diff, float scale, void* out, int64_t n_values, void* stream) {
    using namespace wf;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (!src) {
        if (out_dt < 0 || out_dt > 2) { set_error("wf_dequant_add: dtype code %d", out_dt); return WF_EUNSUPPORTED; }
        if (n_values < 0) { set_error("wf_dequant_add: %lld values", (long long)n_values); return WF_EINVAL; }
        if (n_values == 0) return WF_OK;
        if (!out || !diff) { set_error("wf_dequant_add: null pointer"); return WF_EINVAL; }
        if (!aligned(out, 16) || !aligned(diff, 16)) {
            set_error("wf_dequant_add: out and diff must be 16-byte aligned");
            return WF_EUNSUPPORTED;
        }
        const Launch L = plan((n_values + 7) / 8);
        if (out_dt == WF_F16) add_diff<WF_F16><<<L.grid, 256, 0, s>>>(out, diff, scale, n_values);
        else if (out_dt == WF_BF16) add_diff<WF_BF16><<<L.grid, 256, 0, s>>>(out, diff, scale, n_values);
        else add_diff<WF_F32><<<L.grid, 256, 0, s>>>(out, diff, scale, n_values);
        WF_LAUNCH_CHECK("wf_dequant_add launch");
        return WF_OK;
    }
    int64_t nblocks = 0;
    const int rc = check_blocks("wf_dequant_add", src, src_bytes, qtype, mid_dt, out_dt, out, n_values, &nblocks);
    if (rc != WF_OK || n_values == 0) return rc;
    if (!diff) { set_error("wf_dequant_add: null pointer"); return WF_EINVAL; }
    if (!aligned(diff, 16)) { set_error("wf_dequant_add: diff must be 16-byte aligned"); return WF_EUNSUPPORTED; }
    launch_all<true>(mid_dt, out_dt, qtype, static_cast<const uint8_t*>(src), out, nblocks, diff, scale, s);
    WF_LAUNCH_CHECK("wf_dequant_add launch");
    return WF_OK;
}
