// Device helpers of the fused K-quant dequant + bf16 GEMM kernels (gemm_gguf.hip, gemm_gguf_tall.hip): the raw
// weight bytes of one dequantisation task of a 32-value stage (16, 8 or 4 values) through a buffer
// resource, and their dequantisation with the reference's rounding chain (MID, then bf16 -- enhancers/
// gguf_dequant.py:195-224,250) into packed bf16 pairs.
#pragma once

#include <cstdint>
#include <type_traits>
#include <utility>

#include "kquant.h"
#include "lds_ring.h"

namespace wf {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int QT>
struct GGUFTs { static constexpr int TS = QT == 12 ? 144 : QT == 13 ? 176 : 210; };

template <int QT>
struct QRaw;
template <> struct QRaw<12> { uint4 hdr, q; };
template <> struct QRaw<13> { uint4 hdr, q, qh; };
template <> struct QRaw<14> { uint4 ql; uint32_t ql4; uint4 qh; uint32_t qh4; uint32_t sc, d; };
// raw bytes of a quarter task (4 values)
template <int QT>
struct QRawQ;
template <> struct QRawQ<12> { uint4 hdr; uint32_t q; };
template <> struct QRawQ<13> { uint4 hdr; uint32_t q, qh; };
template <> struct QRawQ<14> { uint32_t ql0, ql1, qh0, qh1, sc, d; };

__device__ __forceinline__ uint4 ld128(__amdgpu_buffer_rsrc_t r, uint32_t o) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, o, 0, 0));
}
__device__ __forceinline__ uint32_t ld32(__amdgpu_buffer_rsrc_t r, uint32_t o) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, o, 0, 0);
}

// Raw bytes of values [16 h, 16 h + 16) of sub-block G (32 values) of the super-block at byte offset b, for stage
// phase G (the stage's sub-block within its super-block, known at compile time). Only what changes at phase G is
// loaded; the rest stays in the registers from an earlier phase of the same super-block (the caller loads the phases
// of a super-block in order into the same QRaw).
template <int QT, int G>
__device__ __forceinline__ void q_load(__amdgpu_buffer_rsrc_t r, uint32_t b, int h, QRaw<QT>& w) {
    if constexpr (QT == 12 || QT == 13) {
        // Q4_K / Q5_K: header (d, dmin, scales) at 0 once per super-block; qs[32 (G / 2) + 16 h ..] (nibble G % 2)
        // once per two phases; Q5_K qh[16 h ..] (bit G) once per super-block (16-byte aligned blocks)
        constexpr uint32_t QS = QT == 12 ? 16 : 48;
        if constexpr (G == 0) w.hdr = ld128(r, b);
        if constexpr (QT == 13 && G == 0) w.qh = ld128(r, b + 16 + 16 * h);
        if constexpr (G % 2 == 0) w.q = ld128(r, b + QS + 32 * (G >> 1) + 16 * h);
    } else {
        // Q6_K (210-byte blocks, 2-byte aligned). Values v0 = 32 G + 16 h ..: hh = v0 / 128 = G / 4, rr = v0 % 128 =
        // 32 (G % 4) + 16 h; ql[64 hh + rr % 64 ..] (nibble rr / 64) every phase, qh[128 + 32 hh + rr % 32 ..] (shift
        // 2 (rr / 32)) once per four phases, both read as 20 bytes from their aligned-down dword (the window stays
        // inside the block; the offsets within the block are multiples of 16, so the shift is b % 4 for both); the
        // scale byte 192 + v0 / 16 every phase, d at 208 once per super-block -- at their exact widths, as the
        // block's last bytes must not be read past its end.
        constexpr uint32_t hh = G >> 2;
        const uint32_t oql = b + 64 * hh + 32 * (G & 1) + 16 * h;
        w.ql = ld128(r, oql & ~3u);
        w.ql4 = ld32(r, (oql & ~3u) + 16);
        if constexpr ((G & 3) == 0) {
            const uint32_t oqh = b + 128 + 32 * hh + 16 * h;
            w.qh = ld128(r, oqh & ~3u);
            w.qh4 = ld32(r, (oqh & ~3u) + 16);
        }
        w.sc = __builtin_amdgcn_raw_buffer_load_b8(r, b + 192 + 2 * G + h, 0, 0);
        if constexpr (G == 0) w.d = __builtin_amdgcn_raw_buffer_load_b16(r, b + 208, 0, 0);
    }
}

// Raw bytes of the quarter task: values [4 qq, 4 qq + 4) of sub-block G of the super-block at byte offset b, by the
// same rules as q_load (one dword of nibbles / high bits; Q6_K's ql and qh as 8 bytes from their aligned-down dword).
template <int QT, int G>
__device__ __forceinline__ void q_load_q(__amdgpu_buffer_rsrc_t r, uint32_t b, int qq, QRawQ<QT>& w) {
    if constexpr (QT == 12 || QT == 13) {
        constexpr uint32_t QS = QT == 12 ? 16 : 48;
        if constexpr (G == 0) w.hdr = ld128(r, b);
        if constexpr (QT == 13 && G == 0) w.qh = ld32(r, b + 16 + 4 * qq);
        if constexpr (G % 2 == 0) w.q = ld32(r, b + QS + 32 * (G >> 1) + 4 * qq);
    } else {
        constexpr uint32_t hh = G >> 2;
        const uint32_t oql = (b + 64 * hh + 32 * (G & 1) + 4 * qq) & ~3u;
        w.ql0 = ld32(r, oql);
        w.ql1 = ld32(r, oql + 4);
        if constexpr ((G & 3) == 0) {
            const uint32_t oqh = (b + 128 + 32 * hh + 4 * qq) & ~3u;
            w.qh0 = ld32(r, oqh);
            w.qh1 = ld32(r, oqh + 4);
        }
        w.sc = __builtin_amdgcn_raw_buffer_load_b8(r, b + 192 + 2 * G + (qq >> 2), 0, 0);
        if constexpr (G == 0) w.d = __builtin_amdgcn_raw_buffer_load_b16(r, b + 208, 0, 0);
    }
}

// the 16 values as 8 packed bf16 pairs (values 2i, 2i + 1 in o[i]), the reference's rounding chain in MID
template <int QT, int MID, int g>
__device__ __forceinline__ void q_dequant(const QRaw<QT>& w, uint32_t sh, uint32_t (&o)[8]) {
    if constexpr (QT == 12 || QT == 13) {
        const uint32_t ns = 4u * (uint32_t)(g & 1);
        const uint32_t qa[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
        uint32_t q[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            q[i] = (qa[i] >> ns) & 0x0f0f0f0fu;
            if constexpr (QT == 13) {
                const uint32_t qh[4] = {w.qh.x, w.qh.y, w.qh.z, w.qh.w};
                q[i] |= ((qh[i] >> g) & 0x01010101u) << 4;
            }
        }
        uint32_t sc, m;
        scale_min_nb(w.hdr.y, w.hdr.z, w.hdr.w, g, sc, m);
        if constexpr (MID == WF_F16) {
            const h2 off = h2s(-1024.0f);
            const h2 pr = as_h2(w.hdr.x) * (as_h2(sc | (m << 16) | 0x64006400u) + off);   // (d * sc, dmin * m)
            const h2 ds = lo2(pr), dm = hi2(pr);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const h2 v0 = ds * (biased_lo(q[i]) + off) - dm, v1 = ds * (biased_hi(q[i]) + off) - dm;
                o[2 * i] = pack_bf16((float)v0[0], (float)v0[1]);
                o[2 * i + 1] = pack_bf16((float)v1[0], (float)v1[1]);
            }
        } else {
            const float d = round_to<MID>(f16_bits_to_f32(w.hdr.x & 0xffffu));
            const float dmin = round_to<MID>(f16_bits_to_f32(w.hdr.x >> 16));
            const float ds = round_to<MID>(d * (float)sc), dm = round_to<MID>(dmin * (float)m);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = round_to<MID>(round_to<MID>(ds * (float)byte_of(q[i], e)) - dm);
                o[2 * i] = pack_bf16(v[0], v[1]);
                o[2 * i + 1] = pack_bf16(v[2], v[3]);
            }
        }
    } else {
        const uint32_t shl = 8u * sh, shh = shl;         // Q6_K: sh = block offset % 4 (0 or 2)
        const uint32_t la[5] = {w.ql.x, w.ql.y, w.ql.z, w.ql.w, w.ql4};
        const uint32_t ha[5] = {w.qh.x, w.qh.y, w.qh.z, w.qh.w, w.qh4};
        const uint32_t ns = 4u * (uint32_t)((g & 3) >> 1), hs = 2u * (uint32_t)(g & 3);
        uint32_t code[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t ql = __builtin_amdgcn_alignbit(la[i + 1], la[i], shl);
            const uint32_t qh = __builtin_amdgcn_alignbit(ha[i + 1], ha[i], shh);
            code[i] = ((ql >> ns) & 0x0f0f0f0fu) | (((qh >> hs) & 0x03030303u) << 4);
        }
        const int sc = (int8_t)(w.sc & 0xffu);
        const uint32_t dbits = w.d & 0xffffu;
        if constexpr (MID == WF_F16) {
            const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)dbits);
            const _Float16 ds1 = d * (_Float16)(float)sc;                 // d * sc rounded to f16
            h2 ds; ds[0] = ds1; ds[1] = ds1;
            const h2 off = h2s(-1056.0f);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const h2 v0 = ds * (biased_lo(code[i]) + off), v1 = ds * (biased_hi(code[i]) + off);
                o[2 * i] = pack_bf16((float)v0[0], (float)v0[1]);
                o[2 * i + 1] = pack_bf16((float)v1[0], (float)v1[1]);
            }
        } else {
            const float ds = round_to<MID>(round_to<MID>(f16_bits_to_f32(dbits)) * (float)sc);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = round_to<MID>(ds * (float)((int)byte_of(code[i], e) - 32));
                o[2 * i] = pack_bf16(v[0], v[1]);
                o[2 * i + 1] = pack_bf16(v[2], v[3]);
            }
        }
    }
}

// the quarter task's 4 values as 2 packed bf16 pairs (values 0, 1 in o0; 2, 3 in o1), as q_dequant
template <int QT, int MID, int g>
__device__ __forceinline__ void q_dequant_q(const QRawQ<QT>& w, uint32_t sh, uint32_t& o0, uint32_t& o1) {
    if constexpr (QT == 12 || QT == 13) {
        uint32_t q = (w.q >> (4 * (g & 1))) & 0x0f0f0f0fu;
        if constexpr (QT == 13) q |= ((w.qh >> g) & 0x01010101u) << 4;
        uint32_t sc, m;
        scale_min_nb(w.hdr.y, w.hdr.z, w.hdr.w, g, sc, m);
        if constexpr (MID == WF_F16) {
            const h2 off = h2s(-1024.0f);
            const h2 pr = as_h2(w.hdr.x) * (as_h2(sc | (m << 16) | 0x64006400u) + off);   // (d * sc, dmin * m)
            const h2 ds = lo2(pr), dm = hi2(pr);
            const h2 v0 = ds * (biased_lo(q) + off) - dm, v1 = ds * (biased_hi(q) + off) - dm;
            o0 = pack_bf16((float)v0[0], (float)v0[1]);
            o1 = pack_bf16((float)v1[0], (float)v1[1]);
        } else {
            const float d = round_to<MID>(f16_bits_to_f32(w.hdr.x & 0xffffu));
            const float dmin = round_to<MID>(f16_bits_to_f32(w.hdr.x >> 16));
            const float ds = round_to<MID>(d * (float)sc), dm = round_to<MID>(dmin * (float)m);
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; e++) v[e] = round_to<MID>(round_to<MID>(ds * (float)byte_of(q, e)) - dm);
            o0 = pack_bf16(v[0], v[1]);
            o1 = pack_bf16(v[2], v[3]);
        }
    } else {
        const uint32_t shb = 8u * sh;
        const uint32_t ql = __builtin_amdgcn_alignbit(w.ql1, w.ql0, shb);
        const uint32_t qh = __builtin_amdgcn_alignbit(w.qh1, w.qh0, shb);
        const uint32_t code = ((ql >> (4 * ((g & 3) >> 1))) & 0x0f0f0f0fu) | (((qh >> (2 * (g & 3))) & 0x03030303u) << 4);
        const int sc = (int8_t)(w.sc & 0xffu);
        const uint32_t dbits = w.d & 0xffffu;
        if constexpr (MID == WF_F16) {
            const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)dbits);
            const _Float16 ds1 = d * (_Float16)(float)sc;
            h2 ds; ds[0] = ds1; ds[1] = ds1;
            const h2 off = h2s(-1056.0f);
            const h2 v0 = ds * (biased_lo(code) + off), v1 = ds * (biased_hi(code) + off);
            o0 = pack_bf16((float)v0[0], (float)v0[1]);
            o1 = pack_bf16((float)v1[0], (float)v1[1]);
        } else {
            const float ds = round_to<MID>(round_to<MID>(f16_bits_to_f32(dbits)) * (float)sc);
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; e++) v[e] = round_to<MID>(ds * (float)((int)byte_of(code, e) - 32));
            o0 = pack_bf16(v[0], v[1]);
            o1 = pack_bf16(v[2], v[3]);
        }
    }
}

}  // namespace wf
