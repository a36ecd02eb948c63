// Fused K-quant dequantisation + bf16 GEMM for gfx950: y[m, n] = bf16(sum_k x[m, k] * W[n, k] (+ bias[n])), W the
// GGUF weight (Q4_K / Q5_K / Q6_K, [N, K] in 256-value super-blocks along K) dequantised inside the kernel with the
// reference's rounding chain (MID, then bf16 -- enhancers/gguf_dequant.py:195-224,250), float32 accumulation.
// The reference does the dequantisation into a bf16 weight in HBM and then ComfyUI-GGUF's F.linear; here the
// weight never leaves the chip in bf16.
//
// Fragment layout of v_mfma_f32_32x32x16_bf16: lane l holds 8 bf16 of row l % 32 at K offset 8 * (l / 32) of the
// 16-wide step; result layout: lane l, register i -> row 8 (i / 4) + 4 (l / 32) + i % 4, column l % 32. The tiling
// and the pipeline are described at gemm_gguf_dl below.

#include <algorithm>
#include <cstdint>
#include <mutex>
#include <type_traits>
#include <utility>

#include "gguf_tile.h"

namespace wf {

// ------------------------------------------------------------------------- direct-to-LDS ring (K % 256 == 0)
// 256 x 256 tiles (2 x 4 waves of 4 x 2 MFMA tiles) or 256 x 320 tiles (4 x 2 waves of 2 x 5), 8 waves, two per
// SIMD; K in stages of 32 values through a 4-stage LDS ring. The activation stage (256 rows x 64 bytes) goes
// global -> LDS by the load unit (buffer_load ... lds), two 1 KiB instructions per wave; the weight stage is
// dequantised by the threads: thread t takes half (16 values) of the stage's 32-value sub-block of weight row t / 2
// (with 320 rows, also the quarter task t % 8 -- 4 values -- of row 256 + t / 8), from raw bytes loaded a step
// earlier, and writes its bf16 into the ring slot three stages ahead. The loop runs whole super-blocks (8 stages),
// so each stage's sub-block index within its super-block is a compile-time constant: raw bytes shared by several
// stages (headers, Q5_K high bits, the nibble bytes of a sub-block pair, Q6_K high bits) are loaded once and kept.
// Step s: barrier; issue the activations of stage s + 3; both MFMA halves of stage s; wait until only those
// activation loads are in flight (so the raw bytes of stage s + 3 have landed -- the wait counts only the fixed
// number of activation loads); dequantise them into the free slot; load the raw bytes of stage s + 4; prefetch
// stage s + 1's first fragments. Stages at or past K are still issued (reads past a row land in a slot never read,
// or read as zeros past the buffer), which keeps the waits exact and the compiler's per-slot load tracking
// branch-free.
template <int QT, int MID, bool BIAS, int VM, int VN, int WM, int WN>
__global__ __launch_bounds__(512) void gemm_gguf_dl(const uint16_t* __restrict__ X, const uint8_t* __restrict__ W,
                                                    const uint16_t* __restrict__ bias, uint16_t* __restrict__ Y,
                                                    int M, int N, int K) {
    static_assert(VM * VN == 8, "8 waves");
    constexpr int BM = VM * WM * 32, BN = VN * WN * 32;
    constexpr int TS = GGUFTs<QT>::TS;
    constexpr int IX = BM / 16 / 8;                    // activation DMA instructions per wave per stage
    constexpr int T2 = 2 * BN - 512;                   // half-row tasks beyond one per thread (waves 0, 1)
    static_assert(BM == 256 && (T2 == 0 || T2 == 128), "256 x 256 or 256 x 320 tiles");
    // separate activation and weight rings: the weight writes never alias an in-flight activation load
    __shared__ uint4 xs0[BM * 4], xs1[BM * 4], xs2[BM * 4], xs3[BM * 4];
    __shared__ uint4 ws0[BN * 4], ws1[BN * 4], ws2[BN * 4], ws3[BN * 4];
    const int ntm = (M + BM - 1) / BM, ntn = (N + BN - 1) / BN;
    int tm, tn;
    tile_order(blockIdx.x, ntm * ntn, ntm, ntn, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / VN, wn = wave % VN;
    const int nk = K / 32;
    const uint32_t row_bytes = (uint32_t)(K / 256) * TS;
    const __amdgpu_buffer_rsrc_t rx = tile_rsrc(X + (int64_t)m0 * K, (int64_t)(M - m0) * K * 2);
    const __amdgpu_buffer_rsrc_t rw = tile_rsrc(W + (int64_t)n0 * row_bytes, (int64_t)(N - n0) * row_bytes);
    uint32_t xoff[IX];
#pragma unroll
    for (int q = 0; q < IX; q++) {
        const int r = (wave * IX + q) * 16 + (lane >> 2);
        xoff[q] = (uint32_t)r * (uint32_t)K * 2u + 16u * (uint32_t)swz4(r, lane & 3);
    }
    auto issue_x = [&](uint4* st, int kt) {
#pragma unroll
        for (int q = 0; q < IX; q++) lds_dma16(rx, st + 64 * (wave * IX + q), xoff[q] + (uint32_t)kt * 64u);
    };
    // thread t dequantises half t & 1 of weight row t / 2; with 320 rows, it also takes the quarter task t % 8
    // (values 4 (t % 8) ..) of row 256 + t / 8
    const int wh = tid & 1, wr = tid >> 1;
    const int qq = tid & 7, wr2 = 256 + ((tid >> 3) & 63);
    const uint32_t wbase = (uint32_t)wr * row_bytes, wbase2 = (uint32_t)wr2 * row_bytes;
    auto blk = [&](uint32_t base, int kt) { return base + (uint32_t)(kt >> 3) * TS; };
    // raw loads and dequantisation of stage kt, whose phase (kt % 8) the caller passes as a compile-time constant
    auto wload = [&](auto G, QRaw<QT>& raw, int kt) { q_load<QT, decltype(G)::value>(rw, blk(wbase, kt), wh, raw); };
    auto wload2 = [&](auto G, QRawQ<QT>& raw, int kt) {
        q_load_q<QT, decltype(G)::value>(rw, blk(wbase2, kt), qq, raw);
    };
    int wslot[2];
#pragma unroll
    for (int c = 0; c < 2; c++) wslot[c] = wr * 4 + swz4(wr, 2 * wh + c);
    const int wslot2 = (wr2 * 4 + swz4(wr2, qq >> 1)) * 2 + (qq & 1);     // in 8-byte units
    auto wstore = [&](auto G, uint4* st, const QRaw<QT>& raw, int kt) {
        uint32_t o[8];
        q_dequant<QT, MID, decltype(G)::value>(raw, blk(wbase, kt) & 3u, o);
        lds_write16(st + wslot[0], make_uint4(o[0], o[1], o[2], o[3]));
        lds_write16(st + wslot[1], make_uint4(o[4], o[5], o[6], o[7]));
    };
    auto wstore2 = [&](auto G, uint4* st, const QRawQ<QT>& raw, int kt) {
        uint32_t o0, o1;
        q_dequant_q<QT, MID, decltype(G)::value>(raw, blk(wbase2, kt) & 3u, o0, o1);
        lds_write8(reinterpret_cast<uint2*>(st) + wslot2, o0, o1);
    };
    constexpr bool two = T2 > 0;
    const int lr = lane & 31, lk = lane >> 5;
    // fragment slots: MFMA tile i's rows are 32 i past tile 0's, where the swizzle term (row >> 2) & 3 is the same,
    // so one base per K half serves every tile (the 512-byte multiples fold into the LDS read offsets)
    int abase[2], bbase[2];
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
        const int ra = wm * WM * 32 + lr, rb = wn * WN * 32 + lr;
        abase[ks] = ra * 4 + swz4(ra, 2 * ks + lk);
        bbase[ks] = rb * 4 + swz4(rb, 2 * ks + lk);
    }
    bf16x8 fa[2][WM], fb[2][WN];
    auto fread = [&](const uint4* xst, const uint4* wst, int ks, int set) {
#pragma unroll
        for (int i = 0; i < WM; i++) fa[set][i] = __builtin_bit_cast(bf16x8, xst[abase[ks] + 128 * i]);
#pragma unroll
        for (int j = 0; j < WN; j++) fb[set][j] = __builtin_bit_cast(bf16x8, wst[bbase[ks] + 128 * j]);
    };
    f32x16 acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;
    auto mfmas = [&](int set) {
#pragma unroll
        for (int i = 0; i < WM; i++)
#pragma unroll
            for (int j = 0; j < WN; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[set][i], fb[set][j], acc[i][j], 0, 0, 0);
    };

    QRaw<QT> w1;                                       // raw bytes of the next stage to dequantise
    QRawQ<QT> w2;                                      // the same for the quarter task (320-row tiles)
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    using P2 = std::integral_constant<int, 2>;
    using P3 = std::integral_constant<int, 3>;
    issue_x(xs0, 0);
    issue_x(xs1, 1);
    issue_x(xs2, 2);
    auto pro = [&](auto G, uint4* st) {
        constexpr int g = decltype(G)::value;
        wload(G, w1, g);
        if constexpr (two) wload2(G, w2, g);
        wait_vm<0>();
        wstore(G, st, w1, g);
        if constexpr (two) wstore2(G, st, w2, g);
    };
    pro(P0{}, ws0);
    pro(P1{}, ws1);
    pro(P2{}, ws2);
    wload(P3{}, w1, 3);
    if constexpr (two) wload2(P3{}, w2, 3);
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));   // lgkmcnt(0): this thread's LDS writes are done
    wave_barrier_sync();
    fread(xs0, ws0, 0, 0);
    // ring step J of the 8 in a super-block (stage s = kt + J): stage s in slot C, s + 1 in slot NX, and slot F
    // (stage s - 1's) receives stage s + 3. The raw weight bytes of stage s + 3 were loaded at the end of the previous
    // step, before this step's activation loads, so waiting for all but those activation loads lands them; once
    // dequantised, the registers take what changes for stage s + 4 (one set of raw registers, each load a whole
    // step ahead of its use).
    auto step = [&](int kt, auto J, uint4* xc, uint4* wc, uint4* xn, uint4* wn_, uint4* xf, uint4* wf) {
        constexpr int j = decltype(J)::value;
        const int s = kt + j;
        using G3 = std::integral_constant<int, (j + 3) & 7>;
        using G4 = std::integral_constant<int, (j + 4) & 7>;
        wave_barrier_sync();
        issue_x(xf, s + 3);
        fread(xc, wc, 1, 1);
        mfmas(0);
        mfmas(1);
        __builtin_amdgcn_sched_barrier(0);
        wait_vm<IX>();                                 // all but this step's activation loads have landed
        __builtin_amdgcn_sched_barrier(0);             // nothing that reads the raw bytes moves above the wait
        wstore(G3{}, wf, w1, s + 3);
        if constexpr (two) wstore2(G3{}, wf, w2, s + 3);
        __builtin_amdgcn_sched_barrier(0);             // the next loads reuse the raw registers
        wload(G4{}, w1, s + 4);
        if constexpr (two) wload2(G4{}, w2, s + 4);
        fread(xn, wn_, 0, 0);                          // stage s + 1's first fragments for the next step
    };
    // K % 256 == 0: whole super-blocks of 8 stages
    for (int kt = 0; kt < nk; kt += 8) {
        step(kt, P0{}, xs0, ws0, xs1, ws1, xs3, ws3);
        step(kt, P1{}, xs1, ws1, xs2, ws2, xs0, ws0);
        step(kt, P2{}, xs2, ws2, xs3, ws3, xs1, ws1);
        step(kt, P3{}, xs3, ws3, xs0, ws0, xs2, ws2);
        step(kt, std::integral_constant<int, 4>{}, xs0, ws0, xs1, ws1, xs3, ws3);
        step(kt, std::integral_constant<int, 5>{}, xs1, ws1, xs2, ws2, xs0, ws0);
        step(kt, std::integral_constant<int, 6>{}, xs2, ws2, xs3, ws3, xs1, ws1);
        step(kt, std::integral_constant<int, 7>{}, xs3, ws3, xs0, ws0, xs2, ws2);
    }

    // epilogue through LDS (the ring is idle once every load has landed and every wave is past its reads): each
    // wave rounds its tile to bf16 into its own ring slot (waves 0-3 the activation slots, 4-7 the weight slots),
    // IP MFMA rows (32 rows each) at a time, and stores whole 16-byte runs of rows
    constexpr int TR = WM * 32, TC = WN * 32;
    constexpr int IP = (BM * 4 * 16) / (32 * TC * 2) < WM ? (BM * 4 * 16) / (32 * TC * 2) : WM;
    static_assert(IP >= 1 && WM % IP == 0, "whole MFMA rows per pass");
    wait_vm<0>();
    wave_barrier_sync();
    uint4* buf = wave == 0 ? xs0 : wave == 1 ? xs1 : wave == 2 ? xs2 : wave == 3 ? xs3
               : wave == 4 ? ws0 : wave == 5 ? ws1 : wave == 6 ? ws2 : ws3;
    uint16_t* ot = reinterpret_cast<uint16_t*>(buf);
    const uint4* ov = reinterpret_cast<const uint4*>(ot);   // the wave's own region: in-order LDS writes and reads
    const int mw = m0 + wm * TR, nw = n0 + wn * TC;
    float bn[WN];
#pragma unroll
    for (int j = 0; j < WN; j++) {
        const int n = nw + j * 32 + lr;
        bn[j] = BIAS && n < N ? __uint_as_float((uint32_t)bias[n] << 16) : 0.0f;
    }
    constexpr int PR = IP * 32, RUNS = TC / 8;        // rows per pass, 16-byte runs per row
#pragma unroll
    for (int p = 0; p < WM / IP; p++) {
#pragma unroll
        for (int ii = 0; ii < IP; ii++) {
            const int i = p * IP + ii;
#pragma unroll
            for (int j = 0; j < WN; j++)
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    float t = acc[i][j][e];
                    if (BIAS) t = t + bn[j];
                    ot[(ii * 32 + 8 * (e >> 2) + 4 * lk + (e & 3)) * TC + j * 32 + lr] =
                        __builtin_bit_cast(uint16_t, (__bf16)t);
                }
        }
        const int mp = mw + p * PR;
        if ((N & 7) == 0 && (reinterpret_cast<uintptr_t>(Y) & 15) == 0) {   // whole aligned 16-byte runs
#pragma unroll
            for (int it = 0; it < PR * RUNS / 64; it++) {
                const int q = it * 64 + lane, r = q / RUNS, c = q % RUNS;
                const int m = mp + r, n = nw + 8 * c;
                const uint4 v = ov[q];
                if (m < M && n < N) *reinterpret_cast<uint4*>(Y + (int64_t)m * N + n) = v;
            }
        } else {
            for (int it = 0; it < PR * RUNS / 64; it++) {
                const int q = it * 64 + lane, r = q / RUNS, c = q % RUNS;
                const int m = mp + r;
                if (m >= M) continue;
                for (int e = 0; e < 8; e++) {
                    const int n = nw + 8 * c + e;
                    if (n < N) Y[(int64_t)m * N + n] = ot[r * TC + 8 * c + e];
                }
            }
        }
    }
}

// ------------------------------------------------------------------------- few activation rows (M <= 16 MT)
// With few rows of activations the product is bound by reading the weight, so the layout streams the quantised
// weight through the whole chip exactly once: workgroup b takes the 16 NR weight rows [16 NR b, +16 NR) over all
// of K (NR groups of 16 rows, each activation fragment feeding NR MFMAs: every workgroup re-reads the activations
// from L2, so NR = 2 halves that traffic -- 1.1-1.7x faster than NR = 1 on the Wan shapes at 16-64 rows), its NW
// waves taking super-blocks w, w + NW, w + 2 NW, ..., each with the raw bytes of its next two super-blocks in
// flight (two register sets). Lane l dequantises the 8 values [8 (l / 16), +8) of each
// 32-value stage of weight row 16 b + l % 16 straight into its B fragment of v_mfma_f32_16x16x32_bf16 (lane l:
// column l % 16, K offset 8 (l / 16)); its A fragment is the 8 activations of row 16 mt + l % 16 at the same K
// offset, read from global memory (a few rows: they stay in the L2). Result layout: lane l, register i -> row
// 4 (l / 16) + i, column l % 16. The waves' partial sums meet in LDS and are added in wave order 0, 1, ..., NW - 1.
// Rows past M or N read the last valid row and are not stored.
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int QT>
struct SkRaw;
// (the 16-byte header as two 8-byte halves: loaded as one 16-byte tuple into the second of two register sets, it
// landed in temporaries the compiler copied out right after the load, the wave waiting for the load there)
template <> struct SkRaw<12> { uint2 h01, h23; uint2 q[4]; };
template <> struct SkRaw<13> { uint2 h01, h23; uint2 q[4]; uint2 qh; };
template <> struct SkRaw<14> { uint2 ql[4], qh[2]; uint32_t sc[4]; uint32_t d; };
// Q8_0 (the whole-rows form only): for each of the 8 blocks of 32 values that make 256, the 12 bytes (from a dword
// boundary) that hold this lane's 8 quants -- and, for the lanes with kq = 0, the block's d as well
typedef uint32_t u32x3q __attribute__((ext_vector_type(3)));
template <> struct SkRaw<8> { u32x3q raw[8]; };

// bytes [o, o + 8) of the block stream at p (o even): aligned dwords funnel-shifted, inside [o - 2, o + 8)
__device__ __forceinline__ uint2 ld8_even(const uint8_t* p, uint32_t o) {
    const uint32_t a = o & ~3u, sh = (o & 3u) * 8u;
    const uint32_t* wp = reinterpret_cast<const uint32_t*>(p + a);
    const uint32_t w2 = *reinterpret_cast<const uint16_t*>(p + a + (sh ? 8 : 6));
    return funnel8(wp[0], wp[1], w2, sh);
}

// raw bytes of K-quarter kq (values 8 kq .. of every stage) of the super-block at b (b: block start, 16-byte aligned
// for Q4_K / Q5_K, 2-byte aligned for Q6_K)
template <int QT>
__device__ __forceinline__ void sk_load(const uint8_t* b, int kq, SkRaw<QT>& w) {
    if constexpr (QT == 12 || QT == 13) {
        constexpr int QS = QT == 12 ? 16 : 48;
        w.h01 = *reinterpret_cast<const uint2*>(b);
        w.h23 = *reinterpret_cast<const uint2*>(b + 8);
#pragma unroll
        for (int p = 0; p < 4; p++) w.q[p] = *reinterpret_cast<const uint2*>(b + QS + 32 * p + 8 * kq);
        if constexpr (QT == 13) w.qh = *reinterpret_cast<const uint2*>(b + 16 + 8 * kq);
    } else {
        // ql[64 h + 32 gp + 8 kq ..] for stages g with g / 4 = h, g % 2 = gp (nibble (g % 4) / 2); qh[128 + 32 h + 8 kq
        // ..] (bits 2 (g % 4)); the scale of stage g is byte 192 + 2 g + kq / 2, read as the 16 bit-pairs at 192 + 4 i
        const uint32_t o = (uint32_t)(uintptr_t)b & 3u;          // 0 or 2
        const uint8_t* a = b - o;                                // dword-aligned
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int gp = 0; gp < 2; gp++) w.ql[2 * h + gp] = ld8_even(a, o + 64 * h + 32 * gp + 8 * kq);
#pragma unroll
        for (int h = 0; h < 2; h++) w.qh[h] = ld8_even(a, o + 128 + 32 * h + 8 * kq);
        const uint2 s0 = ld8_even(a, o + 192), s1 = ld8_even(a, o + 200);
        w.sc[0] = s0.x; w.sc[1] = s0.y; w.sc[2] = s1.x; w.sc[3] = s1.y;
        w.d = *reinterpret_cast<const uint16_t*>(b + 208);
    }
}

// Q6_K's raw bytes of K-quarter kq through a buffer resource over the workgroup's weight rows, b = the super-block's
// byte offset in it (2-byte aligned: 210-byte blocks), for the few-rows and whole-rows forms. Each 8-byte piece is
// one 12-byte load from its aligned-down dword, the 16 scale bytes one 16- and one 4-byte load (the 4 bytes are used
// only when the block starts 2 bytes past a dword, and then end with it), d one 2-byte load at its place: the
// buffer's range check works per dword, so the dword holding d, which runs 2 bytes past a dword-aligned block, would
// read as zeros at the weight's last block. Fewer load instructions than sk_load<14>, whose many narrow loads (each
// touching 16 rows) kept the few-rows kernel's Q6_K waves waiting on the address unit. The words are kept as loaded
// and shifted by q6_unwin where they are dequantised: a shift right behind its load makes the wave wait for that
// prefetch there. Rows past N (past the resource's end) read as zeros.
struct Q6Win { u32x3q ql[4], qh[2]; uint4 sc; uint32_t t, d, sh; };

__device__ __forceinline__ void sk_load_q6w(__amdgpu_buffer_rsrc_t r, uint32_t b, int kq, Q6Win& w) {
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int gp = 0; gp < 2; gp++)
            w.ql[2 * h + gp] = __builtin_bit_cast(
                u32x3q, __builtin_amdgcn_raw_buffer_load_b96(r, (b + 64 * h + 32 * gp + 8 * kq) & ~3u, 0, 0));
#pragma unroll
    for (int h = 0; h < 2; h++)
        w.qh[h] = __builtin_bit_cast(u32x3q, __builtin_amdgcn_raw_buffer_load_b96(r, (b + 128 + 32 * h + 8 * kq) & ~3u,
                                                                                   0, 0));
    const uint32_t a = (b + 192) & ~3u;
    w.sc = ld128(r, a);
    w.t = ld32(r, a + 16);
    w.d = __builtin_amdgcn_raw_buffer_load_b16(r, b + 208, 0, 0);
    w.sh = (b & 3u) * 8u;
}

__device__ __forceinline__ SkRaw<14> q6_unwin(const Q6Win& w) {
    SkRaw<14> s;
#pragma unroll
    for (int i = 0; i < 4; i++) s.ql[i] = funnel8(w.ql[i][0], w.ql[i][1], w.ql[i][2], w.sh);
#pragma unroll
    for (int h = 0; h < 2; h++) s.qh[h] = funnel8(w.qh[h][0], w.qh[h][1], w.qh[h][2], w.sh);
    s.sc[0] = __builtin_amdgcn_alignbit(w.sc.y, w.sc.x, w.sh);
    s.sc[1] = __builtin_amdgcn_alignbit(w.sc.z, w.sc.y, w.sh);
    s.sc[2] = __builtin_amdgcn_alignbit(w.sc.w, w.sc.z, w.sh);
    s.sc[3] = __builtin_amdgcn_alignbit(w.t, w.sc.w, w.sh);
    s.d = w.d;
    return s;
}

// Q8_0 through a buffer resource: 8 blocks of 34 bytes from byte offset o (a multiple of 4: the units are 272 bytes
// in rows of whole units), one 12-byte load per block from the dword at or below 34 g (lanes kq = 0: the block's d
// and their quants) or below 34 g + 2 + 8 kq (the others' quants); sk_dequant<8> takes them apart
__device__ __forceinline__ void sk_load_q8(__amdgpu_buffer_rsrc_t r, uint32_t o, int kq, SkRaw<8>& w) {
#pragma unroll
    for (int g = 0; g < 8; g++) {
        const uint32_t b = (kq == 0 ? o + 34 * g : o + 34 * g + 2 + 8 * kq) & ~3u;
        w.raw[g] = __builtin_bit_cast(u32x3q, __builtin_amdgcn_raw_buffer_load_b96(r, b, 0, 0));
    }
}

// bytes per 256 values: a K-quant super-block, or 8 Q8_0 blocks
template <int QT>
struct QdTs { static constexpr int TS = QT == 8 ? 272 : GGUFTs<QT>::TS; };

template <int QT>
struct QdRaw { typedef SkRaw<QT> type; };
template <>
struct QdRaw<14> { typedef Q6Win type; };

// the 8 values of stage g as a bf16x8 B fragment, the reference's rounding chain in MID
template <int QT, int MID, int g>
__device__ __forceinline__ bf16x8 sk_dequant(const SkRaw<QT>& w, int kq) {
    uint32_t code[2];
    uint32_t o[4];
    if constexpr (QT == 8) {
        // block g's 8 values of this lane: MID(d * q), q the signed byte (the reference's chain for Q8_0). Block g
        // starts at byte 34 g of the unit (a multiple of 4 for even g, 2 past one for odd g); lane kq's quants at
        // 34 g + 2 + 8 kq. The lanes with kq = 0 hold the 12 bytes from the dword at or below 34 g (d, then their
        // quants 2 or 4 bytes in), the others those from the dword at or below their quants (0 or 2 bytes in); d
        // comes from lane (c, 0) through a lane permute
        const u32x3q v = w.raw[g];
        uint2 qq;
        uint32_t dl;
        if constexpr ((g & 1) == 0) {
            qq = funnel8(v[0], v[1], v[2], 16u);
            dl = v[0] & 0xffffu;
        } else {
            qq = kq == 0 ? make_uint2(v[1], v[2]) : make_uint2(v[0], v[1]);
            dl = v[0] >> 16;
        }
        const uint32_t dg = (uint32_t)__shfl((int)dl, (int)(__lane_id() & 15u));
        if constexpr (MID == WF_F16) {
            const h2 d2 = as_h2(dg | (dg << 16));
            const h2 bias = h2s(-1152.0f);                    // 1024 + 128: the signed byte as unsigned ^ 0x80
            const uint32_t u0 = qq.x ^ 0x80808080u, u1 = qq.y ^ 0x80808080u;
            const h2 v0 = d2 * (biased_lo(u0) + bias), v1 = d2 * (biased_hi(u0) + bias);
            const h2 v2 = d2 * (biased_lo(u1) + bias), v3 = d2 * (biased_hi(u1) + bias);
            o[0] = pack_bf16((float)v0[0], (float)v0[1]);
            o[1] = pack_bf16((float)v1[0], (float)v1[1]);
            o[2] = pack_bf16((float)v2[0], (float)v2[1]);
            o[3] = pack_bf16((float)v3[0], (float)v3[1]);
        } else {
            const float d = round_to<MID>(f16_bits_to_f32(dg));
            float t[8];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                t[e] = round_to<MID>(d * (float)(int8_t)byte_of(qq.x, e));
                t[4 + e] = round_to<MID>(d * (float)(int8_t)byte_of(qq.y, e));
            }
#pragma unroll
            for (int e = 0; e < 4; e++) o[e] = pack_bf16(t[2 * e], t[2 * e + 1]);
        }
    } else if constexpr (QT == 12 || QT == 13) {
        const uint2 qq = w.q[g >> 1];
        code[0] = (qq.x >> (4 * (g & 1))) & 0x0f0f0f0fu;
        code[1] = (qq.y >> (4 * (g & 1))) & 0x0f0f0f0fu;
        if constexpr (QT == 13) {
            code[0] |= ((w.qh.x >> g) & 0x01010101u) << 4;
            code[1] |= ((w.qh.y >> g) & 0x01010101u) << 4;
        }
        uint32_t sc, m;
        scale_min(w.h01.y, w.h23.x, w.h23.y, g, sc, m);
        if constexpr (MID == WF_F16) {
            const h2 off = h2s(-1024.0f);
            const h2 pr = as_h2(w.h01.x) * (as_h2(sc | (m << 16) | 0x64006400u) + off);   // (d * sc, dmin * m)
            const h2 ds = lo2(pr), dm = hi2(pr);
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const h2 v0 = ds * (biased_lo(code[i]) + off) - dm, v1 = ds * (biased_hi(code[i]) + off) - dm;
                o[2 * i] = pack_bf16((float)v0[0], (float)v0[1]);
                o[2 * i + 1] = pack_bf16((float)v1[0], (float)v1[1]);
            }
        } else {
            const float d = round_to<MID>(f16_bits_to_f32(w.h01.x & 0xffffu));
            const float dmin = round_to<MID>(f16_bits_to_f32(w.h01.x >> 16));
            const float ds = round_to<MID>(d * (float)sc), dm = round_to<MID>(dmin * (float)m);
#pragma unroll
            for (int i = 0; i < 2; i++) {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = round_to<MID>(round_to<MID>(ds * (float)byte_of(code[i], e)) - dm);
                o[2 * i] = pack_bf16(v[0], v[1]);
                o[2 * i + 1] = pack_bf16(v[2], v[3]);
            }
        }
    } else {
        constexpr int h = g >> 2, gp = g & 1, ns = 4 * ((g & 3) >> 1), hs = 2 * (g & 3);
        const uint2 ql = w.ql[2 * h + gp], qh = w.qh[h];
        code[0] = ((ql.x >> ns) & 0x0f0f0f0fu) | (((qh.x >> hs) & 0x03030303u) << 4);
        code[1] = ((ql.y >> ns) & 0x0f0f0f0fu) | (((qh.y >> hs) & 0x03030303u) << 4);
        // scale byte 2 g + kq / 2 of the 16: dword (2 g + kq / 2) / 4 = g / 2, byte (2 g + kq / 2) % 4
        const int sbyte = 2 * (g & 1) + (kq >> 1);
        const int sc = (int8_t)((w.sc[g >> 1] >> (8 * sbyte)) & 0xffu);
        if constexpr (MID == WF_F16) {
            const _Float16 ds1 = __builtin_bit_cast(_Float16, (uint16_t)(w.d & 0xffffu)) * (_Float16)(float)sc;
            h2 ds;
            ds[0] = ds1;
            ds[1] = ds1;
            const h2 off = h2s(-1056.0f);
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const h2 v0 = ds * (biased_lo(code[i]) + off), v1 = ds * (biased_hi(code[i]) + off);
                o[2 * i] = pack_bf16((float)v0[0], (float)v0[1]);
                o[2 * i + 1] = pack_bf16((float)v1[0], (float)v1[1]);
            }
        } else {
            const float ds = round_to<MID>(round_to<MID>(f16_bits_to_f32(w.d & 0xffffu)) * (float)sc);
#pragma unroll
            for (int i = 0; i < 2; i++) {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = round_to<MID>(ds * (float)((int)byte_of(code[i], e) - 32));
                o[2 * i] = pack_bf16(v[0], v[1]);
                o[2 * i + 1] = pack_bf16(v[2], v[3]);
            }
        }
    }
    return __builtin_bit_cast(bf16x8, make_uint4(o[0], o[1], o[2], o[3]));
}

template <int QT, int MID, bool BIAS, int MT, int NR, int NW, bool AHEAD>
__global__ __launch_bounds__(64 * NW) void gemm_gguf_skinny(const uint16_t* __restrict__ X,
                                                            const uint8_t* __restrict__ W,
                                                            const uint16_t* __restrict__ bias,
                                                            uint16_t* __restrict__ Y, int M, int N, int K) {
    constexpr int TS = QdTs<QT>::TS;
    __shared__ f32x4 red[NW][NR * MT][64];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, kq = lane >> 4;
    const int n0 = blockIdx.x * 16 * NR;
    const int64_t row_bytes = (int64_t)(K / 256) * TS;
    const uint8_t* wrow[NR];
#pragma unroll
    for (int nr = 0; nr < NR; nr++) wrow[nr] = W + (int64_t)min(n0 + 16 * nr + r, N - 1) * row_bytes;
    // Q6_K, Q8_0: the workgroup's rows through a buffer resource (rows past N read as zeros; their sums are not
    // stored)
    const __amdgpu_buffer_rsrc_t rw = tile_rsrc(W + (int64_t)n0 * row_bytes, (int64_t)min(16 * NR, N - n0) * row_bytes);
    uint32_t rofs[NR];
#pragma unroll
    for (int nr = 0; nr < NR; nr++) rofs[nr] = (uint32_t)((16 * nr + r) * row_bytes);
    const uint16_t* xrow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) xrow[mt] = X + (int64_t)min(16 * mt + r, M - 1) * K + 8 * kq;
    f32x4 acc[NR][MT];
#pragma unroll
    for (int nr = 0; nr < NR; nr++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[nr][mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int nsb = K / 256;
    typedef typename QdRaw<QT>::type Raw;
    auto load = [&](Raw (&w)[NR], int sb) {
#pragma unroll
        for (int nr = 0; nr < NR; nr++) {
            if constexpr (QT == 14) sk_load_q6w(rw, rofs[nr] + (uint32_t)sb * TS, kq, w[nr]);
            else if constexpr (QT == 8) sk_load_q8(rw, rofs[nr] + (uint32_t)sb * TS, kq, w[nr]);
            else sk_load<QT>(wrow[nr] + (int64_t)sb * TS, kq, w[nr]);
        }
    };
    auto unwin = [&](const Raw (&w)[NR], SkRaw<QT> (&u)[NR]) {
#pragma unroll
        for (int nr = 0; nr < NR; nr++) {
            if constexpr (QT == 14) u[nr] = q6_unwin(w[nr]);
            else u[nr] = w[nr];
        }
    };
    // NR groups of 16 weight rows share each activation fragment (NR MFMAs per activation load)
    auto mfmas = [&](const bf16x8 (&bw)[NR], const bf16x8& ax, int mt) {
#pragma unroll
        for (int nr = 0; nr < NR; nr++)
            acc[nr][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ax, bw[nr], acc[nr][mt], 0, 0, 0);
    };
    auto dequant = [&](auto G, const SkRaw<QT> (&w)[NR], bf16x8 (&bw)[NR]) {
#pragma unroll
        for (int nr = 0; nr < NR; nr++) bw[nr] = sk_dequant<QT, MID, decltype(G)::value>(w[nr], kq);
    };
    auto act = [&](int mt, int sb, int g) {
        return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(xrow[mt] + sb * 256 + 32 * g));
    };
    Raw w[2][NR];
    if constexpr (AHEAD) {
        static_assert(MT == 1, "activations one super-block ahead: one row group");
        // one activation row group: its 8 fragments of a super-block fit in registers, so they are loaded one
        // super-block ahead, issued in the order A(next), compute(current), raw(current + 2). The loads a compute
        // waits for are then always older than those left in flight, and the in-order load counter never holds a
        // compute back for a prefetch. Super-blocks wave + NW i, i < cnt; loads past the last one repeat it (their
        // registers are never used), so every round issues the same loads.
        bf16x8 ax[2][8];
        auto load_act = [&](bf16x8 (&a)[8], int sb) {
#pragma unroll
            for (int g = 0; g < 8; g++) a[g] = act(0, sb, g);
        };
        auto superblock = [&](const Raw (&wraw)[NR], const bf16x8 (&a)[8]) {
            SkRaw<QT> wr[NR];
            unwin(wraw, wr);
            static_for<8>([&](auto G) {
                bf16x8 bw[NR];
                dequant(G, wr, bw);
                mfmas(bw, a[decltype(G)::value], 0);
            });
        };
        const int cnt = wave < nsb ? (nsb - 1 - wave) / NW + 1 : 0;
        auto sb_of = [&](int i) { return wave + NW * min(i, cnt - 1); };
        if (cnt > 0) {
            load(w[0], sb_of(0));
            load_act(ax[0], sb_of(0));
            load(w[1], sb_of(1));
            int i = 0;
            for (; i + 2 <= cnt; i += 2) {
                load_act(ax[1], sb_of(i + 1));
                superblock(w[0], ax[0]);
                load(w[0], sb_of(i + 2));
                load_act(ax[0], sb_of(i + 2));
                superblock(w[1], ax[1]);
                load(w[1], sb_of(i + 3));
            }
            if (i < cnt) superblock(w[0], ax[0]);
        }
    } else {
        // activation fragments read at each stage; the raw bytes of the next two super-blocks stay in flight (two
        // register sets, each refilled two super-blocks ahead)
        auto superblock = [&](const Raw (&wraw)[NR], int sb) {
            SkRaw<QT> wr[NR];
            unwin(wraw, wr);
            static_for<8>([&](auto G) {
                bf16x8 bw[NR];
                dequant(G, wr, bw);
#pragma unroll
                for (int mt = 0; mt < MT; mt++) mfmas(bw, act(mt, sb, decltype(G)::value), mt);
            });
        };
        int sb = wave;
        if (sb < nsb) load(w[0], sb);
        if (sb + NW < nsb) load(w[1], sb + NW);
        while (sb < nsb) {
            superblock(w[0], sb);
            if (sb + 2 * NW < nsb) load(w[0], sb + 2 * NW);
            sb += NW;
            if (sb >= nsb) break;
            superblock(w[1], sb);
            if (sb + 2 * NW < nsb) load(w[1], sb + 2 * NW);
            sb += NW;
        }
    }
#pragma unroll
    for (int nr = 0; nr < NR; nr++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) red[wave][nr * MT + mt][lane] = acc[nr][mt];
    __syncthreads();
    for (int idx = wave; idx < NR * MT; idx += NW) {
        const int nr = idx / MT, mt = idx % MT;
        const int n = n0 + 16 * nr + r;
        const float bn = BIAS && n < N ? __uint_as_float((uint32_t)bias[n] << 16) : 0.0f;
        f32x4 t = red[0][idx][lane];
#pragma unroll
        for (int v = 1; v < NW; v++) t = t + red[v][idx][lane];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = 16 * mt + 4 * kq + i;
            float y = t[i];
            if (BIAS) y = y + bn;
            if (m < M && n < N) Y[(int64_t)m * N + n] = __builtin_bit_cast(uint16_t, (__bf16)y);
        }
    }
}

// ------------------------------------------------------------- few activation rows, whole rows per CU (M <= 4)
// gemm_gguf_skinny gives each workgroup 32 whole weight rows: 160 workgroups for a 5120-wide output on 256 CUs, which
// at one or two rows are bound by the dequantisation's VALU issue (each weight value is dequantised for one or two
// products). Here workgroup b of G takes the row quads [Qt b / G, Qt (b + 1) / G) (Qt = N / 4 quads of 4 weight rows):
// 20 whole rows of a 5120-wide output on each of 256 CUs. The 16 columns of v_mfma_f32_16x16x32_bf16 hold 4 weight
// rows x 4 parts of K (column c = 4 j + h: row j of the quad, part h = super-blocks [h S, h S + S), S = nsb / 4
// rounded up), its 16 rows the M <= 4 activation rows x the same 4 parts (row a = 4 t + h: activation row t over
// part h), so one step multiplies super-block h S + s of every part at once, and the wanted sums are the diagonal
// blocks D[4 t + h][4 j + h]: lane (c, kq) keeps register h = c % 4 (activation row t = kq), and the 4 parts are
// added across lanes c ^ 1 and c ^ 2. Each lane dequantises its 8 values straight into its B fragment as in the
// few-rows kernel. Unit (quad, s) = one step over super-block s of the 4 parts; a workgroup's units (quad-major) are
// spread evenly over its NW waves, each wave streaming its range with the raw bytes two units ahead and the unit's 8
// activation fragments one unit ahead. A wave's sums for a quad go to LDS (red[quad][wave][4 t + j], zero where a
// wave has no share) and are added in wave order after the barrier: no partial sums leave the workgroup. Weight and
// activation bytes come through buffer resources; parts past K, rows past N and activation rows past M take an
// offset past the resource's end and read as zeros.
constexpr int kQdMaxQuads = 8;           // row quads per workgroup: N < 8192 on 256 workgroups, < 16384 on 512
constexpr int kQdWaves = 4;              // one wave per SIMD (two measured slower: half the units per wave)
constexpr uint32_t kQdNowhere = 0x80000000u;

__device__ __forceinline__ uint2 ld64(__amdgpu_buffer_rsrc_t r, uint32_t o) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, o, 0, 0));
}

// sk_load's bytes through a buffer resource (o: the super-block's byte offset, or kQdNowhere for zeros)
template <int QT>
__device__ __forceinline__ void sk_load_rs(__amdgpu_buffer_rsrc_t r, uint32_t o, int kq, SkRaw<QT>& w) {
    constexpr int QS = QT == 12 ? 16 : 48;
    w.h01 = ld64(r, o);
    w.h23 = ld64(r, o + 8);
#pragma unroll
    for (int p = 0; p < 4; p++) w.q[p] = ld64(r, o + QS + 32 * p + 8 * kq);
    if constexpr (QT == 13) w.qh = ld64(r, o + 16 + 8 * kq);
}

template <int QT>
__device__ __forceinline__ void quad_load(__amdgpu_buffer_rsrc_t r, uint32_t o, int kq, typename QdRaw<QT>::type& w) {
    if constexpr (QT == 14) sk_load_q6w(r, o, kq, w);
    else if constexpr (QT == 8) sk_load_q8(r, o, kq, w);
    else sk_load_rs<QT>(r, o, kq, w);
}


template <int QT, int MID, bool BIAS>
__global__ __launch_bounds__(64 * kQdWaves) void gemm_gguf_quad(const uint16_t* __restrict__ X,
                                                          const uint8_t* __restrict__ W,
                                                          const uint16_t* __restrict__ bias,
                                                          uint16_t* __restrict__ Y, int M, int N, int K, int G) {
    constexpr int TS = QdTs<QT>::TS, NW = kQdWaves;
    __shared__ float red[kQdMaxQuads][NW][16];
    const int tid = threadIdx.x, lane = tid & 63, c = lane & 15, kq = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = c & 3, jt = c >> 2;                 // part; quad row (B) and activation row (A) of this lane
    const int nsb = K / 256, S = (nsb + 3) / 4;
    const int Qt = (N + 3) / 4;
    const int q0 = (int)((int64_t)Qt * blockIdx.x / G), nq = (int)((int64_t)Qt * (blockIdx.x + 1) / G) - q0;
    const int nu = nq * S;
    const int lo = nu * wave / NW, hi = nu * (wave + 1) / NW;
    for (int i = tid; i < kQdMaxQuads * NW * 16; i += 64 * NW) (&red[0][0][0])[i] = 0.0f;
    const uint32_t row_bytes = (uint32_t)nsb * TS;
    const __amdgpu_buffer_rsrc_t rw = tile_rsrc(W, (int64_t)N * row_bytes);
    const __amdgpu_buffer_rsrc_t rx = tile_rsrc(X, (int64_t)M * K * 2);
    // this lane's byte offsets of unit (quad lq of the workgroup's, step ls): weight row 4 (q0 + lq) + jt,
    // super-block h S + ls; activation row jt over the same super-block
    auto wofs = [&](int lq, int ls) {
        const int row = 4 * (q0 + lq) + jt, sb = h * S + ls;
        return row < N && sb < nsb ? (uint32_t)row * row_bytes + (uint32_t)sb * TS : kQdNowhere;
    };
    auto xofs = [&](int ls) {
        const int sb = h * S + ls;
        return jt < M && sb < nsb ? (uint32_t)(jt * K + sb * 256 + 8 * kq) * 2u : kQdNowhere;
    };
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    typedef typename QdRaw<QT>::type Raw;
    auto unit = [&](const Raw& raw, const bf16x8 (&a)[8]) {
        SkRaw<QT> wr;
        if constexpr (QT == 14) wr = q6_unwin(raw);
        else wr = raw;
        static_for<8>([&](auto Gc) {
            const bf16x8 bw = sk_dequant<QT, MID, decltype(Gc)::value>(wr, kq);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[decltype(Gc)::value], bw, acc, 0, 0, 0);
        });
    };
    // the wave's sums for quad cq: register h of lane (c, kq) is D[4 kq + h][c], parts added across lanes c ^ 1, c ^ 2
    auto flush = [&](int cq) {
        float v = h == 0 ? acc[0] : h == 1 ? acc[1] : h == 2 ? acc[2] : acc[3];
        v = v + __shfl_xor(v, 1);
        v = v + __shfl_xor(v, 2);
        if (h == 0 && kq < M) red[cq][wave][4 * kq + jt] = v;
        acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    };
    __syncthreads();                                  // red is zero before any wave's sums land
    if (lo < hi) {
        int li = lo, lq = lo / S, ls = lo - lq * S;   // load cursor; it stops at the range's last unit
        auto next_load = [&]() {
            if (li + 1 < hi) {
                li++;
                if (++ls == S) { ls = 0; lq++; }
            }
        };
        Raw w[2];
        bf16x8 ax[2][8];
        auto load_act = [&](bf16x8 (&a)[8], int s) {
            const uint32_t o = xofs(s);
#pragma unroll
            for (int g = 0; g < 8; g++) a[g] = __builtin_bit_cast(bf16x8, ld128(rx, o + 64 * g));
        };
        int cq = lo / S, cs = lo - cq * S;            // compute cursor
        auto finish_unit = [&](int ui) {
            const bool quad_end = ++cs == S;
            if (quad_end || ui + 1 == hi) flush(cq);
            if (quad_end) { cs = 0; cq++; }
        };
        quad_load<QT>(rw, wofs(lq, ls), kq, w[0]);
        load_act(ax[0], ls);
        next_load();
        quad_load<QT>(rw, wofs(lq, ls), kq, w[1]);
        int i = lo;
        for (; i + 2 <= hi; i += 2) {
            next_load();                              // cursor at unit i + 2 (or the last)
            load_act(ax[1], (i + 1) % S);
            unit(w[0], ax[0]);
            finish_unit(i);
            quad_load<QT>(rw, wofs(lq, ls), kq, w[0]);
            load_act(ax[0], ls);
            unit(w[1], ax[1]);
            finish_unit(i + 1);
            next_load();
            quad_load<QT>(rw, wofs(lq, ls), kq, w[1]);
        }
        if (i < hi) {
            unit(w[0], ax[0]);
            finish_unit(i);
        }
    }
    __syncthreads();
    for (int idx = tid; idx < nq * 4 * M; idx += 64 * NW) {
        const int qq = idx / (4 * M), e = idx - qq * 4 * M, t = e >> 2, j = e & 3;
        const int n = 4 * (q0 + qq) + j;
        if (n >= N) continue;
        float y = red[qq][0][4 * t + j];
#pragma unroll
        for (int v = 1; v < NW; v++) y = y + red[qq][v][4 * t + j];
        if (BIAS) y = y + __uint_as_float((uint32_t)bias[n] << 16);
        Y[(int64_t)t * N + n] = __builtin_bit_cast(uint16_t, (__bf16)y);
    }
}

// ------------------------------------------------------------- few activation rows, split along K (M <= 16 MT)
// The same weight stream as gemm_gguf_skinny, cut into many more workgroups: workgroup (tn, s) takes the 128 weight
// rows [128 tn, +128) -- 4 waves of two 16-row groups -- over super-blocks [KS s, KS s + KS) of K only (slice s of
// S). It issues the raw bytes of all its super-blocks first, then copies the slice's activations X[0:M, slice] into
// LDS once (rows padded by 16 bytes, so the 16 rows of a fragment read fall in different banks); each wave then
// dequantises its rows straight into B fragments as gemm_gguf_skinny does and reads its A fragments from LDS, so a
// workgroup reads the activations from L2 once per 128 weight rows instead of once per 32. A slice's partial sums go
// to part[s][m][n] (float32). The workgroups of a column tile count themselves on counters[tn]; the last one to
// arrive adds the S partials in slice order 0, 1, ..., S - 1, adds the bias, rounds to bf16, stores, and sets the
// counter back to 0 for the next launch: the result does not depend on which workgroup arrives last.
// Hand-over between workgroups (which may sit on different XCDs, each with its own L2): the partials are written
// and read as device-scope relaxed atomics -- stores and loads coherent across the L2s, without the writeback of a
// whole L2 that a device-scope fence costs (two such fences per workgroup made the kernel several times slower) --
// each thread waits until its stores are acknowledged before the workgroup's barrier, and only then is the counter
// incremented; the last workgroup reads the partials after its increment has returned.
constexpr int kSpWaves = 4;
constexpr int kSpRows = 32 * kSpWaves;   // weight rows per workgroup

template <int QT, int MID, bool BIAS, int MT, int KS>
__global__ __launch_bounds__(64 * kSpWaves) void gemm_gguf_splitk(const uint16_t* __restrict__ X,
                                                                  const uint8_t* __restrict__ W,
                                                                  const uint16_t* __restrict__ bias,
                                                                  uint16_t* __restrict__ Y, int M, int N, int K,
                                                                  int S, unsigned* __restrict__ counters,
                                                                  float* __restrict__ part) {
    constexpr int TS = GGUFTs<QT>::TS, NR = 2;
    constexpr int LROW = 512 * KS + 16;               // LDS bytes per activation row of the slice
    constexpr int CPR = 32 * KS;                      // 16-byte chunks per activation row of the slice
    __shared__ __align__(16) uint8_t xs[16 * MT * LROW];
    __shared__ unsigned is_last;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, kq = lane >> 4;
    const int NT = (N + kSpRows - 1) / kSpRows;
    const int tn = blockIdx.x % NT, s = blockIdx.x / NT;
    const int nsb = K / 256;
    const int sb0 = s * KS;
    const int nks = min(KS, nsb - sb0);               // super-blocks of this slice (>= 1)
    const int n0 = tn * kSpRows + wave * 32;
    const int64_t row_bytes = (int64_t)nsb * TS;
    SkRaw<QT> w[KS][NR];
#pragma unroll
    for (int j = 0; j < KS; j++) {
        if (j < nks) {
#pragma unroll
            for (int nr = 0; nr < NR; nr++)
                sk_load<QT>(W + (int64_t)min(n0 + 16 * nr + r, N - 1) * row_bytes + (int64_t)(sb0 + j) * TS, kq,
                            w[j][nr]);
        }
    }
    // the slice's activations: rows past M repeat row M - 1 (their sums are never stored), columns past the slice's
    // last super-block are zeros (never read)
    for (int c = tid; c < 16 * MT * CPR; c += 64 * kSpWaves) {
        const int row = c / CPR, cc = c - row * CPR;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (cc < 32 * nks)
            v = *reinterpret_cast<const uint4*>(X + (int64_t)min(row, M - 1) * K + (int64_t)sb0 * 256 + 8 * cc);
        *reinterpret_cast<uint4*>(xs + row * LROW + 16 * cc) = v;
    }
    __syncthreads();
    f32x4 acc[NR][MT];
#pragma unroll
    for (int nr = 0; nr < NR; nr++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[nr][mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    auto stage = [&](auto G, int j) {
        constexpr int g = decltype(G)::value;
        bf16x8 bw[NR];
#pragma unroll
        for (int nr = 0; nr < NR; nr++) bw[nr] = sk_dequant<QT, MID, g>(w[j][nr], kq);
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const bf16x8 ax = *reinterpret_cast<const bf16x8*>(xs + (16 * mt + r) * LROW + 2 * (256 * j + 32 * g + 8 * kq));
#pragma unroll
            for (int nr = 0; nr < NR; nr++)
                acc[nr][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ax, bw[nr], acc[nr][mt], 0, 0, 0);
        }
    };
#pragma unroll
    for (int j = 0; j < KS; j++) {
        if (j < nks) {
            stage(std::integral_constant<int, 0>{}, j);
            stage(std::integral_constant<int, 1>{}, j);
            stage(std::integral_constant<int, 2>{}, j);
            stage(std::integral_constant<int, 3>{}, j);
            stage(std::integral_constant<int, 4>{}, j);
            stage(std::integral_constant<int, 5>{}, j);
            stage(std::integral_constant<int, 6>{}, j);
            stage(std::integral_constant<int, 7>{}, j);
        }
    }
    // this slice's partial sums: lane (r, kq), register i holds row 16 mt + 4 kq + i, column n0 + 16 nr + r
    float* ps = part + (int64_t)s * M * N;
#pragma unroll
    for (int nr = 0; nr < NR; nr++) {
        const int n = n0 + 16 * nr + r;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = 16 * mt + 4 * kq + i;
                if (m < M && n < N)
                    __hip_atomic_store(ps + (int64_t)m * N + n, acc[nr][mt][i], __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
    }
    __builtin_amdgcn_s_waitcnt(0);                    // this thread's partials acknowledged
    __syncthreads();                                  // ... and every thread's
    if (tid == 0)
        is_last = __hip_atomic_fetch_add(counters + tn, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                  (unsigned)(S - 1);
    __syncthreads();
    if (!is_last) return;
    const int nb = tn * kSpRows;
    for (int idx = tid; idx < M * kSpRows; idx += 64 * kSpWaves) {
        const int m = idx / kSpRows, n = nb + (idx - m * kSpRows);
        if (n >= N) continue;
        float* p = part + (int64_t)m * N + n;
        const int64_t slice = (int64_t)M * N;
        // the partials in batches of 8 loads in flight (one at a time would wait out a memory latency each), then
        // added in slice order
        float t = 0.0f;
        for (int q0 = 0; q0 < S; q0 += 8) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; j++)
                v[j] = q0 + j < S ? __hip_atomic_load(p + (q0 + j) * slice, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                  : 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (q0 + j < S) t = (q0 + j == 0) ? v[j] : t + v[j];
        }
        if (BIAS) t = t + __uint_as_float((uint32_t)bias[n] << 16);
        Y[(int64_t)m * N + n] = __builtin_bit_cast(uint16_t, (__bf16)t);
    }
    if (tid == 0) __hip_atomic_store(counters + tn, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ----------------------------------------------------------------- medium row counts (16 < M <= kPanelMaxRows)
// Between the few-rows kernel (every workgroup reads its activation fragments from L2: too much traffic beyond 64
// rows, and from 17-33 rows on the panel's split K already fills the chip better) and the tiled kernel (256 x 320
// output tiles: 16-128 workgroups on 256 CUs below 2048 rows), a workgroup takes a panel: 128 weight rows (4 waves,
// each two 16-row groups as in the few-rows kernel) against BM = 16 MT activation rows (MT = 2, 4 or 8), over a
// slice of KS super-blocks of K. The activations stream through a two-buffer LDS ring, one
// half super-block (BM rows x 256 bytes) per buffer -- 64 KiB at 128 rows, so two workgroups share a CU --, copied
// by the load unit straight into LDS (buffer_load ... lds) one half ahead, 16-byte chunk c of row r at chunk
// c ^ (r & 15) (the 16 rows of a fragment read fall in 16 different bank groups). The weight's raw bytes of the next
// super-block load into the second of two register sets meanwhile, and each lane dequantises into its B fragments
// as in the few-rows kernel; A fragments come from LDS.
// K is split into S slices only as far as needed to give the chip 256 workgroups: with S > 1 each slice writes its
// float32 partial sums (part[s][m][n]) and gguf_panel_sum adds them in slice order (deterministic), adds the bias
// and rounds to bf16.
constexpr int kPnWaves = 4;
constexpr int kPnRows = 32 * kPnWaves;   // weight rows per workgroup

template <int QT, int MID, bool BIAS, int MT, bool PART>
__global__ __launch_bounds__(64 * kPnWaves) __attribute__((amdgpu_waves_per_eu(2))) void gemm_gguf_panel(const uint16_t* __restrict__ X,
                                                                 const uint8_t* __restrict__ W,
                                                                 const uint16_t* __restrict__ bias,
                                                                 uint16_t* __restrict__ Y, float* __restrict__ part,
                                                                 int M, int N, int K, int NT, int MTI, int KS) {
    constexpr int TS = QdTs<QT>::TS, NR = 2, BM = 16 * MT;
    constexpr int RPW = BM / 4 / kPnWaves;             // 1 KiB DMA runs per wave per half super-block
    __shared__ __align__(1024) uint8_t xs0[BM * 256], xs1[BM * 256];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15, kq = lane >> 4;
    int b = blockIdx.x;
    const int tn = b % NT;
    b /= NT;
    const int tm = b % MTI, s = b / MTI;
    const int nsb = K / 256, sb0 = s * KS, nks = min(KS, nsb - sb0);
    const int m0 = tm * BM, n0 = tn * kPnRows + wave * 32;
    const int64_t row_bytes = (int64_t)nsb * TS;
    const uint8_t* wrow[NR];
#pragma unroll
    for (int nr = 0; nr < NR; nr++) wrow[nr] = W + (int64_t)min(n0 + 16 * nr + r, N - 1) * row_bytes;
    // Q8_0: the wave's 32 weight rows through a buffer resource (rows past N read as zeros; their sums are not stored)
    const __amdgpu_buffer_rsrc_t rw = tile_rsrc(W + (int64_t)min(n0, N) * row_bytes,
                                                (int64_t)max(0, min(32, N - n0)) * row_bytes);
    // rows past M read as zeros (the buffer's range ends at row M); their sums are never stored
    const __amdgpu_buffer_rsrc_t rx = tile_rsrc(X + (int64_t)m0 * K, (int64_t)(M - m0) * K * 2);
    uint32_t aoff[RPW];
#pragma unroll
    for (int q = 0; q < RPW; q++) {
        const int p = 64 * (wave + kPnWaves * q) + lane;          // 16-byte LDS chunk this lane fills
        const int row = p >> 4, c = (p & 15) ^ (row & 15);
        aoff[q] = (uint32_t)row * (uint32_t)K * 2u + 16u * (uint32_t)c;
    }
    // half h of super-block sb: activations [256 sb + 128 h, + 128) of each row
    auto issue_a = [&](uint8_t* buf, int sb, int h) {
#pragma unroll
        for (int q = 0; q < RPW; q++)
            lds_dma16(rx, buf + 1024 * (wave + kPnWaves * q), aoff[q] + (uint32_t)sb * 512u + (uint32_t)h * 256u);
    };
    SkRaw<QT> w0[NR], w1[NR];
    auto load_raw = [&](SkRaw<QT> (&wr)[NR], int sb) {
#pragma unroll
        for (int nr = 0; nr < NR; nr++) {
            if constexpr (QT == 8) sk_load_q8(rw, (uint32_t)((16 * nr + r) * row_bytes + sb * TS), kq, wr[nr]);
            else sk_load<QT>(wrow[nr] + (int64_t)sb * TS, kq, wr[nr]);
        }
    };
    f32x4 acc[NR][MT];
#pragma unroll
    for (int nr = 0; nr < NR; nr++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[nr][mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // the four stages of half H of a super-block: A fragments from the half's buffer (chunk 4 (g % 4) + kq of row
    // 16 mt + r, at chunk ^ r), B fragments dequantised from the super-block's raw bytes
    auto compute = [&](auto H, const uint8_t* buf, const SkRaw<QT> (&wr)[NR]) {
        static_for<4>([&](auto G) {
            constexpr int gl = decltype(G)::value, g = 4 * decltype(H)::value + gl;
            bf16x8 bw[NR];
#pragma unroll
            for (int nr = 0; nr < NR; nr++) bw[nr] = sk_dequant<QT, MID, g>(wr[nr], kq);
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const bf16x8 ax = *reinterpret_cast<const bf16x8*>(buf + (16 * mt + r) * 256 + 16 * ((4 * gl + kq) ^ r));
#pragma unroll
                for (int nr = 0; nr < NR; nr++)
                    acc[nr][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ax, bw[nr], acc[nr][mt], 0, 0, 0);
            }
        });
    };
    // the ring, one half super-block (BM rows x 256 bytes, 32 KiB at 128 rows) per buffer, so that two workgroups
    // fit a CU's LDS (two waves per SIMD): half 0 of every super-block in buffer 0, half 1 in buffer 1. At the top
    // of each half every wave's copies of it have landed (own loads: the counter; the others': the barrier) and
    // every wave is past its reads of the other buffer, which then receives the next half; the next super-block's
    // raw weight bytes load during half 1, into the register set the previous super-block used.
    using H0 = std::integral_constant<int, 0>;
    using H1 = std::integral_constant<int, 1>;
    auto superblock = [&](int i, SkRaw<QT> (&cur)[NR], SkRaw<QT> (&nxt)[NR]) {
        wait_vm<0>();
        wave_barrier_sync();
        issue_a(xs1, sb0 + i, 1);
        compute(H0{}, xs0, cur);
        wait_vm<0>();
        wave_barrier_sync();
        if (i + 1 < nks) {
            issue_a(xs0, sb0 + i + 1, 0);
            load_raw(nxt, sb0 + i + 1);
        }
        compute(H1{}, xs1, cur);
    };
    issue_a(xs0, sb0, 0);
    load_raw(w0, sb0);
    for (int i = 0; i < nks; i += 2) {
        superblock(i, w0, w1);
        if (i + 1 >= nks) break;
        superblock(i + 1, w1, w0);
    }
    // lane (r, kq), register i: row m0 + 16 mt + 4 kq + i, column n0 + 16 nr + r
#pragma unroll
    for (int nr = 0; nr < NR; nr++) {
        const int n = n0 + 16 * nr + r;
        const float bn = !PART && BIAS && n < N ? __uint_as_float((uint32_t)bias[n] << 16) : 0.0f;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = m0 + 16 * mt + 4 * kq + i;
                if (m >= M || n >= N) continue;
                if constexpr (PART) {
                    part[((int64_t)s * M + m) * N + n] = acc[nr][mt][i];
                } else {
                    float t = acc[nr][mt][i];
                    if (BIAS) t = t + bn;
                    Y[(int64_t)m * N + n] = __builtin_bit_cast(uint16_t, (__bf16)t);
                }
            }
    }
}

// y = bf16(part[0] + part[1] + ... + part[S - 1] (+ bias)), four consecutive outputs per thread
template <bool BIAS>
__global__ __launch_bounds__(256) void gguf_panel_sum(const float* __restrict__ part, const uint16_t* __restrict__ bias,
                                                      uint16_t* __restrict__ Y, int64_t MN, int N, int S) {
    const int64_t i0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i0 >= MN) return;
    float t[4];
    // N % 4 == 0: MN % 4 == 0 and every slice starts 16-byte aligned; the four outputs go as one 8-byte store only
    // when Y itself is 8-byte aligned (a caller's view may start at any element)
    if ((N & 3) == 0 && (reinterpret_cast<uintptr_t>(Y) & 7) == 0) {
        float4 v = *reinterpret_cast<const float4*>(part + i0);
        t[0] = v.x; t[1] = v.y; t[2] = v.z; t[3] = v.w;
        for (int q = 1; q < S; q++) {
            v = *reinterpret_cast<const float4*>(part + (int64_t)q * MN + i0);
            t[0] = t[0] + v.x; t[1] = t[1] + v.y; t[2] = t[2] + v.z; t[3] = t[3] + v.w;
        }
        const int n = (int)(i0 % N);
        uint16_t o[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float y = t[e];
            if (BIAS) y = y + __uint_as_float((uint32_t)bias[n + e] << 16);
            o[e] = __builtin_bit_cast(uint16_t, (__bf16)y);
        }
        *reinterpret_cast<uint2*>(Y + i0) = make_uint2(o[0] | ((uint32_t)o[1] << 16), o[2] | ((uint32_t)o[3] << 16));
        return;
    }
    for (int e = 0; e < 4 && i0 + e < MN; e++) {
        float y = part[i0 + e];
        for (int q = 1; q < S; q++) y = y + part[(int64_t)q * MN + i0 + e];
        if (BIAS) y = y + __uint_as_float((uint32_t)bias[(i0 + e) % N] << 16);
        Y[i0 + e] = __builtin_bit_cast(uint16_t, (__bf16)y);
    }
}

// Split-K plan of an [M, K] x [N, K] product: rows per fragment group MT, super-blocks per slice KS, slices S, column
// tiles NT, and the workspace: a fixed block of kSplitCounters counters (the same place for every call, so calls of
// any shape can share one workspace), then S * M * N float32 partial sums.
static constexpr int kSplitCounters = 4096;     // column tiles: N <= 4096 * 128
static constexpr int64_t kSplitCounterBytes = 4 * kSplitCounters;

struct SplitPlan {
    int mt, ks, s, nt;
    int64_t counter_bytes, part_bytes;
    int64_t bytes() const { return counter_bytes + part_bytes; }
};

// Where the split form is the faster one (measured on MI355X against gemm_gguf_skinny, Q4_K / Q6_K, cold weights):
// at most 8 rows of a narrow, deep product (N <= 2048, K >= 8192, K >= 2 N), whose few-rows grid leaves CUs idle:
// 2048 x 8192 at 1 row 12.6 us against 17.1 (Q4_K), 16.3 against 20.3 (Q6_K). Wider products fill the chip with
// few-rows workgroups, which need no hand-over of partial sums (5120 x 13824 Q4_K at 1 row: 25.2 us against 30.9
// split; 3072 x 13824 Q6_K: 27.5 against 36.1); shallower ones gain nothing from more slices (1536 x 5120 Q4_K at 4
// rows: 9.8 against 11.5).
static constexpr int kSplitMaxRows = 8;

static bool split_takes(int64_t M, int64_t N, int64_t K) {
    return M >= 1 && M <= kSplitMaxRows && N >= 1 && N <= 2048 && K >= 8192 && K >= 2 * N;
}

static SplitPlan split_plan(int64_t M, int64_t N, int64_t K) {
    SplitPlan p{};
    p.mt = M <= 16 ? 1 : M <= 32 ? 2 : M <= 64 ? 4 : 8;
    p.nt = (int)((N + kSpRows - 1) / kSpRows);
    const int nsb = (int)(K / 256);
    // the widest slice (fewest partial sums) that still gives every CU a workgroup; LDS: MT * KS <= 8
    int ks = 8 / p.mt < 4 ? 8 / p.mt : 4;
    while (ks > 1 && (int64_t)p.nt * ((nsb + ks - 1) / ks) < 256) ks >>= 1;
    p.ks = ks;
    p.s = (nsb + ks - 1) / ks;
    p.counter_bytes = kSplitCounterBytes;
    p.part_bytes = (int64_t)p.s * M * N * 4;
    return p;
}

template <int QT, int MID, int MT, int KS>
static void launch_splitk_ks(const uint16_t* X, const uint8_t* W, const uint16_t* bias, uint16_t* Y, int M, int N,
                             int K, const SplitPlan& p, void* ws, hipStream_t st) {
    unsigned* counters = static_cast<unsigned*>(ws);
    float* part = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + p.counter_bytes);
    const dim3 grid((unsigned)(p.nt * p.s));
    if (bias)
        gemm_gguf_splitk<QT, MID, true, MT, KS><<<grid, 64 * kSpWaves, 0, st>>>(X, W, bias, Y, M, N, K, p.s, counters, part);
    else
        gemm_gguf_splitk<QT, MID, false, MT, KS><<<grid, 64 * kSpWaves, 0, st>>>(X, W, bias, Y, M, N, K, p.s, counters, part);
}

template <int QT, int MID, int MT>
static void launch_splitk_mt(const uint16_t* X, const uint8_t* W, const uint16_t* bias, uint16_t* Y, int M, int N,
                             int K, const SplitPlan& p, void* ws, hipStream_t st) {
    if constexpr (MT <= 2) {
        if (p.ks == 4) { launch_splitk_ks<QT, MID, MT, 4>(X, W, bias, Y, M, N, K, p, ws, st); return; }
    }
    if constexpr (MT <= 4) {
        if (p.ks == 2) { launch_splitk_ks<QT, MID, MT, 2>(X, W, bias, Y, M, N, K, p, ws, st); return; }
    }
    launch_splitk_ks<QT, MID, MT, 1>(X, W, bias, Y, M, N, K, p, ws, st);
}

template <int QT, int MID>
static void launch_splitk(const uint16_t* X, const uint8_t* W, const uint16_t* bias, uint16_t* Y, int M, int N, int K,
                          const SplitPlan& p, void* ws, hipStream_t st) {
    if (p.mt == 1) launch_splitk_mt<QT, MID, 1>(X, W, bias, Y, M, N, K, p, ws, st);
    else if (p.mt == 2) launch_splitk_mt<QT, MID, 2>(X, W, bias, Y, M, N, K, p, ws, st);
    else if (p.mt == 4) launch_splitk_mt<QT, MID, 4>(X, W, bias, Y, M, N, K, p, ws, st);
    else launch_splitk_mt<QT, MID, 8>(X, W, bias, Y, M, N, K, p, ws, st);
}

template <int QT>
static void launch_splitk_mid(int mid, const uint16_t* X, const uint8_t* W, const uint16_t* bias, uint16_t* Y, int M,
                              int N, int K, const SplitPlan& p, void* ws, hipStream_t st) {
    if (mid == WF_F16) launch_splitk<QT, WF_F16>(X, W, bias, Y, M, N, K, p, ws, st);
    else if (mid == WF_BF16) launch_splitk<QT, WF_BF16>(X, W, bias, Y, M, N, K, p, ws, st);
    else launch_splitk<QT, WF_F32>(X, W, bias, Y, M, N, K, p, ws, st);
}

// The whole-rows form (gemm_gguf_quad): one to three rows where the few-rows kernel's 32-row workgroups leave CUs
// idle (N < 8192: fewer than 256 of them), and for Q6_K, whose few-rows kernel waits on its raw loads, up to
// N < 16384 on 512 workgroups. Measured on MI355X against the few-rows kernel, Wan shapes, cold weights, per layer at
// one row: Q4_K 5120 x 5120 9.3 against 9.8 us, 5120 x 13824 18.6 against 24.3; Q5_K 10.0 against 11.2, 20.1 against
// 26.4; Q6_K 10.2 against 14.4, 23.8 against 37.0, 13824 x 5120 22.3 against 35.2 (512 workgroups). At 13824 x 5120
// the Q4_K / Q5_K few-rows kernel (432 workgroups) stays as fast or faster (Q4_K 17.5 against 18.2 on 512
// workgroups, 18.6 on 256). Q4_K / Q5_K blocks at 3 rows 79.0 / 85.5 against 82.5 / 92.9 us; at 4 rows the few-rows
// kernel's shared activation loads win (Q4_K 83.5 against 87.1). Q6_K keeps the whole-rows form up to four rows
// (block at 4 rows 114.6 against 132.7 us), as does Q8_0 (105 / 115 us at 3 / 4 rows against 143 with the
// few-rows kernel). A second group of four activation rows (two MFMAs per dequantised fragment) lost to the few-rows
// kernel at 5-8 rows for every format (Q8_0 block at 8 rows 168.9 against 124.0 us, Q6_K 168.9 against 123.3).
static constexpr int kQuadMaxRows = 3, kQuadMaxRowsQ6 = 4, kQuadMaxRowsQ8 = 4;
static_assert(kQuadMaxRows <= 4 && kQuadMaxRowsQ6 <= 4 && kQuadMaxRowsQ8 <= 4,
              "the whole-rows kernel takes 4 activation rows at most");

static bool quad_takes(int64_t M, int64_t N, int64_t K, int qtype) {
    const bool wide = qtype == 14 || qtype == 8;
    const int64_t ts = qtype == 12 ? 144 : qtype == 13 ? 176 : qtype == 14 ? 210 : 272;
    const int rows = qtype == 8 ? kQuadMaxRowsQ8 : qtype == 14 ? kQuadMaxRowsQ6 : kQuadMaxRows;
    // (weight and activation bytes both addressed by 32-bit buffer offsets)
    return M >= 1 && M <= rows && (N + 31) / 32 < (wide ? 512 : 256) && M * K * 2 < (1LL << 31) &&
           N * (K / 256) * ts < (1LL << 31);
}

template <int QT, int MID>
static void launch_quad(const uint16_t* X, const uint8_t* W, const uint16_t* bias, uint16_t* Y, int M, int N, int K,
                        hipStream_t st) {
    // 256 workgroups (one per CU) below 8192 rows, 512 (two per CU) up to 16384: at most kQdMaxQuads quads each
    const int G = std::min((N + 3) / 4, N >= 8192 ? 512 : 256);
    if (bias) gemm_gguf_quad<QT, MID, true><<<dim3(G), 64 * kQdWaves, 0, st>>>(X, W, bias, Y, M, N, K, G);
    else gemm_gguf_quad<QT, MID, false><<<dim3(G), 64 * kQdWaves, 0, st>>>(X, W, bias, Y, M, N, K, G);
}


#ifndef WF_SKINNY_NR1_MAX_N
#define WF_SKINNY_NR1_MAX_N 8191
#endif
static constexpr int kSkinnyNr1MaxN = WF_SKINNY_NR1_MAX_N, kSkinnyNr1MaxRows = 7;

template <int QT, int MID, int MT, int NR, int NW, bool AHEAD = false>
static void launch_skinny(const uint16_t* X, const uint8_t* W, const uint16_t* bias, uint16_t* Y, int M, int N, int K,
                          hipStream_t s) {
    const dim3 grid((unsigned)((N + 16 * NR - 1) / (16 * NR)));
    if (bias) gemm_gguf_skinny<QT, MID, true, MT, NR, NW, AHEAD><<<grid, 64 * NW, 0, s>>>(X, W, bias, Y, M, N, K);
    else gemm_gguf_skinny<QT, MID, false, MT, NR, NW, AHEAD><<<grid, 64 * NW, 0, s>>>(X, W, bias, Y, M, N, K);
}

// Q8_0's fused forms: the whole-rows form where it takes the shape, else the few-rows kernel up to 64 rows (its
// 12-byte block loads and d shared by a lane permute as in the whole-rows form; activations read per stage, which
// measured faster than one super-block ahead: 124.0 against 148.0 us at 8 rows). Wan block against the two-step flow
// (wf_dequant, then torch's GEMM), cold weights: 122 / 125 / 130 / 169 / 273 us at 5 / 9 / 16 / 32 / 64 rows against
// 304-337. With a workspace (or the no-alloc scratch) the panel form's rule takes Q8_0 as it takes the K-quants, at
// 33-64 rows and at 17-32 rows of deep products (Wan block at 48 / 64 rows 169 / 174 against 248 / 275 us, at 32 rows
// 160 against 171). Beyond 512 rows Q8_0 is left to the caller's two-step flow (WF_EUNSUPPORTED).
static bool q8_skinny_takes(int64_t M, int64_t N, int64_t K) {
    // (a workgroup's 32 weight rows addressed by 32-bit buffer offsets)
    return M >= 1 && M <= 64 && N >= 1 && 32 * (K / 256) * 272 < (1LL << 31);
}

// (the panel form takes Q8_0 at 65-512 rows, a wave's 32 weight rows in 32-bit buffer offsets as in the few-rows
// kernel; kPanelMaxRows)
static bool q8_takes(int64_t M, int64_t N, int64_t K) {
    return quad_takes(M, N, K, 8) || q8_skinny_takes(M, N, K) || (M > 64 && M <= 512 && q8_skinny_takes(1, N, K));
}

template <int MID>
static void launch_q8(const uint16_t* X, const uint8_t* W, const uint16_t* bias, uint16_t* Y, int M, int N, int K,
                      hipStream_t s) {
    if (quad_takes(M, N, K, 8)) launch_quad<8, MID>(X, W, bias, Y, M, N, K, s);
    else if (M <= 16) launch_skinny<8, MID, 1, 2, 8>(X, W, bias, Y, M, N, K, s);
    else if (M <= 32) launch_skinny<8, MID, 2, 2, 8>(X, W, bias, Y, M, N, K, s);
    else launch_skinny<8, MID, 4, 2, 8>(X, W, bias, Y, M, N, K, s);
}

static void run_gguf_q8(int mid, const void* x_bf16, const void* wq, const void* bias_bf16, void* out_bf16, int M,
                        int N, int K, hipStream_t s) {
    const uint16_t* X = static_cast<const uint16_t*>(x_bf16);
    const uint8_t* W = static_cast<const uint8_t*>(wq);
    const uint16_t* B = static_cast<const uint16_t*>(bias_bf16);
    uint16_t* Y = static_cast<uint16_t*>(out_bf16);
    if (mid == WF_F16) launch_q8<WF_F16>(X, W, B, Y, M, N, K, s);
    else if (mid == WF_BF16) launch_q8<WF_BF16>(X, W, B, Y, M, N, K, s);
    else launch_q8<WF_F32>(X, W, B, Y, M, N, K, s);
}

template <int QT, int MID, int VM, int VN, int WM, int WN>
static void launch_shape(const uint16_t* X, const uint8_t* W, const uint16_t* bias, uint16_t* Y, int M, int N, int K,
                         hipStream_t s) {
    constexpr int BM = VM * WM * 32, BN = VN * WN * 32;
    const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    if (bias) gemm_gguf_dl<QT, MID, true, VM, VN, WM, WN><<<dim3(tiles), 512, 0, s>>>(X, W, bias, Y, M, N, K);
    else gemm_gguf_dl<QT, MID, false, VM, VN, WM, WN><<<dim3(tiles), 512, 0, s>>>(X, W, bias, Y, M, N, K);
}

void run_gguf_tall(int mid, const void* x_bf16, const void* wq, const void* bias_bf16, void* out_bf16, int M, int N,
                   int K, hipStream_t s);   // gemm_gguf_tall.hip (Q6_K)

#ifndef WF_TALL_MIN_ROWS
#define WF_TALL_MIN_ROWS 1024
#endif
// Q6_K takes the 512 x 160 tiles (gemm_gguf_tall.hip) from this many rows, when they take no more modelled cycles than
// the 256-row tiles: half the dequantisation per MFMA, which pays for Q6_K's costlier raw loads (Wan block at 4096
// rows, MI355X: 2.06 against 2.29 ms). Q4_K and Q5_K keep the 256 x 320 tiles, as fast or faster there (Q5_K 1.89
// against 1.94 ms): the smaller dequantisation saves VALU work, but the twice-larger activation stage costs as much.
static constexpr int64_t kTallMinRows = WF_TALL_MIN_ROWS;

static int64_t rounds_x_area(int64_t M, int64_t N, int bm, int bn) {
    const int64_t tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    return (tiles + 255) / 256 * bm * bn;
}

static bool tall_takes(int64_t M, int64_t N, int qtype) {
    return qtype == 14 && M >= kTallMinRows &&
           rounds_x_area(M, N, 512, 160) <= std::min(rounds_x_area(M, N, 256, 320), rounds_x_area(M, N, 256, 256));
}

// 256 x 320 tiles (8 waves of 2 x 5 MFMA tiles; 4096 x 5120 outputs make exactly 256 tiles) or 256 x 256 (8 waves of
// 4 x 2), whichever takes fewer modelled cycles: whole rounds of 256 workgroups (one per CU) x tile area
template <int QT, int MID>
static void launch(const uint16_t* X, const uint8_t* W, const uint16_t* bias, uint16_t* Y, int M, int N, int K,
                   hipStream_t s) {
    // few rows: 32 weight rows per workgroup (two 16-row groups sharing each activation fragment)
    // Up to 8 rows the activations go one super-block ahead: 10-22 % faster than the per-stage reads (Wan shapes,
    // cold weights); from 9 rows on, their 16 distinct rows per fragment make it slower. Q6_K keeps the per-stage
    // reads at every row count: with its raw bytes through sk_load_q6w the 32-row, 8-wave form is the fastest one
    // (Wan shapes at 1-8 rows, per layer: 18.4 / 34.8 / 39.1 us against 20.3 / 37.2 / 47.4 for the 16-row, 4-wave
    // workgroups with activations ahead and the narrow loads).
    // Up to 7 rows of a Q6_K product narrower than 256 workgroups of 32 rows, 16 weight rows per workgroup (NR = 1):
    // more CUs wait on Q6_K's raw loads (Wan block at 5 / 7 rows 115.2 / 118.9 against 118.7 / 119.4 us, cold
    // weights, MI355X); from 8 rows the shared activation loads of 32-row workgroups win (120.0 against 122.1 us at 8,
    // 122.1 against 134.1 at 12, 126.2 against 147.6 at 16). For Q4_K / Q5_K the 64 CUs that then hold two workgroups
    // set the time (88 against 82 us at one row): their few-rows kernel is bound by the dequantisation's VALU work per
    // CU, which the split does not shrink.
    if (quad_takes(M, N, K, QT)) {
        launch_quad<QT, MID>(X, W, bias, Y, M, N, K, s);
        return;
    }
    if (M <= 8 && QT != 14) {
        launch_skinny<QT, MID, 1, 2, 8, true>(X, W, bias, Y, M, N, K, s);
        return;
    }
    if (M <= 16) {
        if (QT == 14 && M <= kSkinnyNr1MaxRows && N <= kSkinnyNr1MaxN)
            launch_skinny<QT, MID, 1, 1, 8>(X, W, bias, Y, M, N, K, s);
        else launch_skinny<QT, MID, 1, 2, 8>(X, W, bias, Y, M, N, K, s);
        return;
    }
    if (M <= 32) { launch_skinny<QT, MID, 2, 2, 8>(X, W, bias, Y, M, N, K, s); return; }
    if (M <= 64) { launch_skinny<QT, MID, 4, 2, 8>(X, W, bias, Y, M, N, K, s); return; }
    auto cost = [&](int bn) {
        const int64_t tiles = (int64_t)((M + 255) / 256) * ((N + bn - 1) / bn);
        return (tiles + 255) / 256 * bn;
    };
    if (cost(320) < cost(256)) launch_shape<QT, MID, 4, 2, 2, 5>(X, W, bias, Y, M, N, K, s);
    else launch_shape<QT, MID, 2, 4, 4, 2>(X, W, bias, Y, M, N, K, s);
}

template <int QT>
static void launch_mid(int mid, const uint16_t* X, const uint8_t* W, const uint16_t* bias, uint16_t* Y, int M,
                       int N, int K, hipStream_t s) {
    if (mid == WF_F16) launch<QT, WF_F16>(X, W, bias, Y, M, N, K, s);
    else if (mid == WF_BF16) launch<QT, WF_BF16>(X, W, bias, Y, M, N, K, s);
    else launch<QT, WF_F32>(X, W, bias, Y, M, N, K, s);
}

}  // namespace wf

namespace wf {
// argument checks shared by the entry points; WF_OK with M == 0 or N == 0 means nothing to do
static int check_gguf(const char* who, const void* x_bf16, int64_t M, int64_t K, const void* wq, int64_t wq_bytes,
                      int qtype, int64_t N, const void* bias_bf16, const void* out_bf16, int mid_dt) {
    if (qtype != 12 && qtype != 13 && qtype != 14 && qtype != 8) {
        set_error("%s: GGML type %d is not handled (Q4_K, Q5_K, Q6_K; Q8_0 at 1-512 rows)", who, qtype);
        return WF_EUNSUPPORTED;
    }
    if (mid_dt < 0 || mid_dt > 2) { set_error("%s: dequant dtype %d", who, mid_dt); return WF_EUNSUPPORTED; }
    if (M < 0 || N < 0 || K <= 0) {
        set_error("%s: M, N, K = %lld, %lld, %lld", who, (long long)M, (long long)N, (long long)K);
        return WF_EINVAL;
    }
    if (K % 256) { set_error("%s: K = %lld is not a multiple of 256", who, (long long)K); return WF_EUNSUPPORTED; }
    const int ts = qtype == 12 ? 144 : qtype == 13 ? 176 : qtype == 14 ? 210 : 272;   // bytes per 256 values
    if (wq_bytes != N * (K / 256) * ts) {
        set_error("%s: %lld weight bytes for [%lld, %lld]", who, (long long)wq_bytes, (long long)N, (long long)K);
        return WF_EUNSUPPORTED;
    }
    if (M == 0 || N == 0) return WF_OK;
    if (!x_bf16 || !wq || !out_bf16) { set_error("%s: null pointer", who); return WF_EINVAL; }
    if (!aligned(x_bf16, 16) || !aligned(wq, 16) || !aligned(out_bf16, 2) || (bias_bf16 && !aligned(bias_bf16, 2))) {
        set_error("%s: x and the weight blocks must be 16-byte aligned", who);
        return WF_EUNSUPPORTED;
    }
    if (M >= (1LL << 31) || N >= (1LL << 31) || K >= (1LL << 31)) {
        set_error("%s: sizes too large", who);
        return WF_EUNSUPPORTED;
    }
    // a workgroup's activation rows (up to 512) through one buffer resource of at most 2^31 - 1 bytes
    if (K > (1LL << 20)) {
        set_error("%s: rows of %lld values, more than the 1048576 the kernels address", who, (long long)K);
        return WF_EUNSUPPORTED;
    }
    if (qtype == 8 && !q8_takes(M, N, K)) {
        set_error("%s: Q8_0 is fused at 1-512 rows only (%lld x %lld here)", who, (long long)M, (long long)N);
        return WF_EUNSUPPORTED;
    }
    return WF_OK;
}

// Medium row counts: the panel kernel's plan. MT = 2 up to 32 rows, 4 up to 64, else 8 (128 activation rows per
// panel); slices S so that NT x MTI x S >= 256 workgroups, at least two super-blocks each, and partial sums no larger
// than max_part bytes (0: one slice, no workspace). Up to 512 rows it beats the tiled kernel (Wan block, Q4_K, one
// slice: 563 against 856 us at 128 rows, 684 against 887 at 512); from 1024 rows the tiled kernel's 256 x 320 tiles,
// which dequantise each weight value once per 256 rows instead of once per 128, are faster (909 against 1334 us).
static constexpr int64_t kPanelMaxRows = 512;
static_assert(kPanelMaxRows == 512, "q8_takes states the panel form's rows");
static constexpr int64_t kPanelMinRowsWs = 17;       // fewest rows the panel form takes with a workspace

// Without a workspace (one slice) the panel form takes 65-512 rows.
static bool panel_takes(int64_t M) { return M > 64 && M <= kPanelMaxRows; }

// With a workspace (K in slices) it also takes 33-64 rows, and 17-32 rows of a deep product (K >= 2 N), where the
// few-rows kernel's one workgroup per 32 weight rows leaves CUs idle or runs long (measured on MI355X, Wan shapes,
// warmed, with the workspace, per layer: Q4_K 5120 x 13824 at 32 rows 34.8 against 38.0 us, at 64 rows 45.1 against
// 70.0; Q6_K 43.9 against 46.5 at 32 rows, 47.1 against 62.5 at 40). Shallow products keep the few-rows kernel up
// to 32 rows (Q4_K 5120 x 5120 at 32 rows 16.5 against 17.0; Q6_K, its raw words shifted where dequantised, 18.8
// against 24.0, 13824 x 5120 36.3 against 47.4, and 16.4 against 22.9 at 17 rows). From 33 rows the panel form
// takes them too: Q6_K's few-rows kernel is still 3-11 % faster on them at 40-48 rows but not at 64, and the deep
// product's panel gain (25-30 %) is larger.
static bool panel_takes_ws(int64_t M, int64_t N, int64_t K) {
    if (M > 32) return M <= kPanelMaxRows;
    return M >= kPanelMinRowsWs && K >= 2 * N;
}

struct PanelPlan {
    int mt, mti, nt, ks, s;
    int64_t part_bytes;
};

// Workgroups the slices aim for: 256 (one per CU), or 512 (two per CU, which the 64 KiB ring allows) where that
// measured faster on MI355X (Wan shapes, warmed, with the workspace): from 385 rows (Q4_K block at 512 rows 473
// against 495 us, Q6_K 739 against 818) and for Q6_K up to 128 rows (254 against 268 at 128); elsewhere the extra
// partial sums cost more than the second workgroup gains (Q4_K 303 against 289 at 256 rows).
static int panel_target(int64_t M, int qtype) { return M > 384 || (qtype == 14 && M <= 128) ? 512 : 256; }

static PanelPlan panel_plan(int64_t M, int64_t N, int64_t K, int64_t max_part, int qtype) {
    PanelPlan p{};
    // (Q8_0's raw bytes, 24 registers per row group and set against the K-quants' 12, leave 128-row panels short of
    // registers at two waves per SIMD: they spilled 60; its panels take 64 rows)
    p.mt = M <= 32 ? 2 : M <= 64 || qtype == 8 ? 4 : 8;
    p.mti = (int)((M + 16 * p.mt - 1) / (16 * p.mt));
    p.nt = (int)((N + kPnRows - 1) / kPnRows);
    const int nsb = (int)(K / 256);
    const int64_t tiles = (int64_t)p.nt * p.mti;
    const int64_t target = panel_target(M, qtype);
    int s = (int)std::min<int64_t>((target + tiles - 1) / tiles, std::max(1, nsb / 2));
    while (s > 1 && (int64_t)s * M * N * 4 > max_part) s--;
    p.ks = (nsb + s - 1) / s;
    p.s = (nsb + p.ks - 1) / p.ks;
    p.part_bytes = p.s > 1 ? (int64_t)p.s * M * N * 4 : 0;
    return p;
}

template <int QT, int MID, int MT>
static void launch_panel_mt(const uint16_t* X, const uint8_t* W, const uint16_t* bias, uint16_t* Y, int M, int N,
                            int K, const PanelPlan& p, void* ws, hipStream_t st) {
    const dim3 grid((unsigned)(p.nt * p.mti * p.s));
    float* part = static_cast<float*>(ws);
    if (p.s > 1) {
        gemm_gguf_panel<QT, MID, false, MT, true><<<grid, 64 * kPnWaves, 0, st>>>(X, W, bias, Y, part, M, N, K, p.nt,
                                                                                   p.mti, p.ks);
        const int64_t MN = (int64_t)M * N;
        const dim3 g2((unsigned)((MN + 1023) / 1024));
        if (bias) gguf_panel_sum<true><<<g2, 256, 0, st>>>(part, bias, Y, MN, N, p.s);
        else gguf_panel_sum<false><<<g2, 256, 0, st>>>(part, bias, Y, MN, N, p.s);
    } else if (bias) {
        gemm_gguf_panel<QT, MID, true, MT, false><<<grid, 64 * kPnWaves, 0, st>>>(X, W, bias, Y, part, M, N, K, p.nt,
                                                                                   p.mti, p.ks);
    } else {
        gemm_gguf_panel<QT, MID, false, MT, false><<<grid, 64 * kPnWaves, 0, st>>>(X, W, bias, Y, part, M, N, K, p.nt,
                                                                                    p.mti, p.ks);
    }
}

template <int QT>
static void launch_panel(int mid, const uint16_t* X, const uint8_t* W, const uint16_t* bias, uint16_t* Y, int M,
                         int N, int K, const PanelPlan& p, void* ws, hipStream_t st) {
    if (p.mt == 2) {
        if (mid == WF_F16) launch_panel_mt<QT, WF_F16, 2>(X, W, bias, Y, M, N, K, p, ws, st);
        else if (mid == WF_BF16) launch_panel_mt<QT, WF_BF16, 2>(X, W, bias, Y, M, N, K, p, ws, st);
        else launch_panel_mt<QT, WF_F32, 2>(X, W, bias, Y, M, N, K, p, ws, st);
    } else if (p.mt == 4 || QT == 8) {                // (Q8_0: 64-row panels at most, panel_plan)
        if (mid == WF_F16) launch_panel_mt<QT, WF_F16, 4>(X, W, bias, Y, M, N, K, p, ws, st);
        else if (mid == WF_BF16) launch_panel_mt<QT, WF_BF16, 4>(X, W, bias, Y, M, N, K, p, ws, st);
        else launch_panel_mt<QT, WF_F32, 4>(X, W, bias, Y, M, N, K, p, ws, st);
    } else if constexpr (QT != 8) {
        if (mid == WF_F16) launch_panel_mt<QT, WF_F16, 8>(X, W, bias, Y, M, N, K, p, ws, st);
        else if (mid == WF_BF16) launch_panel_mt<QT, WF_BF16, 8>(X, W, bias, Y, M, N, K, p, ws, st);
        else launch_panel_mt<QT, WF_F32, 8>(X, W, bias, Y, M, N, K, p, ws, st);
    }
}

static void run_gguf_panel(int qtype, int mid_dt, const void* x_bf16, const void* wq, const void* bias_bf16,
                           void* out_bf16, int M, int N, int K, const PanelPlan& p, void* ws, hipStream_t s) {
    const uint16_t* X = static_cast<const uint16_t*>(x_bf16);
    const uint8_t* W = static_cast<const uint8_t*>(wq);
    const uint16_t* B = static_cast<const uint16_t*>(bias_bf16);
    uint16_t* Y = static_cast<uint16_t*>(out_bf16);
    if (qtype == 12) launch_panel<12>(mid_dt, X, W, B, Y, M, N, K, p, ws, s);
    else if (qtype == 13) launch_panel<13>(mid_dt, X, W, B, Y, M, N, K, p, ws, s);
    else if (qtype == 8) launch_panel<8>(mid_dt, X, W, B, Y, M, N, K, p, ws, s);
    else launch_panel<14>(mid_dt, X, W, B, Y, M, N, K, p, ws, s);
}

static void run_gguf(int qtype, int mid_dt, const void* x_bf16, const void* wq, const void* bias_bf16, void* out_bf16,
                     int M, int N, int K, hipStream_t s) {
    const uint16_t* X = static_cast<const uint16_t*>(x_bf16);
    const uint8_t* W = static_cast<const uint8_t*>(wq);
    const uint16_t* B = static_cast<const uint16_t*>(bias_bf16);
    uint16_t* Y = static_cast<uint16_t*>(out_bf16);
    if (panel_takes(M)) {                             // without a workspace: one slice
        run_gguf_panel(qtype, mid_dt, x_bf16, wq, bias_bf16, out_bf16, M, N, K, panel_plan(M, N, K, 0, qtype), nullptr,
                       s);
        return;
    }
    if (tall_takes(M, N, qtype)) {
        run_gguf_tall(mid_dt, x_bf16, wq, bias_bf16, out_bf16, M, N, K, s);
        return;
    }
    if (qtype == 12) launch_mid<12>(mid_dt, X, W, B, Y, M, N, K, s);
    else if (qtype == 13) launch_mid<13>(mid_dt, X, W, B, Y, M, N, K, s);
    else launch_mid<14>(mid_dt, X, W, B, Y, M, N, K, s);
}

static void run_gguf_split(int qtype, int mid_dt, const void* x_bf16, const void* wq, const void* bias_bf16,
                           void* out_bf16, int M, int N, int K, const SplitPlan& p, void* ws, hipStream_t s) {
    const uint16_t* X = static_cast<const uint16_t*>(x_bf16);
    const uint8_t* W = static_cast<const uint8_t*>(wq);
    const uint16_t* B = static_cast<const uint16_t*>(bias_bf16);
    uint16_t* Y = static_cast<uint16_t*>(out_bf16);
    if (qtype == 12) launch_splitk_mid<12>(mid_dt, X, W, B, Y, M, N, K, p, ws, s);
    else if (qtype == 13) launch_splitk_mid<13>(mid_dt, X, W, B, Y, M, N, K, p, ws, s);
    else launch_splitk_mid<14>(mid_dt, X, W, B, Y, M, N, K, p, ws, s);
}
}  // namespace wf

extern "C" int wf_linear_gguf(const void* x_bf16, int64_t M, int64_t K, const void* wq, int64_t wq_bytes,
                              int qtype, int64_t N, const void* bias_bf16, void* out_bf16, int mid_dt,
                              void* stream) {
    using namespace wf;
    const int rc = check_gguf("wf_linear_gguf", x_bf16, M, K, wq, wq_bytes, qtype, N, bias_bf16, out_bf16, mid_dt);
    if (rc != WF_OK || M == 0 || N == 0) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (qtype == 8 && M <= 64) run_gguf_q8(mid_dt, x_bf16, wq, bias_bf16, out_bf16, (int)M, (int)N, (int)K, s);
    else run_gguf(qtype, mid_dt, x_bf16, wq, bias_bf16, out_bf16, (int)M, (int)N, (int)K, s);
    WF_LAUNCH_CHECK("wf_linear_gguf launch");
    return WF_OK;
}

extern "C" int wf_linear_gguf_workspace(int64_t M, int64_t N, int64_t K, int64_t* bytes) {
    using namespace wf;
    if (!bytes) { set_error("wf_linear_gguf_workspace: null out-pointer"); return WF_EINVAL; }
    *bytes = 0;
    if (M < 0 || N < 0 || K <= 0 || K % 256) { set_error("wf_linear_gguf_workspace: M, N, K"); return WF_EINVAL; }
    // the format is not known here: the largest need over them (Q6_K's panels take more slices up to 128 rows)
    if (split_takes(M, N, K)) *bytes = split_plan(M, N, K).bytes();
    else if (panel_takes_ws(M, N, K)) {
        const int64_t part = std::max({panel_plan(M, N, K, INT64_MAX, 12).part_bytes,
                                       panel_plan(M, N, K, INT64_MAX, 14).part_bytes,
                                       panel_plan(M, N, K, INT64_MAX, 8).part_bytes});
        if (part > 0) *bytes = kSplitCounterBytes + part;   // the split form's counters stay untouched
    }
    return WF_OK;
}

extern "C" int wf_linear_gguf_ws(const void* x_bf16, int64_t M, int64_t K, const void* wq, int64_t wq_bytes,
                                 int qtype, int64_t N, const void* bias_bf16, void* out_bf16, int mid_dt,
                                 void* workspace, int64_t workspace_bytes, void* stream) {
    using namespace wf;
    const int rc = check_gguf("wf_linear_gguf_ws", x_bf16, M, K, wq, wq_bytes, qtype, N, bias_bf16, out_bf16, mid_dt);
    if (rc != WF_OK || M == 0 || N == 0) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // Q8_0 up to 64 rows: the whole-rows or few-rows form (no workspace) unless the panel form's rule below takes it
    if (qtype == 8 && M <= 64 && !(panel_takes_ws(M, N, K) && panel_plan(M, N, K, INT64_MAX, 8).s > 1)) {
        run_gguf_q8(mid_dt, x_bf16, wq, bias_bf16, out_bf16, (int)M, (int)N, (int)K, s);
        WF_LAUNCH_CHECK("wf_linear_gguf_ws launch");
        return WF_OK;
    }
    // up to 64 rows the panel form runs only in more than one slice (in one, the few-rows kernel is faster)
    const bool panel = !split_takes(M, N, K) && panel_takes_ws(M, N, K) &&
                       (panel_takes(M) || panel_plan(M, N, K, INT64_MAX, qtype).s > 1);
    if (panel) {
        // the panel form's partial sums go past the split form's counters, which must stay zero between calls (one
        // workspace serves calls of every shape and form on a stream)
        const PanelPlan p = panel_plan(M, N, K, INT64_MAX, qtype);
        void* part = nullptr;
        if (p.part_bytes > 0) {
            const int64_t need = kSplitCounterBytes + p.part_bytes;
            if (!workspace || !aligned(workspace, 256) || workspace_bytes < need) {
                set_error("wf_linear_gguf_ws: a 256-byte aligned workspace of %lld bytes is needed (given %lld)",
                          (long long)need, (long long)workspace_bytes);
                return WF_EINVAL;
            }
            part = static_cast<uint8_t*>(workspace) + kSplitCounterBytes;
        }
        run_gguf_panel(qtype, mid_dt, x_bf16, wq, bias_bf16, out_bf16, (int)M, (int)N, (int)K, p, part, s);
    } else if (!split_takes(M, N, K)) {
        run_gguf(qtype, mid_dt, x_bf16, wq, bias_bf16, out_bf16, (int)M, (int)N, (int)K, s);
    } else {
        const SplitPlan p = split_plan(M, N, K);
        if (!workspace || !aligned(workspace, 256) || workspace_bytes < p.bytes()) {
            set_error("wf_linear_gguf_ws: a 256-byte aligned workspace of %lld bytes is needed (given %lld)",
                      (long long)p.bytes(), (long long)workspace_bytes);
            return WF_EINVAL;
        }
        run_gguf_split(qtype, mid_dt, x_bf16, wq, bias_bf16, out_bf16, (int)M, (int)N, (int)K, p, workspace, s);
    }
    WF_LAUNCH_CHECK("wf_linear_gguf_ws launch");
    return WF_OK;
}

// ------------------------------------------------------------------------------ the allocation-free entry point
// wf_linear_gguf_noalloc: wf_linear_gguf_ws with the split form's counters and partial sums in `scratch`, device
// memory the library holds from load time (one copy per GPU, until the process ends), so the call allocates nothing.
// In host code `scratch` names a host-side stand-in; its device address comes from hipGetSymbolAddress, looked up once
// per device with that device current, and only that address is handed to kernels.
namespace wf {
static constexpr int64_t kScratchBytes = (int64_t)16 << 20;     // counters (16 KiB) + partial sums
}  // namespace wf

static __device__ __align__(256) uint8_t scratch[wf::kScratchBytes];

namespace wf {
static constexpr int kMaxDevices = 64;
static std::once_flag g_scratch_once[kMaxDevices];
static void* g_scratch_ptr[kMaxDevices];
static hipError_t g_scratch_err[kMaxDevices];

// the device address of `scratch` on the current device
static int scratch_address(void** out) {
    int dev = -1;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) { set_error("wf_linear_gguf_noalloc: device %d", dev); return WF_EUNSUPPORTED; }
    std::call_once(g_scratch_once[dev], [dev] {
        void* p = nullptr;
        g_scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        g_scratch_ptr[dev] = g_scratch_err[dev] == hipSuccess ? p : nullptr;
    });
    if (g_scratch_err[dev] != hipSuccess) return hip_fail(g_scratch_err[dev], "hipGetSymbolAddress(scratch)");
    *out = g_scratch_ptr[dev];
    return WF_OK;
}

// zeroes n 32-bit words (the split form's counters) on the stream: a kernel, not a memset, so the call can be
// captured into a graph
__global__ __launch_bounds__(256) void clear_words(unsigned* __restrict__ p, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0u;
}
}  // namespace wf

extern "C" int wf_linear_gguf_noalloc(const void* x_bf16, int64_t M, int64_t K, const void* wq, int64_t wq_bytes,
                                      int qtype, int64_t N, const void* bias_bf16, void* out_bf16, int mid_dt,
                                      void* stream) {
    using namespace wf;
    const int rc = check_gguf("wf_linear_gguf_noalloc", x_bf16, M, K, wq, wq_bytes, qtype, N, bias_bf16, out_bf16,
                              mid_dt);
    if (rc != WF_OK || M == 0 || N == 0) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // Q8_0 up to 64 rows: the whole-rows or few-rows form (no scratch) unless the panel form's rule below takes it
    if (qtype == 8 && M <= 64 &&
        !(panel_takes_ws(M, N, K) && panel_plan(M, N, K, kScratchBytes - kSplitCounterBytes, 8).s > 1)) {
        run_gguf_q8(mid_dt, x_bf16, wq, bias_bf16, out_bf16, (int)M, (int)N, (int)K, s);
        WF_LAUNCH_CHECK("wf_linear_gguf_noalloc launch");
        return WF_OK;
    }
    // (up to 64 rows only when the scratch holds more than one slice: in one slice the few-rows kernel is faster)
    if (!split_takes(M, N, K) && panel_takes_ws(M, N, K) &&
        (panel_takes(M) || panel_plan(M, N, K, kScratchBytes - kSplitCounterBytes, qtype).s > 1)) {
        // the panel form's partial sums in the scratch array, as many slices as fit there
        const PanelPlan p = panel_plan(M, N, K, kScratchBytes - kSplitCounterBytes, qtype);
        void* part = nullptr;
        if (p.part_bytes > 0) {
            void* ws = nullptr;
            const int src = scratch_address(&ws);
            if (src != WF_OK) return src;
            part = static_cast<uint8_t*>(ws) + kSplitCounterBytes;
        }
        run_gguf_panel(qtype, mid_dt, x_bf16, wq, bias_bf16, out_bf16, (int)M, (int)N, (int)K, p, part, s);
    } else if (!split_takes(M, N, K)) {
        run_gguf(qtype, mid_dt, x_bf16, wq, bias_bf16, out_bf16, (int)M, (int)N, (int)K, s);
    } else {
        const SplitPlan p = split_plan(M, N, K);
        if (p.bytes() > kScratchBytes) {
            set_error("wf_linear_gguf_noalloc: [%lld, %lld] x [%lld, %lld] needs %lld bytes of scratch, more than the "
                      "%lld the library holds (wf_linear_gguf_ws takes a workspace of any size)", (long long)M,
                      (long long)K, (long long)N, (long long)K, (long long)p.bytes(), (long long)kScratchBytes);
            return WF_EUNSUPPORTED;
        }
        void* ws = nullptr;
        const int src = scratch_address(&ws);
        if (src != WF_OK) return src;
        clear_words<<<dim3((kSplitCounters + 255) / 256), 256, 0, s>>>(static_cast<unsigned*>(ws), kSplitCounters);
        run_gguf_split(qtype, mid_dt, x_bf16, wq, bias_bf16, out_bf16, (int)M, (int)N, (int)K, p, ws, s);
    }
    WF_LAUNCH_CHECK("wf_linear_gguf_noalloc launch");
    return WF_OK;
}
