// Fused Q6_K dequant + bf16 GEMM for many activation rows: 512 x 160 output tiles, so that each dequantised weight
// value feeds 512 rows of MACs -- half the dequantisation work per MFMA of gemm_gguf_dl's 256-row tiles, which pays
// for Q6_K's costlier raw loads (its 210-byte blocks are 2-byte aligned). y[m, n] = bf16(sum_k x[m, k] * W[n, k]
// (+ bias[n])), W dequantised with the reference's rounding chain (MID, then bf16 -- enhancers/gguf_dequant.py:
// 213-224,250), float32 accumulation.
//
// 8 waves, two per SIMD, each a 64 x 160 slab of the tile (2 x 5 MFMA tiles of v_mfma_f32_32x32x16_bf16), K in
// stages of 32 values:
//  * activations: two LDS slots of a stage pair (512 rows x 128 bytes, K values 64 p .. 64 p + 63), copied global ->
//    LDS by the load unit (buffer_load ... lds) as whole 128-byte lines (chunks swizzled by swz8), eight 1 KiB
//    instructions (8 rows each) per wave per pair; pair p + 1 is issued at the first stage of pair p (the
//    vector-memory return path pays per cache line touched, so 64-byte half-line stages cost it twice the work);
//  * weight: a 3-slot LDS ring of 160 rows x 32 bf16, dequantised by the threads from raw bytes loaded a step
//    ahead -- thread t takes 8 values (a quarter of the stage's 32-value sub-block) of row t / 4, and the threads of
//    waves 0-3 (one per SIMD) also 4 values of row 128 + t / 8 -- and written into the slot of stage s + 2 during s.
// The loop runs whole super-blocks (8 stages), so a stage's sub-block index is a compile-time constant and raw bytes
// shared by several stages of a super-block are loaded once (the step is described at its lambda). Stages at or past K
// are still issued (reads land in slots never read, or read as zeros past the buffers), which keeps every wait exact.
// 4096 x 5120 outputs make exactly 256 tiles (one per CU).

#include "gguf_tile.h"

namespace wf {

typedef uint32_t u32x3t __attribute__((ext_vector_type(3)));

// raw bytes of an 8-value task: the ql and qh pieces as the 12-byte windows that hold them, and the pieces' byte
// offset in their windows (the same for both) in bits
struct Q6Raw8 { u32x3t ql, qh; uint32_t sh, sc, d; };

// the 12-byte window of 8 bytes at an even offset o: one load from the aligned-down dword (the window [o & ~3, +12)
// ends at most 4 bytes past o + 8, inside the block for every piece loaded here). The 8 bytes are funnel-shifted out
// of it where they are dequantised, after the wait for the load: a shift right behind the load would make the wave
// wait for it there.
__device__ __forceinline__ u32x3t ld8_window(__amdgpu_buffer_rsrc_t r, uint32_t o) {
    return __builtin_bit_cast(u32x3t, __builtin_amdgcn_raw_buffer_load_b96(r, o & ~3u, 0, 0));
}

// Raw bytes of values [8 e, 8 e + 8) of sub-block G of the Q6_K super-block at byte offset b, at phase G, v0 = 32 G +
// 8 e: ql[64 (G / 4) + 32 (G % 2) + 8 e ..] (nibble (G % 4) / 2) every phase, qh[128 + 32 (G / 4) + 8 e ..] (bits
// 2 (G % 4)) once per four phases, the scale byte 192 + 2 G + e / 2 every phase, d at 208 once per super-block (the
// caller loads the phases of a super-block in order into the same Q6Raw8)
template <int G>
__device__ __forceinline__ void q6_load8(__amdgpu_buffer_rsrc_t r, uint32_t b, int e, Q6Raw8& w) {
    constexpr uint32_t hh = G >> 2;
    w.ql = ld8_window(r, b + 64 * hh + 32 * (G & 1) + 8 * e);
    if constexpr ((G & 3) == 0) w.qh = ld8_window(r, b + 128 + 32 * hh + 8 * e);
    w.sh = (b & 3u) * 8u;                              // (both pieces sit a multiple of 4 bytes past b)
    w.sc = __builtin_amdgcn_raw_buffer_load_b8(r, b + 192 + 2 * G + (e >> 1), 0, 0);
    if constexpr (G == 0) w.d = __builtin_amdgcn_raw_buffer_load_b16(r, b + 208, 0, 0);
}

// the 8 values as 4 packed bf16 pairs (values 2i, 2i + 1 in o[i]): x = R_MID(R_MID(d * sc) * (q - 32)), then bf16
template <int MID, int g>
__device__ __forceinline__ void q6_dequant8(const Q6Raw8& w, uint32_t (&o)[4]) {
    const uint32_t ns = 4u * (uint32_t)((g & 3) >> 1), hs = 2u * (uint32_t)(g & 3);
    const uint2 ql = funnel8(w.ql[0], w.ql[1], w.ql[2], w.sh), qh = funnel8(w.qh[0], w.qh[1], w.qh[2], w.sh);
    uint32_t code[2];
    code[0] = ((ql.x >> ns) & 0x0f0f0f0fu) | (((qh.x >> hs) & 0x03030303u) << 4);
    code[1] = ((ql.y >> ns) & 0x0f0f0f0fu) | (((qh.y >> hs) & 0x03030303u) << 4);
    const int sc = (int8_t)(w.sc & 0xffu);
    const uint32_t dbits = w.d & 0xffffu;
    if constexpr (MID == WF_F16) {
        const _Float16 ds1 = __builtin_bit_cast(_Float16, (uint16_t)dbits) * (_Float16)(float)sc;
        h2 ds;
        ds[0] = ds1;
        ds[1] = ds1;
        const h2 off = h2s(-1056.0f);                 // (1024 + code) - 1056 = code - 32, exact
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const h2 v0 = ds * (biased_lo(code[i]) + off), v1 = ds * (biased_hi(code[i]) + off);
            o[2 * i] = pack_bf16((float)v0[0], (float)v0[1]);
            o[2 * i + 1] = pack_bf16((float)v1[0], (float)v1[1]);
        }
    } else {
        const float ds = round_to<MID>(round_to<MID>(f16_bits_to_f32(dbits)) * (float)sc);
#pragma unroll
        for (int i = 0; i < 2; i++) {
            float v[4];
#pragma unroll
            for (int k = 0; k < 4; k++) v[k] = round_to<MID>(ds * (float)((int)byte_of(code[i], k) - 32));
            o[2 * i] = pack_bf16(v[0], v[1]);
            o[2 * i + 1] = pack_bf16(v[2], v[3]);
        }
    }
}

constexpr int kTallBM = 512, kTallBN = 160;

template <int MID, bool BIAS>
__global__ __launch_bounds__(512) void gemm_gguf_tall(const uint16_t* __restrict__ X, const uint8_t* __restrict__ W,
                                                      const uint16_t* __restrict__ bias, uint16_t* __restrict__ Y,
                                                      int M, int N, int K) {
    constexpr int BM = kTallBM, BN = kTallBN, WM = 2, WN = 5;
    constexpr int QT = 14, TS = GGUFTs<QT>::TS;
    constexpr int IXP = BM / 8 / 8;                    // activation DMA instructions per wave per stage pair
    constexpr int WSLOT = BN * 4;                      // uint4 per weight slot
    __shared__ uint4 xp0[BM * 8], xp1[BM * 8];
    __shared__ uint4 wring[3 * WSLOT];
    const int ntm = (M + BM - 1) / BM, ntn = (N + BN - 1) / BN;
    int tm, tn;
    tile_order(blockIdx.x, ntm * ntn, ntm, ntn, tm, tn);
    // (the tile order's divisions run on the vector unit: its results go back to scalar registers here, or the
    // compiler keeps the buffer resources in vector registers and loops over lanes around every load)
    const int m0 = __builtin_amdgcn_readfirstlane(tm * BM), n0 = __builtin_amdgcn_readfirstlane(tn * BN);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nk = K / 32;
    const uint32_t row_bytes = (uint32_t)(K / 256) * TS;
    const __amdgpu_buffer_rsrc_t rx = tile_rsrc(X + (int64_t)m0 * K, (int64_t)(M - m0) * K * 2);
    const __amdgpu_buffer_rsrc_t rw = tile_rsrc(W + (int64_t)n0 * row_bytes, (int64_t)(N - n0) * row_bytes);
    // a pair DMA instruction copies 8 rows x 128 bytes (stages 2p and 2p + 1: whole cache lines); lane l writes LDS
    // slot l % 8 of row r = 8 run + l / 8, which holds chunk swz8(r, l % 8) of the row (swz8 is its own inverse). The
    // swizzle depends on r's bits 0-3: on l / 8, and through bit 3 on the run's parity, which flips bit 2 of the chunk
    // (bit 6 of the byte offset; the row part, a multiple of 2 K bytes, has bits 0-8 clear): xlane ^ 64 for odd runs
    const uint32_t xlane = (uint32_t)(lane >> 3) * (uint32_t)K * 2u + 16u * (uint32_t)swz8(lane >> 3, lane & 7);
    const uint32_t xlane_odd = xlane ^ 64u;
    // (the wave-uniform part of each offset is summed in a scalar register at each issue: kept apart from the lane
    // part, the compiler would hold IXP lane offsets across the loop and spill them)
    auto issue_pair = [&](uint4* st, int p) {
#pragma unroll
        for (int q = 0; q < IXP; q++) {
            const int run = wave * IXP + q;                // IXP even: run parity = q parity
            const uint32_t sofs = __builtin_amdgcn_readfirstlane((uint32_t)(run * 8) * (uint32_t)K * 2u + (uint32_t)p * 128u);
            lds_dma16(rx, st + 64 * run, (q & 1 ? xlane_odd : xlane) + sofs);
        }
    };
    // dequantisation tasks: 8 values (e = t % 4) of row t / 4; waves 0-3 also 4 values (qq = t % 8) of row
    // 128 + t / 8
    const int e8 = tid & 3, wr = tid >> 2;
    const int qq = tid & 7, wr2 = 128 + ((tid >> 3) & 31);
    const bool quarter = wave < 4;
    const uint32_t wbase = (uint32_t)wr * row_bytes, wbase2 = (uint32_t)wr2 * row_bytes;
    auto blk = [&](uint32_t base, int kt) { return base + (uint32_t)(kt >> 3) * TS; };
    const int wslot8 = wr * 4 + swz4(wr, e8);
    const int wslot4 = (wr2 * 4 + swz4(wr2, qq >> 1)) * 2 + (qq & 1);      // in 8-byte units
    Q6Raw8 w1;
    QRawQ<QT> w2;
    auto wload = [&](auto G, int kt) {
        constexpr int g = decltype(G)::value;
        q6_load8<g>(rw, blk(wbase, kt), e8, w1);
        if (quarter) q_load_q<QT, g>(rw, blk(wbase2, kt), qq, w2);
    };
    auto wstore = [&](auto G, uint4* st, int kt) {
        constexpr int g = decltype(G)::value;
        uint32_t o[4];
        q6_dequant8<MID, g>(w1, o);
        lds_write16(st + wslot8, make_uint4(o[0], o[1], o[2], o[3]));
        if (quarter) {
            uint32_t o0, o1;
            q_dequant_q<QT, MID, g>(w2, blk(wbase2, kt) & 3u, o0, o1);
            lds_write8(reinterpret_cast<uint2*>(st) + wslot4, o0, o1);
        }
    };
    const int lr = lane & 31, lk = lane >> 5;
    // fragment slots: chunk 4 h + 2 ks + lk of row ra (MFMA tile i's rows are 32 i further: the same swizzle); the
    // second stage of a pair (h = 1) is chunk bit 2 flipped, slot index ^ 4 (ra * 8 has bits 0-2 clear)
    int abase[2], bbase[2];
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
        const int ra = wave * WM * 32 + lr, rb = lr;
        abase[ks] = ra * 8 + swz8(ra, 2 * ks + lk);
        bbase[ks] = rb * 4 + swz4(rb, 2 * ks + lk);
    }
    bf16x8 fa[2][WM], fb[2][WN];
    // fragments of K half ks of the stage in half h of pair slot xst and weight slot wst, into register set `set`
    auto fread = [&](const uint4* xst, const uint4* wst, int h, int ks, int set) {
        const int ab = h ? abase[ks] ^ 4 : abase[ks];
#pragma unroll
        for (int i = 0; i < WM; i++) fa[set][i] = __builtin_bit_cast(bf16x8, xst[ab + 256 * i]);
#pragma unroll
        for (int j = 0; j < WN; j++) fb[set][j] = __builtin_bit_cast(bf16x8, wst[bbase[ks] + 128 * j]);
    };
    f32x16 acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++)
#pragma unroll
            for (int k = 0; k < 16; k++) acc[i][j][k] = 0.0f;
    auto mfmas = [&](int set) {
#pragma unroll
        for (int i = 0; i < WM; i++)
#pragma unroll
            for (int j = 0; j < WN; j++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[set][i], fb[set][j], acc[i][j], 0, 0, 0);
    };
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    using P2 = std::integral_constant<int, 2>;
    // weight ring slots as indices, the pointers formed at each use: reads through a pointer carried around the loop
    // have no known object, and the compiler then waits for every LDS DMA in flight before each of them
    int wcur = 0;                                      // stage s
    int wnxt = 1;                                      // stage s + 1
    int wnew = 2;                                      // stage s + 2 (stage s - 1's slot)
    auto wslot = [&](int i) { return wring + i * WSLOT; };
    issue_pair(xp0, 0);
    wload(P0{}, 0);
    wait_vm<0>();
    wstore(P0{}, wslot(wcur), 0);
    wload(P1{}, 1);
    wait_vm<0>();
    wstore(P1{}, wslot(wnxt), 1);
    wload(P2{}, 2);
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));   // lgkmcnt(0): this thread's LDS writes are done
    // Step s = kt + J of pair p = s / 2 (pair slot xc; the other slot xo): J even -- barrier (pair p has landed for
    // every wave, pair p - 1 is no longer read), issue pair p + 1 into xo, read stage s's first fragments; J odd --
    // barrier. Then stage s's second fragments, its MFMAs, the wait for the raw bytes of s + 2 (and, J odd, for pair
    // p + 1: every load of this wave), the dequantisation of s + 2, the raw loads of s + 3 and, J even, stage s + 1's
    // first fragments (same pair).
    auto step = [&](int kt, auto J, uint4* xc, uint4* xo) {
        constexpr int j = decltype(J)::value;
        constexpr int h = j & 1;
        const int s = kt + j;
        using G2 = std::integral_constant<int, (j + 2) & 7>;
        using G3 = std::integral_constant<int, (j + 3) & 7>;
        wave_barrier_sync();
        if constexpr (h == 0) {
            issue_pair(xo, (s >> 1) + 1);
            __builtin_amdgcn_sched_barrier(0);         // the loads leave now, not where the scheduler would sink them
            fread(xc, wslot(wcur), 0, 0, 0);
        }
        fread(xc, wslot(wcur), h, 1, 1);
        mfmas(0);
        mfmas(1);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (h == 0) wait_vm<IXP>();         // all but this step's pair loads have landed
        else wait_vm<0>();
        __builtin_amdgcn_sched_barrier(0);
        wstore(G2{}, wslot(wnew), s + 2);
        __builtin_amdgcn_sched_barrier(0);             // the next loads reuse the raw registers
        wload(G3{}, s + 3);
        if constexpr (h == 0) fread(xc, wslot(wnxt), 1, 0, 0);
        const int t = wcur;
        wcur = wnxt;
        wnxt = wnew;
        wnew = t;
    };
    for (int kt = 0; kt < nk; kt += 8) {
        step(kt, P0{}, xp0, xp1);
        step(kt, P1{}, xp0, xp1);
        step(kt, P2{}, xp1, xp0);
        step(kt, std::integral_constant<int, 3>{}, xp1, xp0);
        step(kt, std::integral_constant<int, 4>{}, xp0, xp1);
        step(kt, std::integral_constant<int, 5>{}, xp0, xp1);
        step(kt, std::integral_constant<int, 6>{}, xp1, xp0);
        step(kt, std::integral_constant<int, 7>{}, xp1, xp0);
    }
    // epilogue through LDS (idle once every load has landed and every wave is past its reads): each wave rounds its
    // 64 x 160 slab to bf16 in two passes of 32 rows into its own 10 KiB region (four per pair slot) and stores
    // whole 16-byte runs of rows
    constexpr int TC = WN * 32, RUNS = TC / 8;
    wait_vm<0>();
    wave_barrier_sync();
    uint16_t* ot = reinterpret_cast<uint16_t*>(wave < 4 ? xp0 : xp1) + (wave & 3) * 32 * TC;
    const uint4* ov = reinterpret_cast<const uint4*>(ot);
    const int mw = m0 + wave * WM * 32;
    float bn[WN];
#pragma unroll
    for (int j = 0; j < WN; j++) {
        const int n = n0 + j * 32 + lr;
        bn[j] = BIAS && n < N ? __uint_as_float((uint32_t)bias[n] << 16) : 0.0f;
    }
    const bool vec = (N & 7) == 0 && (reinterpret_cast<uintptr_t>(Y) & 15) == 0;
#pragma unroll
    for (int i = 0; i < WM; i++) {
#pragma unroll
        for (int j = 0; j < WN; j++)
#pragma unroll
            for (int k = 0; k < 16; k++) {
                float t = acc[i][j][k];
                if (BIAS) t = t + bn[j];
                ot[(8 * (k >> 2) + 4 * lk + (k & 3)) * TC + j * 32 + lr] = __builtin_bit_cast(uint16_t, (__bf16)t);
            }
        const int mp = mw + i * 32;
        if (vec) {
#pragma unroll
            for (int it = 0; it < 32 * RUNS / 64; it++) {
                const int q = it * 64 + lane, r = q / RUNS, c = q % RUNS;
                const int m = mp + r, n = n0 + 8 * c;
                const uint4 v = ov[q];
                if (m < M && n < N) *reinterpret_cast<uint4*>(Y + (int64_t)m * N + n) = v;
            }
        } else {
            for (int it = 0; it < 32 * RUNS / 64; it++) {
                const int q = it * 64 + lane, r = q / RUNS, c = q % RUNS;
                const int m = mp + r;
                if (m >= M) continue;
                for (int k = 0; k < 8; k++) {
                    const int n = n0 + 8 * c + k;
                    if (n < N) Y[(int64_t)m * N + n] = ot[r * TC + 8 * c + k];
                }
            }
        }
    }
}

template <int MID>
static void launch_tall(const uint16_t* X, const uint8_t* W, const uint16_t* bias, uint16_t* Y, int M, int N, int K,
                        hipStream_t s) {
    const int tiles = ((M + kTallBM - 1) / kTallBM) * ((N + kTallBN - 1) / kTallBN);
    if (bias) gemm_gguf_tall<MID, true><<<dim3(tiles), 512, 0, s>>>(X, W, bias, Y, M, N, K);
    else gemm_gguf_tall<MID, false><<<dim3(tiles), 512, 0, s>>>(X, W, bias, Y, M, N, K);
}

// the 512 x 160 form of a Q6_K [M, K] x [N, K] product (K % 256 == 0, operands checked by the caller)
void run_gguf_tall(int mid, const void* x_bf16, const void* wq, const void* bias_bf16, void* out_bf16, int M, int N,
                   int K, hipStream_t s) {
    const uint16_t* X = static_cast<const uint16_t*>(x_bf16);
    const uint8_t* W = static_cast<const uint8_t*>(wq);
    const uint16_t* B = static_cast<const uint16_t*>(bias_bf16);
    uint16_t* Y = static_cast<uint16_t*>(out_bf16);
    if (mid == WF_F16) launch_tall<WF_F16>(X, W, B, Y, M, N, K, s);
    else if (mid == WF_BF16) launch_tall<WF_BF16>(X, W, B, Y, M, N, K, s);
    else launch_tall<WF_F32>(X, W, B, Y, M, N, K, s);
}

}  // namespace wf
