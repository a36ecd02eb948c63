// Main loop and epilogue store of the GEMMs whose operands stream in whole 128-byte lines (gemm_bf16.hip, the int8
// GEMM's wl forms in gemm_i8.hip): C[BM x BN] += A[BM rows, K] . B[BN rows, K]^T, both operands K-major, 16-byte
// MFMA fragments (v_mfma_f32_32x32x16_bf16 and v_mfma_i32_32x32x32_i8 both take 16 bytes of row l % 32 at byte
// 16 (l / 32) of a 32-byte K step).
//
// Each K stage is 128 bytes of every row of both operands, loaded global -> LDS by the load unit (buffer_load ...
// lds): one 1 KiB load covers 8 rows x one whole cache line, the swizzle applied on the global side (lane l loads
// the chunk that belongs in slot l). Two stage buffers: the loads of stage p + 1 fly while stage p is computed. The
// texture-data return path pays per cache line touched, so whole-line stages cost it half of what 64-byte half-line
// stages do; that path, not the MFMA, bounded the 64-byte form of these tilings.
//
// One barrier per stage, before the last K step's MFMAs: each wave has waited for its own loads of stage p + 1 and
// for its own fragment reads of stage p, so after the barrier stage p + 1 is whole and stage p's buffer is free; the
// loads of stage p + 2 go out into it at once (a scheduling barrier keeps the compiler from sinking them towards the
// next wait), the first fragments of stage p + 1 are read, and the MFMAs of stage p's last K step cover that read.
#pragma once

#include "lds_ring.h"

namespace wf {

typedef int32_t wl_frag __attribute__((ext_vector_type(4)));   // one 16-byte MFMA operand fragment

template <int VM_, int VN_, int WM_, int WN_>
struct WlShape {
    static constexpr int VM = VM_, VN = VN_, WM = WM_, WN = WN_;
    static constexpr int NT = 64 * VM * VN, NW = NT / 64;
    static constexpr int BM = VM * WM * 32, BN = VN * WN * 32;
    static constexpr int AI = BM / 8, BI = BN / 8;            // 1 KiB loads per stage (8 rows of 128 bytes)
    static constexpr int IPW = (AI + BI + NW - 1) / NW;       // per wave; spare issues of the last waves fill pad slots
    static constexpr int SLOTS = NW * IPW * 64;               // 16-byte slots per stage buffer
    static_assert(2 * SLOTS * 16 <= 160 * 1024, "two stage buffers fit the LDS");
};

// acc[i][j] (MFMA tile i of the wave's rows, j of its columns) over nk stages of rows [0, BM) of ra and [0, BN) of
// rb, KB bytes a row. sb0 / sb1: the kernel's two __shared__ stage buffers of S::SLOTS fragments (separate arrays,
// so the compiler tracks the loads into each on its own). mma(acc, a, b) returns acc + a . b.
template <typename S, typename Acc, typename Mma>
__device__ __forceinline__ void wl_mainloop(__amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb, uint32_t KB, int nk,
                                            int wave, int lane, wl_frag* sb0, wl_frag* sb1,
                                            Acc (&acc)[S::WM][S::WN], Mma&& mma) {
    constexpr int WM = S::WM, WN = S::WN, AI = S::AI, BI = S::BI, IPW = S::IPW, BM = S::BM;
    const int wm = wave / S::VN, wn = wave % S::VN;
    // load gi covers rows 8 g .. 8 g + 7 of its operand (g = gi, or gi - AI for B); lane l takes row 8 g + l / 8,
    // chunk swz8(row, l % 8) = swz8(l / 8, l % 8) ^ 4 (g & 1): two per-lane offsets and a wave-uniform row term
    const uint32_t lo_even = (uint32_t)(lane / 8) * KB + 16u * (uint32_t)swz8(lane / 8, lane % 8);
    const uint32_t lo_odd = lo_even ^ 64u;
    auto issue = [&](wl_frag* st, int kt) {
        const uint32_t k0 = (uint32_t)kt * 128u;
#pragma unroll
        for (int q = 0; q < IPW; q++) {
            const int gi = wave * IPW + q;
            const int gc = min(gi, AI + BI - 1);           // a pad issue repeats the last B run into its pad slot
            const int g = gc < AI ? gc : gc - AI;
            lds_dma16(gc < AI ? ra : rb, st + 64 * gi, ((g & 1) ? lo_odd : lo_even) + (uint32_t)(8 * g) * KB + k0);
        }
    };
    // fragment of K step ks (this lane's 16-byte half lk) of row r sits at slot r * 8 + swz8(r, 2 ks + lk) =
    // (r * 8 + swz8(r, lk)) ^ 2 ks; the swizzle depends on r % 16 only, so the wave's MFMA tiles (32 rows apart) sit
    // at constant distances from its first: one base per operand, XORed per K step
    const int lr = lane & 31, lk = lane >> 5;
    const int arow = wm * WM * 32 + lr, brow = wn * WN * 32 + lr;
    const int abase = arow * 8 + swz8(arow, lk), bbase = BM * 8 + brow * 8 + swz8(brow, lk);
    wl_frag fa[2][WM], fb[2][WN];
    auto fread = [&](const wl_frag* st, int ks, int set) {
        const wl_frag* pa = st + (abase ^ (2 * ks));
        const wl_frag* pb = st + (bbase ^ (2 * ks));
#pragma unroll
        for (int i = 0; i < WM; i++) fa[set][i] = pa[i * 256];
#pragma unroll
        for (int j = 0; j < WN; j++) fb[set][j] = pb[j * 256];
    };
    auto mfmas = [&](int set) {
#pragma unroll
        for (int i = 0; i < WM; i++)
#pragma unroll
            for (int j = 0; j < WN; j++) acc[i][j] = mma(acc[i][j], fa[set][i], fb[set][j]);
    };
    // stages at or past K read past the row's end (other rows' bytes, or zeros past the buffer) into a buffer no later
    // stage reads: the loads always issue, so the compiler's per-buffer load tracking stays exact
    issue(sb0, 0);
    issue(sb1, 1);
    wait_vm<IPW>();                                      // stage 0 landed; 1 may be in flight
    wave_barrier_sync();
    fread(sb0, 0, 0);
    // stage p in cur (its first fragments already in set 0), stage p + 1 flying into oth
    auto step = [&](int p, wl_frag* cur, wl_frag* oth) {
        fread(cur, 1, 1);
        mfmas(0);
        fread(cur, 2, 0);
        mfmas(1);
        fread(cur, 3, 1);
        mfmas(0);
        wait_vm<0>();                                    // stage p + 1 landed (this wave's loads)
        __builtin_amdgcn_s_waitcnt(0xc07f);              // lgkmcnt(0): this wave's reads of cur are done
        wave_barrier_sync();                             // ... and every wave's: cur is free, p + 1 is whole
        issue(cur, p + 2);
        __builtin_amdgcn_sched_barrier(0);               // the loads leave now, not where the scheduler would sink them
        fread(oth, 0, 0);
        mfmas(1);
    };
    int p = 0;
    for (; p + 2 <= nk; p += 2) {
        step(p, sb0, sb1);
        step(p + 1, sb1, sb0);
    }
    if (p < nk) step(p, sb0, sb1);
    wait_vm<0>();                                        // the stage buffers are idle from here on
    __builtin_amdgcn_s_waitcnt(0xc07f);
    wave_barrier_sync();
}

// Region of wave w for the epilogue: 32 rows x WN * 32 values of 16 bits in the idle stage buffers.
template <typename S>
__device__ __forceinline__ uint16_t* wl_out_region(wl_frag* sb0, wl_frag* sb1, int wave) {
    constexpr int PER_BUF = S::SLOTS * 16 / (32 * S::WN * 32 * 2);
    static_assert(PER_BUF >= 1 && S::NW <= PER_BUF * 2, "the output rows fit in the stage buffers");
    return reinterpret_cast<uint16_t*>(wave / PER_BUF == 0 ? sb0 : sb1) + (wave % PER_BUF) * 32 * S::WN * 32;
}

// Stores the wave's WM * 32 x WN * 32 output tile at rows mw.., columns nw.. of Y [M, N] (16-bit values), 32 rows at
// a time through its LDS region ot: bits(i, j, e) gives the output bits of accumulator element e of MFMA tile (i, j)
// (row mw + 32 i + 8 (e / 4) + 4 (lane / 32) + e % 4, column nw + 32 j + lane % 32). Whole 16-byte row runs go out
// when N % 8 == 0 and Y is 16-byte aligned, single values otherwise. The wave reads back only its own region, and its
// LDS writes and reads execute in order.
template <int WM, int WN, typename Bits>
__device__ __forceinline__ void wl_store_tile(uint16_t* ot, uint16_t* Y, int M, int N, int mw, int nw, int lane,
                                              Bits&& bits) {
    constexpr int TC = WN * 32, RUNS = TC / 8;
    const int lr = lane & 31, lk = lane >> 5;
    const uint4* ov = reinterpret_cast<const uint4*>(ot);
    const bool vec = (N & 7) == 0 && (reinterpret_cast<uintptr_t>(Y) & 15) == 0;
#pragma unroll
    for (int i = 0; i < WM; i++) {
        const int mi = mw + i * 32;
#pragma unroll
        for (int e = 0; e < 16; e++)
#pragma unroll
            for (int j = 0; j < WN; j++) ot[(8 * (e >> 2) + 4 * lk + (e & 3)) * TC + j * 32 + lr] = bits(i, j, e);
        if (vec) {
#pragma unroll
            for (int it = 0; it < 32 * RUNS / 64; it++) {
                const int q = it * 64 + lane, r = q / RUNS, c = q % RUNS;
                const int m = mi + r, n = nw + 8 * c;
                const uint4 v = ov[q];
                if (m < M && n < N) *reinterpret_cast<uint4*>(Y + (int64_t)m * N + n) = v;
            }
        } else {
            for (int it = 0; it < 32 * RUNS / 64; it++) {
                const int q = it * 64 + lane, r = q / RUNS, c = q % RUNS;
                const int m = mi + r;
                if (m >= M) continue;
                const uint16_t* row = ot + r * TC + 8 * c;
                for (int e = 0; e < 8; e++) {
                    const int n = nw + 8 * c + e;
                    if (n < N) Y[(int64_t)m * N + n] = row[e];
                }
            }
        }
    }
}

}  // namespace wf
