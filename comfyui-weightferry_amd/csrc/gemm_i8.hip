// Int8 W8A8 linear for gfx950: out[m, n] = OUT((float(acc) * xs[m]) * ws[n] (+ bias[n])), acc = sum_k xq[m, k] *
// wq[n, k] exactly in int32 -- the role of kitchen's cutlass_int8_dequant (enhancers/fused_int8.py:191-206).
//
// Operand layout (both operands K-major): lane l of a v_mfma_i32_32x32x32_i8 fragment holds 16 bytes of row l % 32
// at K offset 16 * (l / 32) of the 32-wide K step. Result layout: lane l, register i holds row 8 (i / 4) +
// 4 (l / 32) + i % 4, column l % 32 of the 32x32 tile.
//
// Two kernels:
//  * gemm_i8_dl (K % 64 == 0, the workload): 256 x 320, 256 x 256, 256 x 128 or 128 x 160 tiles (chosen per
//    shape, see launch_dl), operands streamed global -> LDS by the load unit (no register staging) through a
//    4-stage ring of 64-byte K stages (128-byte for 128 x 160 tiles), and an epilogue that stages the rounded
//    tile in LDS and stores whole 16-byte runs of output rows.
//  * gemm_i8 (K % 16 == 0 otherwise): 2 x 2 waves, predicated loads staged through registers into a
//    double-buffered LDS tile of 128-byte K stages. Rows are 8 chunks of 16 bytes; chunk c of row r sits at slot
//    c ^ (((r >> 1) ^ ((r & 1) << 2)) & 7), conflict-free for stage writes and fragment reads.
//
// Tile order is XCD-aware: workgroup w runs on XCD w % 8, so consecutive tile indices are dealt to one XCD's
// workgroups and that XCD's L2 sees neighbouring tiles (they share A rows / B rows); within the order, tiles are
// grouped GROUP_M tile-rows at a time.

#include <algorithm>

#include "lds_ring.h"
#include "wl_ring.h"

namespace wf {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

constexpr int kBK = 128;        // K bytes per stage of gemm_i8

__device__ __forceinline__ int swz(int row, int chunk) { return swz8(row, chunk); }

__device__ __forceinline__ float to_f32_out(const void* p, int64_t i, int dt) {
    if (dt == WF_BF16) return __uint_as_float((uint32_t)static_cast<const uint16_t*>(p)[i] << 16);
    if (dt == WF_F16) return (float)__builtin_bit_cast(_Float16, static_cast<const uint16_t*>(p)[i]);
    return static_cast<const float*>(p)[i];
}

// Epilogue operands of the residual variant: out = bf16(resid + gate[m / rows_per_group] * bf16(t)), t the plain
// epilogue value: the plain GEMM's bf16 output followed by torch's addcmul on bf16 tensors (the product of two bf16
// values is exact in float32, the sum rounds once to float32, then to bf16). The reference states the same bits for
// kitchen's cutlass_int8_dequant_residual (enhancers/fused_int8.py:212-268, enhancers/fused_block.py:24-26).
struct Residual {
    const uint16_t* gate;    // bf16 [groups, N]
    const uint16_t* resid;   // bf16 [M, N]
    int rows_per_group;
};

// The per-row activation scales of a wave's R = 32 WM output rows from row mw: lane l loads xs[mw + l] (and
// xs[mw + 64 + l] for R = 128), one load each; row(ro) gives any lane the scale of row mw + ro by a lane permute
// (ds_bpermute). A global load per output element instead left each tile's epilogue waiting on 16-32 loads in
// turn. Rows at or past M read as zero (their outputs are not stored).
template <int WM>
struct RowScales {
    static constexpr int T = (WM * 32 + 63) / 64;
    float v[T];
    __device__ __forceinline__ RowScales(const float* __restrict__ xs, int mw, int M, int lane) {
#pragma unroll
        for (int t = 0; t < T; t++) {
            const int m = mw + 64 * t + lane;
            v[t] = m < M ? xs[m] : 0.0f;
        }
    }
    __device__ __forceinline__ float row(int ro) const {
        float x = v[0];
#pragma unroll
        for (int t = 1; t < T; t++)
            if ((ro >> 6) == t) x = v[t];
        return __shfl(x, ro & 63);
    }
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
    tile_order(blockIdx.x, ntm * ntn, ntm, ntn, tm, tn);
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
                    t = r + g * (float)(__bf16)t;
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

// ------------------------------------------------------------------------- K % 64 == 0: direct-to-LDS ring
// VM x VN waves of WM x WN MFMA tiles, the operands streamed through a 4-stage LDS ring of BK-byte K stages. The
// loads go from global memory straight into LDS (buffer_load_dwordx4 ... lds: lane l of an instruction writes the 16
// bytes at LDS slot l of a 1 KiB run, so the swizzle is applied on the global side -- lane l loads the chunk that
// belongs in slot l), with no register staging and no LDS write instructions; rows past M or N read as zeros. When
// the stage's 1 KiB runs do not divide evenly over the waves, the last waves' spare issues repeat the final run into
// pad slots after the stage, so every wave issues (and waits for) the same count. Stage kt + 3 is issued
// while stage kt is computed. The barrier at the top of stage kt certifies that stage kt + 1 has landed (every wave
// waited for its own loads) and that stage kt - 1 is no longer read, so the wave can prefetch stage kt + 1's first
// fragments during stage kt and never waits on LDS right after a barrier. A stage row is BK bytes = BK / 16 chunks,
// swizzled by row_swz so that the 16 lanes that read 16 rows' same chunk hit 16 different bank groups.
//
// BK = 64 (16 rows per load instruction); BK = 128 (8 rows of one whole 128-byte line each) for the 128 x 160
// tiling, whose 4 stages of 36 KiB fit the LDS. The vector memory return path (TD) pays per cache line touched, so
// half-line row segments cost it as much as whole lines: at 1024 x 5120 it was 69 % busy at 26 % MFMA busy with
// 64-byte stages, and 128-byte stages take that product from 39.3 to 33.3 us. The larger tilings hold 72 or 64 KiB
// per 128-byte stage, room for two stage buffers only: they run gemm_i8_wl below when K % 128 == 0, this ring
// otherwise.
constexpr int kDlBK = 64;

// slot of chunk c in a stage row r of CH chunks: 4 chunks (64 bytes) c ^ ((r >> 2) & 3); 8 chunks (128 bytes) swz
template <int CH>
__device__ __forceinline__ int row_swz(int row, int chunk) {
    static_assert(CH == 4 || CH == 8, "64- or 128-byte stage rows");
    if constexpr (CH == 4) return swz4(row, chunk);
    else return swz(row, chunk);
}

template <int VM, int VN, int WM, int WN, int OUT, bool BIAS, bool RESID, int BK>
__global__ __launch_bounds__(64 * VM * VN) void gemm_i8_dl(const int8_t* __restrict__ A, const int8_t* __restrict__ B,
                                                           const float* __restrict__ xs,
                                                           const float* __restrict__ ws,
                                                           const void* __restrict__ bias, void* __restrict__ out,
                                                           int M, int N, int K, Residual res) {
    constexpr int NT = 64 * VM * VN, NW = NT / 64;
    constexpr int BM = VM * WM * 32, BN = VN * WN * 32;
    constexpr int CH = BK / 16, RPI = 64 / CH, KS = BK / 32;   // 16-byte chunks per row, rows per load, K steps
    constexpr int AI = BM / RPI, BI = BN / RPI;           // 1 KiB load instructions per stage (RPI rows each)
    constexpr int IPW = (AI + BI + NW - 1) / NW;          // per wave; spare issues of the last waves fill pad slots
    constexpr int SLOTS = NW * IPW * 64;                  // 16-byte slots per stage, pad slots after the B rows
    static_assert(4 * SLOTS * 16 <= 160 * 1024, "the ring fits the LDS");
    __shared__ i32x4 st0[SLOTS], st1[SLOTS], st2[SLOTS], st3[SLOTS];
    const int ntm = (M + BM - 1) / BM, ntn = (N + BN - 1) / BN;
    int tm, tn;
    tile_order(blockIdx.x, ntm * ntn, ntm, ntn, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);     // wave-uniform: scalar load bases
    const int wm = wave / VN, wn = wave % VN;
    const int nk = K / BK;
    const __amdgpu_buffer_rsrc_t ra = tile_rsrc(A + (int64_t)m0 * K, (int64_t)(M - m0) * K);
    const __amdgpu_buffer_rsrc_t rb = tile_rsrc(B + (int64_t)n0 * K, (int64_t)(N - n0) * K);
    // this wave's load instructions: global chunk run gi = wave * IPW + q (A rows for gi < AI, then B rows)
    uint32_t voff[IPW];
#pragma unroll
    for (int q = 0; q < IPW; q++) {
        const int gi = min(wave * IPW + q, AI + BI - 1);  // a pad issue repeats the last B run into its pad slot
        const int r = (gi < AI ? gi : gi - AI) * RPI + lane / CH;
        voff[q] = (uint32_t)(r * K + 16 * row_swz<CH>(r, lane % CH));
    }
    auto issue = [&](i32x4* st, int kt) {
        const int k0 = kt * BK;
#pragma unroll
        for (int q = 0; q < IPW; q++) {
            const int gi = wave * IPW + q;
            lds_dma16(gi < AI ? ra : rb, st + 64 * gi, voff[q] + (uint32_t)k0);
        }
    };
    const int lr = lane & 31, lk = lane >> 5;
    int aslot[WM][KS], bslot[WN][KS];
#pragma unroll
    for (int i = 0; i < WM; i++) {
        const int row = wm * WM * 32 + i * 32 + lr;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) aslot[i][ks] = row * CH + row_swz<CH>(row, 2 * ks + lk);
    }
#pragma unroll
    for (int j = 0; j < WN; j++) {
        const int row = wn * WN * 32 + j * 32 + lr;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) bslot[j][ks] = BM * CH + row * CH + row_swz<CH>(row, 2 * ks + lk);
    }
    i32x4 fa[2][WM], fb[2][WN];
    auto fread = [&](const i32x4* st, int ks, int set) {
#pragma unroll
        for (int i = 0; i < WM; i++) fa[set][i] = st[aslot[i][ks]];
#pragma unroll
        for (int j = 0; j < WN; j++) fb[set][j] = st[bslot[j][ks]];
    };
    i32x16 acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0;
    auto mfmas = [&](int set) {
#pragma unroll
        for (int i = 0; i < WM; i++)
#pragma unroll
            for (int j = 0; j < WN; j++)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[set][i], fb[set][j], acc[i][j], 0, 0, 0);
    };
    // The ring always issues: stages at or past K read past the row's end -- inside the buffer range (other rows'
    // bytes) or past it (zeros) -- into a buffer no later stage reads. Branch-free issue keeps the compiler's
    // per-buffer tracking of the outstanding loads exact, so it adds no waits of its own before LDS reads.
    // the epilogue's scales (and bias) load first: their latency passes under the main loop instead of after it
    const int mw = m0 + wm * WM * 32, nw = n0 + wn * WN * 32;
    const RowScales<WM> rs(xs, mw, M, lane);
    float wsn[WN], bn[WN];
#pragma unroll
    for (int j = 0; j < WN; j++) {
        const int n = nw + j * 32 + lr;
        wsn[j] = n < N ? ws[n] : 0.0f;
        bn[j] = BIAS && n < N ? to_f32_out(bias, n, OUT) : 0.0f;
    }
    issue(st0, 0);
    issue(st1, 1);
    issue(st2, 2);
    wait_vm<2 * IPW>();                                          // stage 0 landed; 1 and 2 may be in flight
    wave_barrier_sync();
    fread(st0, 0, 0);
    // one ring step: stage kt in buffer CUR; NXT holds kt + 1, FREE (kt - 1) receives kt + 3
    auto step = [&](int kt, i32x4* cur, i32x4* nxt, i32x4* free_) {
        wait_vm<IPW>();                                          // stage kt + 1 landed (kt + 2 may be in flight)
        wave_barrier_sync();
        issue(free_, kt + 3);
        static_for<KS>([&](auto ksc) {                          // K step ks computes from fragment set ks & 1
            constexpr int ks = decltype(ksc)::value;
            if constexpr (ks + 1 < KS) fread(cur, ks + 1, (ks + 1) & 1);
            else fread(nxt, 0, 0);
            mfmas(ks & 1);
        });
    };
    int kt = 0;
    for (; kt + 4 <= nk; kt += 4) {
        step(kt, st0, st1, st3);
        step(kt + 1, st1, st2, st0);
        step(kt + 2, st2, st3, st1);
        step(kt + 3, st3, st0, st2);
    }
    if (kt < nk) step(kt, st0, st1, st3);
    if (kt + 1 < nk) step(kt + 1, st1, st2, st0);
    if (kt + 2 < nk) step(kt + 2, st2, st3, st1);

    // epilogue: (float(acc) * xs[m]) * ws[n] (+ bias[n]), rounded once to OUT
    if constexpr (!RESID) {
        // Through LDS: each wave writes its WM*32 x WN*32 tile, rounded, into its own LDS region (row-major,
        // WN*32 values a row), then stores whole 16-byte runs of output rows. The ring is idle by now: every
        // wave's last loads have landed (s_waitcnt) and every wave is past its last fragment reads (barrier).
        constexpr int TR = WM * 32, TC = WN * 32;          // this wave's rows and columns
        constexpr int PER_BUF = SLOTS * 16 / (TR * TC * 2); // wave regions per ring buffer
        static_assert(PER_BUF >= 1 && NW <= PER_BUF * 4, "the output tiles fit in the ring");
        __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0)
        wave_barrier_sync();
        const int wb = wave / PER_BUF;
        i32x4* buf = wb == 0 ? st0 : wb == 1 ? st1 : wb == 2 ? st2 : st3;
        uint16_t* ot = reinterpret_cast<uint16_t*>(buf) + (wave % PER_BUF) * TR * TC;
#pragma unroll
        for (int j = 0; j < WN; j++) {
#pragma unroll
            for (int i = 0; i < WM; i++) {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int r0 = i * 32 + 8 * q + 4 * lk;    // rows r0 .. r0 + 3 of this wave's tile
                    float xm[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) xm[e] = rs.row(r0 + e);
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        float t = ((float)acc[i][j][4 * q + e] * xm[e]) * wsn[j];
                        if (BIAS) t = t + bn[j];
                        ot[(r0 + e) * TC + j * 32 + lr] = OUT == WF_BF16 ? __builtin_bit_cast(uint16_t, (__bf16)t)
                                                                         : __builtin_bit_cast(uint16_t, (_Float16)t);
                    }
                }
            }
        }
        // the wave reads back only its own region: its LDS writes and reads execute in order
        const uint4* ov = reinterpret_cast<const uint4*>(ot);
        constexpr int RUNS = TC / 8;                       // 16-byte runs per row
        uint16_t* Y = static_cast<uint16_t*>(out);
        if ((N & 7) == 0 && (reinterpret_cast<uintptr_t>(Y) & 15) == 0) {   // whole aligned 16-byte runs
#pragma unroll
            for (int it = 0; it < TR * RUNS / 64; it++) {
                const int q = it * 64 + lane, r = q / RUNS, c = q % RUNS;
                const int m = mw + r, n = nw + 8 * c;
                const uint4 v = ov[q];
                if (m < M && n < N) *reinterpret_cast<uint4*>(Y + (int64_t)m * N + n) = v;   // N % 8: whole runs
            }
        } else {
            for (int it = 0; it < TR * RUNS / 64; it++) {
                const int q = it * 64 + lane, r = q / RUNS, c = q % RUNS;
                const int m = mw + r;
                if (m >= M) continue;
                const uint16_t* row = ot + r * TC + 8 * c;
                for (int e = 0; e < 8; e++) {
                    const int n = nw + 8 * c + e;
                    if (n < N) Y[(int64_t)m * N + n] = row[e];
                }
            }
        }
        return;
    }
    // the residual form: element stores, once the ring's last loads (stages past K among them) have landed -- no
    // copy into this workgroup's LDS may outlive it
    // (every lane reaches each row permute: a lane that skipped it would hand a zero to the lanes reading its row)
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0)
#pragma unroll
    for (int j = 0; j < WN; j++) {
        const int n = nw + j * 32 + lr;
        const bool in_n = n < N;
#pragma unroll
        for (int i = 0; i < WM; i++) {
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int ro = i * 32 + 8 * (e >> 2) + 4 * lk + (e & 3);
                const int m = mw + ro;
                const float xm = rs.row(ro);
                if (!in_n || m >= M) continue;
                float t = ((float)acc[i][j][e] * xm) * wsn[j];
                if (BIAS) t = t + bn[j];
                const int64_t o = (int64_t)m * N + n;
                if constexpr (RESID) {
                    const float g = __uint_as_float((uint32_t)res.gate[(int64_t)(m / res.rows_per_group) * N + n] << 16);
                    const float r = __uint_as_float((uint32_t)res.resid[o] << 16);
                    t = r + g * (float)(__bf16)t;
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

// K % 128 == 0, the 256-row tilings: whole 128-byte lines through two stage buffers (wl_ring.h), whose barrier sits
// before the last K step's MFMAs and whose loads leave right after it (16384 x 13824 x 5120: 1049 against 1137 us
// for the 64-byte ring, 4096 x 5120 x 5120: 100.1 against 105.4 us). The 128 x 160 tiling keeps the 4-stage ring of
// 128-byte stages (1024 x 5120 x 5120: 35.5 against 38.3 us on two buffers). Epilogue as above; the residual form
// stores single elements.
template <typename S, int OUT, bool BIAS, bool RESID>
__global__ __launch_bounds__(S::NT) void gemm_i8_wl(const int8_t* __restrict__ A, const int8_t* __restrict__ B,
                                                    const float* __restrict__ xs, const float* __restrict__ ws,
                                                    const void* __restrict__ bias, void* __restrict__ out, int M,
                                                    int N, int K, Residual res) {
    constexpr int WM = S::WM, WN = S::WN;
    __shared__ wl_frag sb0[S::SLOTS], sb1[S::SLOTS];
    const int ntm = (M + S::BM - 1) / S::BM, ntn = (N + S::BN - 1) / S::BN;
    int tm, tn;
    tile_order(blockIdx.x, ntm * ntn, ntm, ntn, tm, tn);
    const int m0 = __builtin_amdgcn_readfirstlane(tm * S::BM), n0 = __builtin_amdgcn_readfirstlane(tn * S::BN);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const __amdgpu_buffer_rsrc_t ra = tile_rsrc(A + (int64_t)m0 * K, (int64_t)(M - m0) * K);
    const __amdgpu_buffer_rsrc_t rb = tile_rsrc(B + (int64_t)n0 * K, (int64_t)(N - n0) * K);
    i32x16 acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0;
    wl_mainloop<S>(ra, rb, (uint32_t)K, K / 128, wave, lane, sb0, sb1, acc,
                   [](const i32x16& c, const wl_frag& a, const wl_frag& b) {
                       return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
                   });
    // (the scales load after the main loop here: held through it, the 256-row tilings' accumulators spill)
    const int wm = wave / S::VN, wn = wave % S::VN;
    const int mw = m0 + wm * WM * 32, nw = n0 + wn * WN * 32;
    const int lr = lane & 31, lk = lane >> 5;
    float wsn[WN], bn[WN];
#pragma unroll
    for (int j = 0; j < WN; j++) {
        const int n = nw + j * 32 + lr;
        wsn[j] = n < N ? ws[n] : 0.0f;
        bn[j] = BIAS && n < N ? to_f32_out(bias, n, OUT) : 0.0f;
    }
    const RowScales<WM> rs(xs, mw, M, lane);
    if constexpr (!RESID) {
        wl_store_tile<WM, WN>(wl_out_region<S>(sb0, sb1, wave), static_cast<uint16_t*>(out), M, N, mw, nw, lane,
                              [&](int i, int j, int e) {
                                  const float xm = rs.row(i * 32 + 8 * (e >> 2) + 4 * lk + (e & 3));
                                  float t = ((float)acc[i][j][e] * xm) * wsn[j];
                                  if (BIAS) t = t + bn[j];
                                  return OUT == WF_BF16 ? __builtin_bit_cast(uint16_t, (__bf16)t)
                                                        : __builtin_bit_cast(uint16_t, (_Float16)t);
                              });
    } else {
        // (every lane reaches each row permute: a lane that skipped it would hand a zero to the lanes reading its row)
#pragma unroll
        for (int j = 0; j < WN; j++) {
            const int n = nw + j * 32 + lr;
#pragma unroll
            for (int i = 0; i < WM; i++) {
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int ro = i * 32 + 8 * (e >> 2) + 4 * lk + (e & 3);
                    const int m = mw + ro;
                    const float xm = rs.row(ro);
                    if (n >= N || m >= M) continue;
                    const float t = ((float)acc[i][j][e] * xm) * wsn[j];
                    const int64_t o = (int64_t)m * N + n;
                    const float g = __uint_as_float((uint32_t)res.gate[(int64_t)(m / res.rows_per_group) * N + n] << 16);
                    const float r = __uint_as_float((uint32_t)res.resid[o] << 16);
                    static_cast<__bf16*>(out)[o] = (__bf16)(r + g * (float)(__bf16)t);
                }
            }
        }
    }
}

template <int VM, int VN, int WM, int WN, int OUT>
static void launch_wl_shape(const int8_t* A, const int8_t* B, const float* xs, const float* ws, const void* bias,
                            void* out, int M, int N, int K, Residual r, bool resid, hipStream_t s) {
    using S = WlShape<VM, VN, WM, WN>;
    const int tiles = ((M + S::BM - 1) / S::BM) * ((N + S::BN - 1) / S::BN);
    if (resid) gemm_i8_wl<S, OUT, false, true><<<dim3(tiles), S::NT, 0, s>>>(A, B, xs, ws, nullptr, out, M, N, K, r);
    else if (bias) gemm_i8_wl<S, OUT, true, false><<<dim3(tiles), S::NT, 0, s>>>(A, B, xs, ws, bias, out, M, N, K, r);
    else gemm_i8_wl<S, OUT, false, false><<<dim3(tiles), S::NT, 0, s>>>(A, B, xs, ws, bias, out, M, N, K, r);
}

// K % 64 == 0: the direct-to-LDS kernel in one of three tilings, chosen by the modelled time: rounds of 256 workgroups
// (one per CU) times the tile's area, over the tiling's measured MFMA efficiency.
//   256 x 320: 8 waves of 2 x 5 MFMA tiles (64 x 160); fewest LDS fragment reads per MFMA, and 4096 x 5120 outputs
//              make exactly 256 tiles.
//   256 x 256: 8 waves of 4 x 2 MFMA tiles (128 x 64).
//   256 x 128: 4 waves of 4 x 2 MFMA tiles, one per SIMD: more workgroups for small outputs.
//   128 x 160: 4 waves of 1 x 5 MFMA tiles: 1024 x 5120 outputs make exactly 256 tiles (1.2 LDS fragment reads per
//              MFMA against 0.75 for 4 x 2, but every CU busy: 42.7 against 50.9 us for the 256 x 128 tiling);
//              128-byte K stages where K % 128 == 0.
template <int VM, int VN, int WM, int WN, int OUT, int BK = kDlBK>
static void launch_dl_shape(const int8_t* A, const int8_t* B, const float* xs, const float* ws, const void* bias,
                            void* out, int M, int N, int K, Residual r, bool resid, hipStream_t s) {
    constexpr int BM = VM * WM * 32, BN = VN * WN * 32, NT = 64 * VM * VN;
    const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    if (resid) gemm_i8_dl<VM, VN, WM, WN, OUT, false, true, BK><<<dim3(tiles), NT, 0, s>>>(A, B, xs, ws, nullptr, out, M, N, K, r);
    else if (bias) gemm_i8_dl<VM, VN, WM, WN, OUT, true, false, BK><<<dim3(tiles), NT, 0, s>>>(A, B, xs, ws, bias, out, M, N, K, r);
    else gemm_i8_dl<VM, VN, WM, WN, OUT, false, false, BK><<<dim3(tiles), NT, 0, s>>>(A, B, xs, ws, bias, out, M, N, K, r);
}

// modelled time of a tiling: whole rounds of 256 workgroups x tile area / relative efficiency (per mille)
static int64_t dl_cost(int M, int N, int bm, int bn, int64_t eff) {
    const int64_t tiles = (int64_t)((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    return (tiles + 255) / 256 * bm * bn * 1000 / eff;
}

template <int OUT>
static void launch_dl(const int8_t* A, const int8_t* B, const float* xs, const float* ws, const void* bias,
                      void* out, int M, int N, int K, Residual r, bool resid, hipStream_t s) {
    const int64_t c320 = dl_cost(M, N, 256, 320, 1030), c256 = dl_cost(M, N, 256, 256, 1000);
    const int64_t c128 = dl_cost(M, N, 256, 128, 780), c160 = dl_cost(M, N, 128, 160, 581);
    const int64_t best = std::min(std::min(c320, c256), std::min(c128, c160));
    if (c160 == best && K % 128 == 0) launch_dl_shape<4, 1, 1, 5, OUT, 128>(A, B, xs, ws, bias, out, M, N, K, r, resid, s);
    else if (K % 128 == 0) {
        if (c128 == best) launch_wl_shape<2, 2, 4, 2, OUT>(A, B, xs, ws, bias, out, M, N, K, r, resid, s);
        else if (c256 == best) launch_wl_shape<2, 4, 4, 2, OUT>(A, B, xs, ws, bias, out, M, N, K, r, resid, s);
        else launch_wl_shape<4, 2, 2, 5, OUT>(A, B, xs, ws, bias, out, M, N, K, r, resid, s);
    } else if (c160 == best) launch_dl_shape<4, 1, 1, 5, OUT>(A, B, xs, ws, bias, out, M, N, K, r, resid, s);
    else if (c128 == best) launch_dl_shape<2, 2, 4, 2, OUT>(A, B, xs, ws, bias, out, M, N, K, r, resid, s);
    else if (c256 == best) launch_dl_shape<2, 4, 4, 2, OUT>(A, B, xs, ws, bias, out, M, N, K, r, resid, s);
    else launch_dl_shape<4, 2, 2, 5, OUT>(A, B, xs, ws, bias, out, M, N, K, r, resid, s);
}

// K % 16 == 0 otherwise: the predicated register-staged kernel
template <int OUT>
static void dispatch(const int8_t* A, const int8_t* B, const float* xs, const float* ws, const void* bias,
                     void* out, int M, int N, int K, hipStream_t s) {
    if (K % kDlBK == 0) {
        launch_dl<OUT>(A, B, xs, ws, bias, out, M, N, K, {}, false, s);
        return;
    }
    // large outputs: 256 x 256 tiles (4 x 4 MFMA tiles per wave); small ones keep 128 x 128 to fill the chip
    const int64_t big_tiles = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
    if (big_tiles >= 512) {
        const int tiles = ((M + 255) / 256) * ((N + 255) / 256);
        if (bias) gemm_i8<4, 4, OUT, true><<<dim3(tiles), 256, 0, s>>>(A, B, xs, ws, bias, out, M, N, K);
        else gemm_i8<4, 4, OUT, false><<<dim3(tiles), 256, 0, s>>>(A, B, xs, ws, bias, out, M, N, K);
    } else {
        const int tiles = ((M + 127) / 128) * ((N + 127) / 128);
        if (bias) gemm_i8<2, 2, OUT, true><<<dim3(tiles), 256, 0, s>>>(A, B, xs, ws, bias, out, M, N, K);
        else gemm_i8<2, 2, OUT, false><<<dim3(tiles), 256, 0, s>>>(A, B, xs, ws, bias, out, M, N, K);
    }
}

static void dispatch_resid(const int8_t* A, const int8_t* B, const float* xs, const float* ws, void* out, int M, int N,
                           int K, Residual r, hipStream_t s) {
    if (K % kDlBK == 0) {
        launch_dl<WF_BF16>(A, B, xs, ws, nullptr, out, M, N, K, r, true, s);
        return;
    }
    const int64_t big_tiles = (int64_t)((M + 255) / 256) * ((N + 255) / 256);
    if (big_tiles >= 512) {
        const int tiles = ((M + 255) / 256) * ((N + 255) / 256);
        gemm_i8<4, 4, WF_BF16, false, true><<<dim3(tiles), 256, 0, s>>>(A, B, xs, ws, nullptr, out, M, N, K, r);
    } else {
        const int tiles = ((M + 127) / 128) * ((N + 127) / 128);
        gemm_i8<2, 2, WF_BF16, false, true><<<dim3(tiles), 256, 0, s>>>(A, B, xs, ws, nullptr, out, M, N, K, r);
    }
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
    dispatch_resid(xq, wq, xs, ws, out_bf16, (int)M, (int)N, (int)K, r, s);
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
        set_error("wf_linear_i8: sizes beyond the kernels' 32-bit tile indices");
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
