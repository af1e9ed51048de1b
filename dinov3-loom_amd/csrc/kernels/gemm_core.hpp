// f16 MFMA GEMM core for gfx950: C[m][n] = sum_k A[m][k] * W[n][k], fp32
// accumulation, shared by every GEMM variant of the forward pass.
//
// A workgroup of WGM x WGN waves owns a BM x BN output tile; the K loop walks
// BK-deep stages. Two loops:
// - gemm_main (the patch embedding): both operands HBM/L2 -> registers ->
//   LDS (row pitch LDK) with two register sets and two LDS buffers, so the
//   loads of stage s+2 are in flight while stage s feeds the MFMAs and stage
//   s+1 is written to LDS.
// - gemm_main_dma (QKV, residual, SwiGLU, split-K): activations in fragment
//   order straight into registers (ActFrags), weights in fragment order moved
//   into three LDS buffers by DMA (WeightDma); its comment has the ordering
//   rules the waits rely on.
// The barriers only wait for LDS traffic (and, in the DMA loop, for the DMA
// loads they must): __syncthreads() would also drain every outstanding
// global load (its workgroup release fence waits on vmcnt(0)) and serialise
// the pipeline. Loads are unconditional where possible (indices clamped) so
// the compiler's vmcnt waits count exactly the loads they need.
//
// Each wave owns TM x TN of the tile as 32x32 tiles of
// v_mfma_f32_32x32x16_f16. The MFMA's first operand is the weight row (n) and
// its second the activation row (m): lane l then holds activation row l%32
// and weight rows 8*(r/4) + 4*(l/32) + r%4 of register r, i.e. 4 consecutive
// output columns per register group, so epilogues write 8-/16-byte vectors
// and the partner columns n and n+32 of a 64-wide wave tile share a lane.
#pragma once
#include <algorithm>

#include "common.hpp"

namespace dhx {
namespace gemm {

template <int BM_, int BN_, int WGM_, int WGN_, int BK_ = 64>
struct Tile {
    static constexpr int BM = BM_, BN = BN_, WGM = WGM_, WGN = WGN_;
    static constexpr int BK = BK_;
    // LDS row pitch in halfs (144 B for BK 64, 80 B for BK 32): the 16-byte
    // fragment reads of 8 consecutive rows hit disjoint banks.
    static constexpr int LDK = BK + 8;
    static_assert(BK == 128 || BK == 64 || BK == 32, "stage depth");
    static constexpr int WAVES = WGM * WGN, THREADS = 64 * WAVES;
    static constexpr int TM = BM / WGM, TN = BN / WGN;
    static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile is a multiple of the 32x32 MFMA tile");
    static constexpr int FM = TM / 32, FN = TN / 32;
    static constexpr int STAGE_HALFS = (BM + BN) * LDK;
    static constexpr int WF_HALFS = BN * BK;  // weight-only stage in fragment order (WeightDma)
    static constexpr int LDS_HALFS = 2 * STAGE_HALFS;
    static constexpr int LDS_BYTES = LDS_HALFS * 2;
};

// Rows r0 .. r0+ROWS-1 of a row-major f16 [*][ld] matrix, BK columns from
// k0, staged through registers into LDS rows of pitch LDK. Every load is
// unconditional, which keeps the compiler's vmcnt accounting exact (a
// predicated load makes every later wait drain the prefetches too).
template <int ROWS, int THREADS, int BK, int LDK>
struct HalfTile {
    // 16-byte chunks of one stage; when they do not split evenly over the
    // workgroup, the surplus threads repeat the last chunk (same data to the
    // same LDS location), which keeps every load unconditional.
    static constexpr int CPR = BK / 8;  // chunks per row
    static constexpr int TOTAL = ROWS * CPR;
    static constexpr int CHUNKS = (TOTAL + THREADS - 1) / THREADS;
    half8_t r[CHUNKS];
    __device__ __forceinline__ static int chunk(int tid, int i) {
        const int c = tid + i * THREADS;
        return TOTAL % THREADS == 0 ? c : min(c, TOTAL - 1);
    }
    __device__ __forceinline__ void load_all(const half_t* base, int ld, int r0, int k0, int tid) {
#pragma unroll
        for (int i = 0; i < CHUNKS; ++i) {
            const int c = chunk(tid, i), row = c / CPR, col = (c % CPR) * 8;
            r[i] = *(const half8_t*)(base + (size_t)(r0 + row) * ld + k0 + col);
        }
    }
    __device__ __forceinline__ void store(half_t* s, int tid) const {
#pragma unroll
        for (int i = 0; i < CHUNKS; ++i) {
            const int c = chunk(tid, i), row = c / CPR, col = (c % CPR) * 8;
            *(half8_t*)(s + row * LDK + col) = r[i];
        }
    }
};

// Weight operand: rows n0 .. n0+BN-1 of W[N][ldw] (the launchers only use N
// that are multiples of BN, so every row exists).
template <class T>
struct WeightRows {
    HalfTile<T::BN, T::THREADS, T::BK, T::LDK> t;
    const half_t* w;
    int ldw, k_off;
    __device__ __forceinline__ void load(int /*m0*/, int n0, int kt, int tid) {
        t.load_all(w, ldw, n0, k_off + kt * T::BK, tid);
    }
    __device__ __forceinline__ void store(half_t* s, int tid) const { t.store(s, tid); }
};

// A operand in fragment order (common.hpp), loaded straight into the
// registers the MFMAs read: each wave loads the fragments of its own TM rows
// (waves split the tile along M only, so no two waves load the same data).
// Blocks past the last one repeat it (they only feed unstored rows).
template <class T>
struct ActFrags {
    static constexpr bool kInRegs = true;
    static constexpr int KS = T::BK / 16;
    static_assert(T::WGN == 1, "each wave owns whole rows of the tile");
    half8_t f[T::FM][KS];
    const half_t* a;
    int ksteps;   // K / 16 of the whole matrix
    int mblocks;  // 32-row blocks of the matrix
    int ks_off;   // first k-step (split-K)
    __device__ __forceinline__ void load(int m0, int /*n0*/, int kt, int tid) {
        const int lane = tid & 63, wm = (tid >> 6) % T::WGM;
#pragma unroll
        for (int j = 0; j < T::FM; ++j) {
            const int mb = min((m0 + wm * T::TM) / 32 + j, mblocks - 1);
            const half_t* base = a + ((size_t)mb * ksteps + ks_off + kt * KS) * 512 + lane * 8;
#pragma unroll
            for (int kk = 0; kk < KS; ++kk) f[j][kk] = *(const half8_t*)(base + kk * 512);
        }
    }
};

// Weight operand in fragment order, moved from global memory straight into
// LDS. W[N][K] is stored as 32-row x 16-column blocks (the layout of
// fragment-order activations, common.hpp: block (nb, ks) at
// (nb * K/16 + ks) * 512 halfs, lane hi*32 + l holding row l, columns
// 8hi .. 8hi+7). buffer_load_dwordx4 with the lds flag writes each lane's
// 16 bytes to M0 + 16 * lane, so one instruction moves one 1 KB block and
// the LDS stage keeps the fragment order: block (nb, ks) of the stage at
// (nb * BK/16 + ks) * 512 halfs, read back conflict-free with
// ds_read_b128. No registers, no ds_write. The stage's blocks are split
// evenly over the waves. The buffer descriptor bounds every access to W.
template <class T>
struct WeightDma {
    static constexpr int KS = T::BK / 16;
    static constexpr int BLOCKS = T::BN / 32 * KS;  // per stage
    static constexpr int PER_WAVE = BLOCKS / T::WAVES;
    static_assert(BLOCKS % T::WAVES == 0, "whole blocks per wave");
    __amdgpu_buffer_rsrc_t rsrc;
    int ksteps;  // K / 16 of W
    int ks_off;  // first k-step (split-K)
    __device__ __forceinline__ WeightDma(const half_t* w, int n, int k)
        : rsrc(__builtin_amdgcn_make_buffer_rsrc(const_cast<half_t*>(w), 0, n * k * 2, kBufferRsrcWord3)),
          ksteps(k / 16),
          ks_off(0) {}
    __device__ __forceinline__ void load(half_t* stage, int n0, int kt, int tid) const {
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
#pragma unroll
        for (int b = 0; b < PER_WAVE; ++b) {
            const int blk = wave * PER_WAVE + b, nb = blk / KS, ks = blk % KS;
            const int off = (((n0 >> 5) + nb) * ksteps + ks_off + kt * KS + ks) * 1024;  // uniform
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)(stage + blk * 512),
                                                     16, (tid & 63) * 16, off, 0, 0);
        }
    }
};

template <class T>
struct Acc {
    float16_t v[T::FN][T::FM];
};

// One BK-deep stage of MFMAs from LDS. Fragments are double-buffered in
// registers: the reads for k-slice kk+1 are issued before the MFMAs of kk, so
// LDS latency overlaps the matrix pipe instead of stalling each MFMA.
template <class T>
__device__ __forceinline__ void mma_stage(const half_t* stage, int tid, Acc<T>& acc) {
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave % T::WGM, wn = wave / T::WGM;
    const int l32 = lane & 31, hi = lane >> 5;
    const half_t* a_s = stage + (wm * T::TM + l32) * T::LDK + hi * 8;
    const half_t* w_s = stage + (T::BM + wn * T::TN + l32) * T::LDK + hi * 8;
    half8_t wf[2][T::FN], af[2][T::FM];
    auto fetch = [&](int kk, int b) {
#pragma unroll
        for (int i = 0; i < T::FN; ++i) wf[b][i] = *(const half8_t*)(w_s + i * 32 * T::LDK + kk * 16);
#pragma unroll
        for (int j = 0; j < T::FM; ++j) af[b][j] = *(const half8_t*)(a_s + j * 32 * T::LDK + kk * 16);
    };
    fetch(0, 0);
#pragma unroll
    for (int kk = 0; kk < T::BK / 16; ++kk) {
        if (kk + 1 < T::BK / 16) fetch(kk + 1, (kk + 1) & 1);
#pragma unroll
        for (int i = 0; i < T::FN; ++i)
#pragma unroll
            for (int j = 0; j < T::FM; ++j) acc.v[i][j] = mfma32x32x16(wf[kk & 1][i], af[kk & 1][j], acc.v[i][j]);
    }
}

// One stage of MFMAs with the activation fragments already in registers
// (ActFrags) and the weight stage in LDS in fragment order (WeightDma): the
// wave reads every column of the stage (WGN == 1), one contiguous 1 KB block
// per fragment, for k-slice kk+1 while kk computes.
template <class T, class AF>
__device__ __forceinline__ void mma_stage_frag(const half_t* stage, int tid, const AF& af, Acc<T>& acc) {
    constexpr int KS = T::BK / 16;
    const half_t* w_s = stage + (tid & 63) * 8;
    half8_t wf[2][T::FN];
    auto fetch = [&](int kk, int b) {
#pragma unroll
        for (int i = 0; i < T::FN; ++i) wf[b][i] = *(const half8_t*)(w_s + (i * KS + kk) * 512);
    };
    fetch(0, 0);
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
        if (kk + 1 < KS) fetch(kk + 1, (kk + 1) & 1);
#pragma unroll
        for (int i = 0; i < T::FN; ++i)
#pragma unroll
            for (int j = 0; j < T::FM; ++j) acc.v[i][j] = mfma32x32x16(wf[kk & 1][i], af.f[j][kk], acc.v[i][j]);
    }
}

// The workgroup's tile: hardware workgroup ids are dispatched round-robin
// over the 8 XCDs (each with its own L2); the tile space (n fastest) is cut
// into 8 contiguous chunks and XCD x takes chunk x, so the workgroups of one
// XCD work on neighbouring tiles and share A rows and W in that XCD's L2.
// The grid is the tile count rounded up to a multiple of 8; workgroups past
// the end of their chunk have no tile.
__device__ __forceinline__ int xcd_tile(int total) {
    const int g = blockIdx.x, per = (total + 7) >> 3;
    const int t = (g & 7) * per + (g >> 3);
    return (g >> 3) < per && t < total ? t : -1;
}

// xcd_tile with the N tiles split into NS slices (NS divides 8 and n_tiles):
// XCD x takes N slice x % NS over M range x / NS of 8 / NS (n fastest within
// the XCD, as above). Each XCD's L2 then holds 1/NS of W, which survives the
// epilogue's output stream, for NS times the A reads. Returns the tile as
// m_tile * n_tiles + n_tile, or -1.
template <int NS>
__device__ __forceinline__ int xcd_tile_split(int m_tiles, int n_tiles) {
    static_assert(8 % NS == 0, "slices divide the XCDs");
    constexpr int MS = 8 / NS;
    const int g = blockIdx.x, x = g & 7, local = g >> 3;
    const int nsl = n_tiles / NS, mr = x / NS;
    const int m_lo = mr * m_tiles / MS, m_hi = (mr + 1) * m_tiles / MS;
    if (local >= (m_hi - m_lo) * nsl) return -1;
    return (m_lo + local / nsl) * n_tiles + (x % NS) * nsl + local % nsl;
}

// Workgroups for xcd_tile_split: 8 x the largest XCD share.
template <int NS>
inline int tile_grid_split(int m_tiles, int n_tiles) {
    constexpr int MS = 8 / NS;
    return 8 * ((m_tiles + MS - 1) / MS) * (n_tiles / NS);
}

// The pipelined K loop of one tile with P = 2 register sets and two LDS
// buffers: at step s the workgroup computes stage s from LDS buffer s%2, the
// loads of stage s+2 go into register set s%2 (whose stage s is already in
// LDS), and register set (s+1)%2, loaded one step earlier, is written to
// buffer (s+1)%2 (which held stage s-1, finished by every wave at the
// previous barrier). Loads past the last stage repeat it (unconditional
// loads keep the compiler's vmcnt waits exact). The loaders take the tile origin
// (m0, n0) and the stage. settle() runs once the first stages' loads are
// issued and before the first barrier: it can consume loads the caller
// issued earlier (they are older, so waiting for them does not wait for the
// stage loads) and write LDS that the epilogue reads.
template <class T, int P, class AL, class WL, class Settle>
__device__ __forceinline__ void gemm_main(AL (&al)[P], WL (&wl)[P], int m0, int n0, int k_tiles, half_t* lds,
                                          Acc<T>& acc, Settle&& settle) {
    static_assert(P == 2, "two register sets");
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < T::FN; ++i)
#pragma unroll
        for (int j = 0; j < T::FM; ++j) acc.v[i][j] = float16_t{};
    const int last = k_tiles - 1;
#pragma unroll
    for (int i = 0; i < P; ++i) {
        al[i].load(m0, n0, min(i, last), tid);
        wl[i].load(m0, n0, min(i, last), tid);
    }
    settle();
    al[0].store(lds, tid);
    wl[0].store(lds + T::BM * T::LDK, tid);
    lds_barrier();
    for (int base = 0; base < k_tiles; base += 2) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int s = base + i;
            if (s >= k_tiles) break;  // uniform
            half_t* const cur = lds + i * T::STAGE_HALFS;
            half_t* const nxt = lds + (1 - i) * T::STAGE_HALFS;
            al[i].load(m0, n0, min(s + 2, last), tid);
            wl[i].load(m0, n0, min(s + 2, last), tid);
            mma_stage<T>(cur, tid, acc);
            if (s + 1 < k_tiles) {
                al[1 - i].store(nxt, tid);
                wl[1 - i].store(nxt + T::BM * T::LDK, tid);
            }
            lds_barrier();
        }
    }
}

// Runs the tile of this workgroup (if any): issue(m0, n0) first (the
// epilogue's own loads: row statistics, column constants), then the K loop
// with settle() after its first loads (see gemm_main), then epi(acc, m0, n0).
// Issuing the epilogue's loads ahead of the K loop hides their latency, and
// since they are the oldest loads, the waits that consume them do not wait
// for the stage loads.
template <class T, int P, int NS = 1, class AL, class WL, class Issue, class Settle, class Epi>
__device__ __forceinline__ void gemm_tile(AL (&al)[P], WL (&wl)[P], int n_tiles, int total_tiles, int k_tiles,
                                          half_t* lds, Issue&& issue, Settle&& settle, Epi&& epi) {
    const int t = NS == 1 ? xcd_tile(total_tiles) : xcd_tile_split<NS>(total_tiles / n_tiles, n_tiles);
    if (t < 0) return;  // uniform per workgroup
    const int n0 = (t % n_tiles) * T::BN, m0 = (t / n_tiles) * T::BM;
    issue(m0, n0);
    Acc<T> acc;
    gemm_main<T, P>(al, wl, m0, n0, k_tiles, lds, acc, settle);
    epi(acc, m0, n0);
}

// gemm_tile without epilogue loads of its own.
template <class T, int P, class AL, class WL, class Epi>
__device__ __forceinline__ void gemm_tile(AL (&al)[P], WL (&wl)[P], int n_tiles, int total_tiles, int k_tiles,
                                          half_t* lds, Epi&& epi) {
    gemm_tile<T, P>(al, wl, n_tiles, total_tiles, k_tiles, lds, [](int, int) {}, [] {}, epi);
}

// Waits until at most N of this wave's vector-memory operations are
// outstanding and its LDS traffic is done, then joins the workgroup barrier.
template <int N>
__device__ __forceinline__ void vm_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Keeps the compiler from moving memory accesses across this point.
__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }

// Waiting for LDS DMA. Measured on the MI355X: a DMA load can land in LDS
// after vector loads issued later have completed, so "at most N outstanding"
// does not prove that a DMA issued before N register loads has landed (a
// two-buffer loop that relied on it returned different results from launch
// to launch). DMA loads do complete in issue order among themselves. A wait
// for DMA stage X is therefore "at most N outstanding" only where every one
// of the N may be a DMA load issued after X: all register loads are issued
// before the DMA loads they are waited with.

// Calls f(integral_constant<int, I>) for I = 0 .. N-1.
template <int N, int I = 0, class F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<N, I + 1>(f);
    }
}

// No work between the stages of the K loop.
struct NoMid {
    template <class A>
    __device__ __forceinline__ void operator()(A&, int) const {}
};

// The K loop with activations in registers (two sets, ActFrags) and the
// weight stages moved into three LDS buffers by DMA (WeightDma). Step s
// issues the activation loads of stage s+1 into the register set that held
// stage s-1, then the DMA of stage s+2 into the buffer that held stage s-1
// (both released by the previous barrier), computes stage s, and ends with a
// barrier that waits until only the DMA of stage s+2 may be outstanding:
// by DMA order stage s+1 has then landed for every wave. Activations get
// one step to arrive, weights up to two (the compiler places the DMA
// instructions among the step's last MFMAs; holding them at the top of the
// step with a scheduling barrier measured no faster). The three buffers are separate LDS
// variables and the loop is unrolled over them, so the compiler can tell a
// buffer being read from the ones being filled and does not wait for the
// DMA in flight. Nothing is loaded past the last stage. With KT > 0 the
// stage count is KT, known at compile time, and the steps are fully unrolled
// (any KT); otherwise k_tiles must be a multiple of 6 (the launchers check).
// mid(acc, s) runs in step s after its loads are issued and before its
// MFMAs: additive work on the accumulators there issues beside the MFMAs.
template <class T, int KT = 0, class AL, class WD, class Settle, class Mid = NoMid>
__device__ __forceinline__ void gemm_main_dma(AL (&al)[2], const WD& wd, half_t* b0, half_t* b1, half_t* b2, int m0,
                                              int n0, int k_tiles_rt, Acc<T>& acc, Settle&& settle, Mid&& mid = Mid{}) {
    const int k_tiles = KT > 0 ? KT : k_tiles_rt;
    static_assert(AL::kInRegs, "activations in registers");
    constexpr int NW = WD::PER_WAVE;
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < T::FN; ++i)
#pragma unroll
        for (int j = 0; j < T::FM; ++j) acc.v[i][j] = float16_t{};
    al[0].load(m0, n0, 0, tid);
    compiler_fence();
    wd.load(b0, n0, 0, tid);
    if (k_tiles > 1) wd.load(b1, n0, 1, tid);  // uniform
    settle();
    if (k_tiles > 1)
        vm_barrier<NW>();
    else
        vm_barrier<0>();
    auto step = [&](const half_t* cur, half_t* fill, AL& a, AL& next, int s) {
        const bool more = s + 2 < k_tiles;  // uniform
        if (s + 1 < k_tiles) next.load(m0, n0, s + 1, tid);
        compiler_fence();
        if (more) wd.load(fill, n0, s + 2, tid);
        mid(acc, s);
        mma_stage_frag<T>(cur, tid, a, acc);
        if (more)
            vm_barrier<NW>();
        else if (s + 1 < k_tiles)
            vm_barrier<0>();
    };
    if constexpr (KT > 0) {
        half_t* const bufs[3] = {b0, b1, b2};
#pragma unroll
        for (int s = 0; s < KT; ++s) step(bufs[s % 3], bufs[(s + 2) % 3], al[s & 1], al[(s + 1) & 1], s);
    } else {
        for (int kt = 0; kt < k_tiles; kt += 6) {
            step(b0, b2, al[0], al[1], kt);
            step(b1, b0, al[1], al[0], kt + 1);
            step(b2, b1, al[0], al[1], kt + 2);
            step(b0, b2, al[1], al[0], kt + 3);
            step(b1, b0, al[0], al[1], kt + 4);
            step(b2, b1, al[1], al[0], kt + 5);
        }
    }
}

// gemm_tile over gemm_main_dma.
template <class T, int NS = 1, int KT = 0, class AL, class WD, class Issue, class Settle, class Epi, class Mid = NoMid>
__device__ __forceinline__ void gemm_tile_dma(AL (&al)[2], WD& wd, half_t* b0, half_t* b1, half_t* b2, int n_tiles,
                                              int total_tiles, int k_tiles, Issue&& issue, Settle&& settle,
                                              Epi&& epi, Mid&& mid = Mid{}) {
    const int t = NS == 1 ? xcd_tile(total_tiles) : xcd_tile_split<NS>(total_tiles / n_tiles, n_tiles);
    if (t < 0) return;  // uniform per workgroup
    const int n0 = (t % n_tiles) * T::BN, m0 = (t / n_tiles) * T::BM;
    issue(m0, n0);
    Acc<T> acc;
    gemm_main_dma<T, KT>(al, wd, b0, b1, b2, m0, n0, k_tiles, acc, settle, mid);
    epi(acc, m0, n0);
}

// Workgroups for a launch: one per tile (a persistent walk over several
// tiles per resident workgroup measured slower: the hardware balances the
// last wave of tiles better), rounded up to a multiple of 8 for xcd_tile.
inline int tile_grid(int total_tiles) { return std::max(8, (total_tiles + 7) & ~7); }

__device__ __forceinline__ float4_t group4(const float16_t& a, int g) {
    return float4_t{a[4 * g], a[4 * g + 1], a[4 * g + 2], a[4 * g + 3]};
}

__device__ __forceinline__ half4_t to_half4(float4_t v) {
    return half4_t{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
}

__device__ __forceinline__ float4_t ld4(const float* p) { return *(const float4_t*)p; }

// Position of this lane's outputs: row m_base + 32j + l32, columns
// n_base + 32i + 8g + 4hi .. +3 for register group g of acc.v[i][j].
template <class T>
struct Frag {
    int l32, hi, m_base, n_base;
    __device__ __forceinline__ Frag(int m0, int n0) {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        l32 = lane & 31;
        hi = lane >> 5;
        m_base = m0 + (wave % T::WGM) * T::TM;
        n_base = n0 + (wave / T::WGM) * T::TN;
    }
    __device__ __forceinline__ int row(int j) const { return m_base + j * 32 + l32; }
    __device__ __forceinline__ int col(int i, int g) const { return n_base + i * 32 + g * 8 + hi * 4; }
};

template <class T>
inline int tiles_for(int rows, int n) {
    return (n / T::BN) * ((rows + T::BM - 1) / T::BM);
}

}  // namespace gemm
}  // namespace dhx
