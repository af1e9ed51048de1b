// Online-softmax attention for gfx950 (replaces the reference's
// kernels/attention_online_f16_wmma_cf16.loom).
//
// One workgroup = 4 waves = 128 queries of one (image, head); each wave owns
// 32 queries. Keys stream through LDS in blocks of 32 or 64 (K and V both as
// [key][ch]), so the same kernel serves 201 tokens (224x224) and 1029
// tokens (512x512). q, k and v come per (image, head) as [tpad][64]
// matrices in fragment order (a wave's Q fragments are then 1 KB contiguous
// loads). The blocks move from global memory straight into three
// LDS buffers with DMA loads (buffer_load ... lds), two blocks ahead; each
// 128-byte key row is stored with its 16-byte chunks XOR-swizzled by the
// row (swz below), so the row reads of K and the transpose reads of V hit
// distinct banks.
//
// Everything is computed transposed so that a lane owns one query:
//   S^T = K . Q^T      (MFMA a = K rows from LDS, b = Q^T held in registers)
//   O^T += V^T . P^T   (MFMA a = V^T rows, read out of the [key][ch] V block
//                       with LDS transpose reads; b = P^T straight from the
//                       S^T accumulators)
// Lane l holds query (l % 32) and 16 of every 32 keys; the other 16 are in
// lane l ^ 32, so each row max / row sum is 15 in-register ops plus one
// cross-half exchange, and the running rescale of O^T is a per-lane scalar.
// Q is scaled by 1/8 in registers and log2(e) is folded into one FMA per
// score, so the softmax runs on v_exp_f32; the running max is updated lazily
// (only when a block's weights against it sum past e^8), which skips
// most rescales of O and, on the common path, the block max itself.
// P is rounded to f16 for the PV product; the denominator keeps the fp32
// weights (as in the reference, attention_online_f16_wmma_cf16.loom:195-216).
#include "launch.hpp"

namespace dhx {
namespace {

constexpr int kThreads = 256;
constexpr int QB = 128;                  // queries per workgroup
// The lazy rescaling's slack: the running max moves only when a block's
// weights against it sum past e^8 (some score more than 8 above it).
constexpr float kLazySum = 2980.957987f;  // e^8

// LDS on gfx950 has 64 banks of 4 bytes: two 128-byte key rows per bank
// cycle. Chunk c of key row r sits at slot c ^ swz_slot(r), with
// swz_slot(r) = f((r / 2) % 8), f(t) = 4 (t % 2) + t / 2 (a bijection). The
// K row reads of 16 lanes (16 consecutive rows, one chunk) then cover all
// 64 banks, and so do the V transpose reads (4 consecutive rows x 4 aligned
// chunks per 32 lanes: rows 2 apart differ in bit 2 of the slot).
__device__ __forceinline__ int swz_slot(int r) {
    const int t = (r >> 1) & 7;
    return ((t & 1) << 2) | (t >> 1);
}

// Element offset of channel ch (a multiple of 4) of key row r inside a
// swizzled block.
__device__ __forceinline__ int swz(int r, int ch) {
    return r * kHeadDim + ((((ch >> 3) ^ swz_slot(r)) & 7) << 3) + (ch & 7);
}

// Waits until at most N of this wave's vector-memory operations are
// outstanding and its LDS traffic is done, then joins the workgroup barrier.
template <int N>
__device__ __forceinline__ void vm_barrier() {
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// The running softmax state of one lane's query (lane l holds query l % 32
// and half of each 32-key sub-block's scores; see the top of this file).
struct QueryState {
    half8_t qf[4];                      // Q^T fragments, pre-scaled by 1/8
    float16_t o[2];                     // O^T accumulators: channels 32ct + 8(r/4) + 4hi + r%4
    float m_run = -1e30f, l_run = 0.f;  // running max (lazy) and denominator
};

// Transpose-read position of this lane inside a 4-key x 32-channel patch of
// a V block: lane j of each 16-lane group receives channel 16*(group%2) + j
// of four consecutive keys.
__device__ __forceinline__ int tr_row_of(int lane) { return (lane & 15) >> 2; }
__device__ __forceinline__ int tr_col_of(int lane) { return 16 * ((lane >> 4) & 1) + 4 * (lane & 3); }

// One sub-block of 32 keys (rows row0 .. row0+31 of the swizzled K and V
// blocks in LDS, keys key0 .. key0+31 of the sequence of T):
// S^T = K Q^T, masked past T, lazy running max, P = 2^(s log2e - m log2e),
// O^T += V^T P^T with P in f16 and the denominator in f32. FIRST: the first
// sub-block of a walk (O and l still zero), whose weights against the
// initial max of -1e30 would all overflow: its block max becomes the
// running max directly, with one pass of exponentials instead of two (the
// same values and rounding as the rescale path).
template <bool FIRST = false>
__device__ __forceinline__ void attend32(QueryState& st, const half_t* sK, const half_t* sV, int row0, int key0,
                                         int T, int lane) {
    const int l32 = lane & 31, hi = lane >> 5;
    const float neg_inf = -__builtin_inff();
    float16_t s = {};
    const int kr = row0 + l32;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) s = mfma32x32x16(*(const half8_t*)(sK + swz(kr, kk * 16 + hi * 8)), st.qf[kk], s);
    // The V^T operands do not depend on the softmax: read them now so their
    // LDS latency hides under the exponentials. va[ct][ks] holds channel
    // ct*32 + l32 of keys key0 + 16ks + (j < 4 ? 4hi + j : 8 + 4hi + j - 4).
    const int tr_row = tr_row_of(lane), tr_col = tr_col_of(lane);
    half8_t va[2][2];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int vr = row0 + ks * 16 + 4 * hi + tr_row;
            const half4_t a0 = lds_read_tr16(sV + swz(vr, ct * 32 + tr_col));
            const half4_t a1 = lds_read_tr16(sV + swz(vr + 8, ct * 32 + tr_col));
            va[ct][ks] = __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7);
        }
    // s[r] is the score of key key0 + 8(r/4) + 4*hi + r%4 for query l32.
    if (key0 + 32 > T) {  // the last, partial block of keys (uniform)
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if (key0 + 8 * (r >> 2) + 4 * hi + (r & 3) >= T) s[r] = neg_inf;
    }
    // Weights against the running max; after the first sub-block (which
    // takes its own max), the block max is needed only when some lane's
    // weights sum past e^8 (a weight may then exceed it): blocks whose
    // scores grew by more than 8. Those lanes move their max to the
    // block's, rescale O and l, and recompute; every weight is then at most
    // its sum, at most e^8, well inside f16.
    float p[16];
    auto weights = [&](float m) {  // p = 2^(s log2e - m log2e); the pair's sum
        const float mb = m * kLog2e;
        float sum = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            p[r] = fast_exp2(fmaf(s[r], kLog2e, -mb));
            sum += p[r];
        }
        return half_pair_sum(sum);
    };
    auto block_max = [&] {
        float mx = s[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
        return half_pair_max(mx);  // every sub-block holds a valid key of each pair
    };
    float sum;
    if constexpr (FIRST) {
        st.m_run = block_max();
        sum = weights(st.m_run);
    } else {
        sum = weights(st.m_run);
        const bool grow = !(sum <= kLazySum);
        if (__any(grow)) {  // uniform across the wave
            const float m_new = grow ? fmaxf(block_max(), st.m_run) : st.m_run;
            const float alpha = fast_exp2((st.m_run - m_new) * kLog2e);
            st.l_run *= alpha;
            st.o[0] *= alpha;
            st.o[1] *= alpha;
            st.m_run = m_new;
            sum = weights(m_new);
        }
    }
    st.l_run += sum;
    // P^T as the b operand: k-slice element j of this lane is key
    // key0 + 16ks + (j < 4 ? 4hi + j : 8 + 4hi + j - 4), as in va.
    half8_t pb[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e) pb[ks][e] = (half_t)p[8 * ks + e];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) st.o[ct] = mfma32x32x16(va[ct][ks], pb[ks], st.o[ct]);
}

// Output of one lane's query: O / l in f16 into out (fragment order): each
// 16-channel half of a 32-channel block becomes one 8-channel piece per lane
// after frag_swap. row0: the first query row of the wave (wave-uniform); the
// wave's 32 rows lie in its 32-row block and the next, which the
// write-through descriptor covers.
__device__ __forceinline__ void store_query(const QueryState& st, half_t* out, int row0, int row, int head, int hi) {
    const size_t base = (size_t)(row0 / 32) * (kHidden / 16) * 512;
    const WtOut o(out + base, 2 * (kHidden / 16) * 1024);
    const float inv = 1.0f / st.l_run;
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const float16_t& a = st.o[ct];
            const half4_t g0 = {(half_t)(a[8 * kk] * inv), (half_t)(a[8 * kk + 1] * inv),
                                (half_t)(a[8 * kk + 2] * inv), (half_t)(a[8 * kk + 3] * inv)};
            const half4_t g1 = {(half_t)(a[8 * kk + 4] * inv), (half_t)(a[8 * kk + 5] * inv),
                                (half_t)(a[8 * kk + 6] * inv), (half_t)(a[8 * kk + 7] * inv)};
            const half8_t piece = frag_swap(g0, g1);
            const int c = head * kHeadDim + ct * 32 + kk * 16 + hi * 8;
            o.store((uint32_t)(frag_piece(row, c, kHidden) - base) * 2, piece);
        }
}

// NKB > 0: the number of key blocks of KB = 32 keys, known at compile time
// (the block loop is then unrolled, which keeps the compiler's wait counts
// exact; used for 201 tokens, whose 24 KB of LDS also leave room for other
// image groups' kernels). NKB = 0: any count of KB = 64-key blocks.
template <int NKB>
struct KeyBlock {
    static constexpr int KB = NKB > 0 ? 32 : 64;   // keys per LDS block
    static constexpr int BLK = KB * kHeadDim;      // halfs per K (or V) block
    static constexpr int LOADS = KB / 32;          // DMA loads of 8 rows per matrix and wave
};

// DMA offsets for moving 8 key rows (one 1 KB load) out of a
// fragment-order [tpad][64] matrix: lane i lands at LDS slot (row i/8, chunk
// slot i%8) of rows r0 .. r0+7 and fetches the chunk c the swizzle puts
// there (r0 % 8 == 0, so row % 16 = r0 % 16 + i/8). Chunk c (channels 8c ..
// 8c+7) of row r sits at byte ((r/32)*4 + c/2)*1024 + ((c%2)*32 + r%32)*16:
// the lane part holds c and i/8, the scalar part (dma_row_offset) r0's
// 32-row block and r0 % 32 (no carry: r0 % 32 + 7 < 32). A load reads 8
// runs of 128 bytes (8 rows of one chunk each).
__device__ __forceinline__ int dma_lane_offset(int lane, int r0) {
    const int c = (lane & 7) ^ swz_slot(r0 % 16 + (lane >> 3));
    return ((c >> 1) << 10) + ((c & 1) << 9) + (lane >> 3) * 16;
}
__device__ __forceinline__ int dma_row_offset(int r0) { return (r0 >> 5) * 4096 + (r0 & 31) * 16; }

template <int NKB>
__global__ __launch_bounds__(kThreads, 3) void attention_kernel(AttentionArgs p) {
    using KBT = KeyBlock<NKB>;
    __shared__ __attribute__((aligned(16))) half_t sK0[KBT::BLK], sK1[KBT::BLK], sK2[KBT::BLK];
    __shared__ __attribute__((aligned(16))) half_t sV0[KBT::BLK], sV1[KBT::BLK], sV2[KBT::BLK];
    // 1-D grid, XCD-aware: the tile space (query block fastest, then head,
    // then image) is cut into 8 contiguous chunks, one per XCD, so the query
    // blocks of one (image, head) share K and V in that XCD's L2.
    const int nqb = (p.tokens + QB - 1) / QB, total = nqb * kHeads * p.images;
    const int per = (total + 7) >> 3, g = blockIdx.x, t = (g & 7) * per + (g >> 3);
    if ((g >> 3) >= per || t >= total) return;  // uniform per workgroup
    const int qb = t % nqb, head = (t / nqb) % kHeads, img = t / (nqb * kHeads);
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, hi = lane >> 5;
    const int T = p.tokens;
    const size_t bh = (size_t)img * kHeads + head;
    const half_t* qg = p.q + bh * p.tpad * kHeadDim;
    const int nkb = NKB > 0 ? NKB : (T + KBT::KB - 1) / KBT::KB;  // nkb * KB <= tpad, so every block row exists

    // Block kb of K and V: each wave moves KB/4 key rows of each, as 1 KB
    // DMA loads of 8 rows.
    const uint32_t bytes = (uint32_t)p.tpad * kHeadDim * 2;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<half_t*>(p.k + bh * p.tpad * kHeadDim), 0, bytes, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<half_t*>(p.v + bh * p.tpad * kHeadDim), 0, bytes, kBufferRsrcWord3);
    // Wave w moves key rows (KB/4) w .. +KB/4-1 as KB/32 loads of 8 rows per
    // matrix; load j covers rows (KB/4) w + 8j.
    // Sized 2, not KBT::LOADS: with a local array whose size depends on the
    // template parameter this compiler silently drops the host launch stub.
    int voff[2];
#pragma unroll
    for (int j = 0; j < KBT::LOADS; ++j) voff[j] = dma_lane_offset(lane, (tid >> 6) * (KBT::KB / 4) + 8 * j);
    auto dma = [&](half_t* k_buf, half_t* v_buf, int kb) {
#pragma unroll
        for (int j = 0; j < KBT::LOADS; ++j) {
            const int row = wave * (KBT::KB / 4) + j * 8, soff = dma_row_offset(kb * KBT::KB + row);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)(k_buf + row * kHeadDim),
                                                     16, voff[j], soff, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (__attribute__((address_space(3))) void*)(v_buf + row * kHeadDim),
                                                     16, voff[j], soff, 0, 0);
        }
    };
    constexpr int kDmaPerBlock = 2 * KBT::LOADS;  // per wave

    // Block 0 first, then the Q fragments (registers), then block 1: the
    // wait for block 0 counts only the DMA loads of block 1 (DMA loads land
    // in issue order among themselves, but not in order with register loads).
    dma(sK0, sV0, 0);
    // Queries past T load row T-1 (unconditional loads keep the wait counts
    // exact); their results are never stored.
    const int qrow = qb * QB + wave * 32 + l32;
    QueryState st;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
        st.qf[kk] = *(const half8_t*)(qg + frag_piece(min(qrow, T - 1), kk * 16 + hi * 8, kHeadDim));
    asm volatile("" ::: "memory");
    if (NKB == 0 || nkb > 1) {  // with a runtime count, block 1 repeats block 0 when there is one block
        dma(sK1, sV1, min(1, nkb - 1));
        vm_barrier<kDmaPerBlock>();
    } else {
        vm_barrier<0>();
    }

    // Scores are s = (q / 8) . k: Q is scaled by 1/8 once (a power of two,
    // exact for normal f16 values), and the softmax weight of a score is
    // 2^(s*log2e - m*log2e), one FMA and one v_exp_f32.
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) st.qf[kk] *= (half_t)0.125f;
    st.o[0] = st.o[1] = float16_t{};
    // Waves whose 32 queries all lie past T only help move K and V.
    const bool active = qb * QB + wave * 32 < T;

    auto block = [&](const half_t* sK, const half_t* sV, int kb) {
#pragma unroll
        for (int sub = 0; sub < KBT::KB / 32 && active; ++sub) {
            const int key0 = kb * KBT::KB + sub * 32;
            if (key0 >= T) break;  // uniform across the workgroup
            if (NKB > 0 && kb == 0 && sub == 0)  // the unrolled walk: its first block is known at compile time
                attend32<true>(st, sK, sV, 0, key0, T, lane);
            else
                attend32(st, sK, sV, sub * 32, key0, T, lane);
        }
    };
    // Block kb is computed from buffer kb % 3 while the DMA of block kb+2
    // fills the buffer of block kb-1 (released by the previous barrier). The
    // barrier after block kb waits until only block kb+2's DMA may be in
    // flight, so block kb+1 has landed for every wave.
    auto step = [&](const half_t* k_cur, const half_t* v_cur, half_t* k_fill, half_t* v_fill, int kb) {
        const bool more = kb + 2 < nkb;  // uniform
        if (more) dma(k_fill, v_fill, kb + 2);
        block(k_cur, v_cur, kb);
        if (more)
            vm_barrier<kDmaPerBlock>();
        else if (kb + 1 < nkb)
            vm_barrier<0>();
    };
    if constexpr (NKB > 0) {
        half_t* const kbuf[3] = {sK0, sK1, sK2};
        half_t* const vbuf[3] = {sV0, sV1, sV2};
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) step(kbuf[kb % 3], vbuf[kb % 3], kbuf[(kb + 2) % 3], vbuf[(kb + 2) % 3], kb);
    } else {
        // Runtime block count: every step issues its DMA (past the last block
        // it repeats the last one into the buffer just released) and waits
        // the same way, so no branch makes the compiler's counts conservative;
        // the repeats are drained before the workgroup ends.
        auto step_rt = [&](const half_t* k_cur, const half_t* v_cur, half_t* k_fill, half_t* v_fill, int kb) {
            dma(k_fill, v_fill, min(kb + 2, nkb - 1));
            block(k_cur, v_cur, kb);
            vm_barrier<kDmaPerBlock>();
        };
        for (int kb = 0; kb < nkb; kb += 3) {
            step_rt(sK0, sV0, sK2, sV2, kb);
            if (kb + 1 >= nkb) break;
            step_rt(sK1, sV1, sK0, sV0, kb + 1);
            if (kb + 2 >= nkb) break;
            step_rt(sK2, sV2, sK1, sV1, kb + 2);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }

    if (qrow < T) store_query(st, p.out, img * T + qb * QB + wave * 32, img * T + qrow, head, hi);
}

// Long sequences (512x512: 1029 tokens): each workgroup of 8 waves holds 128
// queries as 4 query waves x 2 key halves. Half h walks key blocks
// h*NH .. h*NH+NH-1 (32 keys each, NH known at compile time so the walk is
// unrolled and every wait exact), streamed by its own 4 waves through its own
// three DMA buffers; both halves meet at the same barriers. At the end the
// second half's (running max, denominator, O^T) go through LDS to the first
// half, which merges them (rescaling both to the larger max) and writes the
// output. Twice the waves of attention_kernel for the same workgroups, so
// the softmax VALU work of one wave overlaps the MFMAs and loads of others.
constexpr int kSplitThreads = 512;
constexpr int kSplitBlk = 32 * kHeadDim;  // halfs per 32-key K (or V) block

// One key half's walk: blocks first .. first+NH-1 (past the sequence's last
// block the DMA repeats that block and the compute is skipped), through the
// half's own three K and three V buffers. The buffers are separate LDS
// variables chosen at compile time (the caller branches on the half), so the
// compiler can tell the buffer being read from the ones being filled and
// adds no waits of its own for the DMA in flight.
template <int NH>
__device__ __forceinline__ void split_walk(QueryState& st, half_t* const (&kbuf)[3], half_t* const (&vbuf)[3],
                                           const __amdgpu_buffer_rsrc_t& rk, const __amdgpu_buffer_rsrc_t& rv,
                                           const half_t* qg, int first, int nkb, int qrow, bool active, int T,
                                           int hwave, int lane) {
    const int hi = lane >> 5;
    const int voff = dma_lane_offset(lane, 8 * hwave), last = min(first + NH, nkb) - 1;
    auto dma = [&](int buf, int s) {
        const int kb = min(first + s, last), row = 8 * hwave, soff = dma_row_offset(kb * 32 + row);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)(kbuf[buf] + row * kHeadDim),
                                                 16, voff, soff, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (__attribute__((address_space(3))) void*)(vbuf[buf] + row * kHeadDim),
                                                 16, voff, soff, 0, 0);
    };
    // As in attention_kernel: block 0, the Q fragments, block 1; the first
    // wait counts only block 1's two DMA loads.
    dma(0, 0);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
        st.qf[kk] = *(const half8_t*)(qg + frag_piece(min(qrow, T - 1), kk * 16 + hi * 8, kHeadDim));
    asm volatile("" ::: "memory");
    dma(1, 1);
    vm_barrier<2>();
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) st.qf[kk] *= (half_t)0.125f;
    st.o[0] = st.o[1] = float16_t{};
    // Step s: block first+s from buffer s % 3 while block s+2's DMA fills
    // buffer (s+2) % 3 (released by the previous barrier); the barrier
    // leaves only that DMA in flight, so block s+1 has landed for every wave.
#pragma unroll
    for (int s = 0; s < NH; ++s) {
        if (s + 2 < NH) dma((s + 2) % 3, s + 2);
        const int kb = first + s;
        if (active && kb < nkb) {
            if (s == 0)
                attend32<true>(st, kbuf[0], vbuf[0], 0, kb * 32, T, lane);
            else
                attend32(st, kbuf[s % 3], vbuf[s % 3], 0, kb * 32, T, lane);
        }
        if (s + 2 < NH)
            vm_barrier<2>();
        else
            vm_barrier<0>();
    }
}

// Two workgroups per CU: four waves per SIMD (the bound below), which caps
// the kernel at 128 VGPRs; one register more halves the resident workgroups.
template <int NH>
__global__ __launch_bounds__(kSplitThreads, 4) void attention_split_kernel(AttentionArgs p) {
    // Per half three K and three V blocks of 4 KB (48 KB), as separate
    // variables (the compiler tells distinct variables apart, not the rows of
    // one array); reused at the end for the merge.
    __shared__ __attribute__((aligned(16))) half_t k00[kSplitBlk], k01[kSplitBlk], k02[kSplitBlk];
    __shared__ __attribute__((aligned(16))) half_t v00[kSplitBlk], v01[kSplitBlk], v02[kSplitBlk];
    __shared__ __attribute__((aligned(16))) half_t k10[kSplitBlk], k11[kSplitBlk], k12[kSplitBlk];
    __shared__ __attribute__((aligned(16))) half_t v10[kSplitBlk], v11[kSplitBlk], v12[kSplitBlk];
    const int nqb = (p.tokens + QB - 1) / QB, total = nqb * kHeads * p.images;
    const int per = (total + 7) >> 3, g = blockIdx.x, t = (g & 7) * per + (g >> 3);
    if ((g >> 3) >= per || t >= total) return;  // uniform per workgroup
    const int qb = t % nqb, head = (t / nqb) % kHeads, img = t / (nqb * kHeads);
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int qw = wave & 3, half = wave >> 2;  // query wave; key half (uniform per wave)
    const int l32 = lane & 31, hi = lane >> 5;
    const int T = p.tokens, nkb = (T + 31) / 32;  // nkb <= 2 * NH and nkb * 32 <= tpad (launcher checks)
    const size_t bh = (size_t)img * kHeads + head;
    const uint32_t bytes = (uint32_t)p.tpad * kHeadDim * 2;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<half_t*>(p.k + bh * p.tpad * kHeadDim), 0, bytes, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<half_t*>(p.v + bh * p.tpad * kHeadDim), 0, bytes, kBufferRsrcWord3);
    const half_t* qg = p.q + bh * p.tpad * kHeadDim;
    const int qrow = qb * QB + qw * 32 + l32;
    const bool active = qb * QB + qw * 32 < T;  // waves whose queries all lie past T only move K and V
    QueryState st;
    if (half == 0) {
        half_t* const kb[3] = {k00, k01, k02};
        half_t* const vb[3] = {v00, v01, v02};
        split_walk<NH>(st, kb, vb, rk, rv, qg, 0, nkb, qrow, active, T, qw, lane);
    } else {
        half_t* const kb[3] = {k10, k11, k12};
        half_t* const vb[3] = {v10, v11, v12};
        split_walk<NH>(st, kb, vb, rk, rv, qg, NH, nkb, qrow, active, T, qw, lane);
    }
    // Merge: the second half hands its 34 values per lane (max, denominator,
    // O^T) to the first through LDS; both are rescaled to the larger max.
    // Every wave passed the walk's last barrier, which waited for all of its
    // DMA loads, so the buffers are free. Value f of query wave qw sits in
    // buffer f / 4 at [(f % 4) * 4 + qw][lane] (f is a constant, so each
    // access names its buffer).
    half_t* const bufs[12] = {k00, k01, k02, v00, v01, v02, k10, k11, k12, v10, v11, v12};
    auto slot = [&](int f) -> float* {
        return reinterpret_cast<float*>(bufs[f / 4]) + ((f % 4) * 4 + qw) * 64 + lane;
    };
    if (half == 1) {
        *slot(0) = st.m_run;
        *slot(1) = st.l_run;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            *slot(2 + r) = st.o[0][r];
            *slot(18 + r) = st.o[1][r];
        }
    }
    __syncthreads();
    if (half == 1 || qrow >= T) return;
    const float m1 = *slot(0), m = fmaxf(st.m_run, m1);
    const float a0 = fast_exp2((st.m_run - m) * kLog2e), a1 = fast_exp2((m1 - m) * kLog2e);
    st.l_run = st.l_run * a0 + *slot(1) * a1;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        st.o[0][r] = st.o[0][r] * a0 + *slot(2 + r) * a1;
        st.o[1][r] = st.o[1][r] * a0 + *slot(18 + r) * a1;
    }
    store_query(st, p.out, img * T + qb * QB + qw * 32, img * T + qrow, head, hi);
}

}  // namespace

hipError_t launch_attention(const AttentionArgs& a, hipStream_t s) {
    const int total = (a.tokens + QB - 1) / QB * kHeads * a.images;
    const dim3 grid((total + 7) & ~7), block(kThreads);
    // 224x224 (201 tokens): seven blocks of 32 keys, unrolled. 512x512 (1029
    // tokens, 33 blocks of 32): the split-key kernel with 17 blocks per half.
    // Otherwise blocks of 64 with a run-time count.
    const int nkb32 = (a.tokens + 31) / 32;
    if (nkb32 == 7) {
        hipLaunchKernelGGL(attention_kernel<7>, grid, block, 0, s, a);
    } else if ((nkb32 + 1) / 2 == 17 && nkb32 * 32 <= a.tpad) {
        hipLaunchKernelGGL(attention_split_kernel<17>, grid, dim3(kSplitThreads), 0, s, a);
    } else {
        hipLaunchKernelGGL(attention_kernel<0>, grid, block, 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace dhx
