// Online-softmax attention for gfx950 (replaces the reference's
// kernels/attention_online_f16_wmma_cf16.loom).
//
// One workgroup = 4 waves = 128 queries of one (image, head); each wave owns
// 32 queries. Keys stream through LDS in blocks of 64 (K and V both as
// [key][ch], double-buffered), so the same kernel serves 201 tokens
// (224x224) and 1029 tokens (512x512).
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
// (only when it grows by more than kLazy), which skips most rescales of O.
// P is rounded to f16 for the PV product; the denominator keeps the fp32
// weights (as in the reference, attention_online_f16_wmma_cf16.loom:195-216).
#include "launch.hpp"

namespace dhx {
namespace {

constexpr int kThreads = 256;
constexpr int KB = 64;    // keys per LDS block
constexpr int KLD = 72;   // LDS row pitch in halfs
constexpr int QB = 128;   // queries per workgroup
constexpr float kLazy = 8.0f;  // running-max slack of the lazy rescaling (score units)

__device__ __forceinline__ half8_t zero8() {
    half8_t z = {};
    return z;
}

__global__ __launch_bounds__(kThreads, 3) void attention_kernel(AttentionArgs p) {
    __shared__ half_t sK[2][KB * KLD];
    __shared__ half_t sV[2][KB * KLD];
    // 1-D grid, XCD-aware: the tile space (query block fastest, then head,
    // then image) is cut into 8 contiguous chunks, one per XCD, so the query
    // blocks of one (image, head) share K and V in that XCD's L2.
    const int nqb = (p.tokens + QB - 1) / QB, total = nqb * kHeads * p.images;
    const int per = (total + 7) >> 3, g = blockIdx.x, t = (g & 7) * per + (g >> 3);
    if ((g >> 3) >= per || t >= total) return;  // uniform per workgroup
    const int qb = t % nqb, head = (t / nqb) % kHeads, img = t / (nqb * kHeads);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, hi = lane >> 5;
    const int T = p.tokens;
    const size_t bh = (size_t)img * kHeads + head;
    const half_t* qg = p.q + bh * p.tpad * kHeadDim;
    const half_t* kg = p.k + bh * p.tpad * kHeadDim;
    const half_t* vg = p.v + bh * p.tpad * kHeadDim;

    const int nkb = (T + KB - 1) / KB;
    const int qrow = qb * QB + wave * 32 + l32;
    half8_t qf[4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
        qf[kk] = qrow < T ? *(const half8_t*)(qg + (size_t)qrow * kHeadDim + kk * 16 + hi * 8) : zero8();

    // Each thread moves two 16-byte pieces of the K block and two of V. Two
    // register sets: the loads of block kb+2 are issued while block kb is
    // computed, so each has two blocks of compute to land (a block is short
    // next to an L2 round trip). Loads past the last block repeat it.
    half8_t kr[2][2], vr[2][2];
    auto load = [&](int set, int kb) {
        kb = min(kb, nkb - 1);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = tid + i * kThreads, row = c >> 3, col = (c & 7) * 8;
            kr[set][i] = *(const half8_t*)(kg + (size_t)(kb * KB + row) * kHeadDim + col);
            vr[set][i] = *(const half8_t*)(vg + (size_t)(kb * KB + row) * kHeadDim + col);
        }
    };
    auto store = [&](int set, int buf) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int c = tid + i * kThreads, row = c >> 3, col = (c & 7) * 8;
            *(half8_t*)(&sK[buf][row * KLD + col]) = kr[set][i];
            *(half8_t*)(&sV[buf][row * KLD + col]) = vr[set][i];
        }
    };

    // Transpose-read position of this lane inside a 4-key x 32-channel patch
    // of the V block: lane j of each 16-lane group then receives channel
    // 16*(group%2) + j of four consecutive keys.
    const int tr_row = (lane & 15) >> 2, tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

    // Scores are s = (q / 8) . k: Q is scaled by 1/8 once (a power of two,
    // exact for normal f16 values), and the softmax weight of a score is
    // 2^(s*log2e - m*log2e), one FMA and one v_exp_f32.
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) qf[kk] *= (half_t)0.125f;
    const float neg_inf = -__builtin_inff();
    float16_t o[2] = {float16_t{}, float16_t{}};
    float m_run = -1e30f, l_run = 0.f;
    // Waves whose 32 queries all lie past T only help move K and V.
    const bool active = qb * QB + wave * 32 < T;

    load(0, 0);
    load(1, 1);
    store(0, 0);
    lds_barrier();
    auto block = [&](int kb, int buf) {
#pragma unroll
        for (int sub = 0; sub < 2 && active; ++sub) {
            const int key0 = kb * KB + sub * 32;
            if (key0 >= T) break;  // uniform across the workgroup
            float16_t s = {};
            const half_t* krow = &sK[buf][(sub * 32 + l32) * KLD + hi * 8];
    #pragma unroll
            for (int kk = 0; kk < 4; ++kk) s = mfma32x32x16(*(const half8_t*)(krow + kk * 16), qf[kk], s);
            // s[r] is the score of key key0 + 8(r/4) + 4*hi + r%4 for query l32.
            if (key0 + 32 > T) {  // the last, partial block of keys (uniform)
    #pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (key0 + 8 * (r >> 2) + 4 * hi + (r & 3) >= T) s[r] = neg_inf;
            }
            float mx = s[0];
    #pragma unroll
            for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
            mx = half_pair_max(mx);  // every sub-block holds a valid key of each pair
            // Lazy rescaling: the running max moves only when a score exceeds
            // it by more than kLazy, so weights stay below e^kLazy (well inside
            // f16 for P) and most sub-blocks skip rescaling O entirely.
            const bool grow = mx > m_run + kLazy;
            if (__any(grow)) {  // uniform across the wave
                const float m_new = grow ? mx : m_run;
                const float alpha = fast_exp2((m_run - m_new) * kLog2e);
                l_run *= alpha;
                o[0] *= alpha;
                o[1] *= alpha;
                m_run = m_new;
            }
            const float mb = m_run * kLog2e;
            float sum = 0.f;
    #pragma unroll
            for (int r = 0; r < 16; ++r) {
                s[r] = fast_exp2(fmaf(s[r], kLog2e, -mb));
                sum += s[r];
            }
            sum = half_pair_sum(sum);
            l_run += sum;
            // P^T as the b operand: k-slice element j of this lane is key
            // key0 + 16ks + (j < 4 ? 4hi + j : 8 + 4hi + j - 4); the V^T
            // transpose reads below give channel ct*32 + l32 of the same keys.
            half8_t pb[2];
    #pragma unroll
            for (int ks = 0; ks < 2; ++ks)
    #pragma unroll
                for (int e = 0; e < 8; ++e) pb[ks][e] = (half_t)s[8 * ks + e];
    #pragma unroll
            for (int ct = 0; ct < 2; ++ct)
    #pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    const half_t* vb = &sV[buf][(sub * 32 + ks * 16 + 4 * hi + tr_row) * KLD + ct * 32 + tr_col];
                    const half4_t a0 = lds_read_tr16(vb), a1 = lds_read_tr16(vb + 8 * KLD);
                    const half8_t va = __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7);
                    o[ct] = mfma32x32x16(va, pb[ks], o[ct]);
                }
        }
    };
    for (int kb = 0; kb < nkb; kb += 2) {
        load(0, kb + 2);
        block(kb, 0);
        if (kb + 1 < nkb) store(1, 1);
        lds_barrier();
        if (kb + 1 >= nkb) break;
        load(1, kb + 3);
        block(kb + 1, 1);
        if (kb + 2 < nkb) store(0, 0);
        lds_barrier();
    }

    if (qrow < T) {
        // out is in fragment order: the lane's 4 channels are half of one
        // 8-channel piece of row img*T + qrow (the partner lane l ^ 32 holds
        // the other half), so the 32 queries of a wave fill whole pieces.
        const float inv = 1.0f / l_run;
        const int row = img * T + qrow;
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int c = head * kHeadDim + ct * 32 + g * 8 + hi * 4;
                half4_t v = {(half_t)(o[ct][4 * g] * inv), (half_t)(o[ct][4 * g + 1] * inv),
                             (half_t)(o[ct][4 * g + 2] * inv), (half_t)(o[ct][4 * g + 3] * inv)};
                *(half4_t*)(p.out + frag_piece(row, c & ~7, kHidden) + (c & 7)) = v;
            }
    }
}

}  // namespace

hipError_t launch_attention(const AttentionArgs& a, hipStream_t s) {
    const int total = (a.tokens + QB - 1) / QB * kHeads * a.images;
    hipLaunchKernelGGL(attention_kernel, dim3((total + 7) & ~7), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace dhx
