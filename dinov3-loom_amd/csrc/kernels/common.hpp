// Shared device definitions for the gfx950 (CDNA4, wave64) kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dhx {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float2_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t uint2_t __attribute__((ext_vector_type(2)));
typedef uint32_t uint4_t __attribute__((ext_vector_type(4)));

constexpr int kHidden = 384;
constexpr int kHeads = 6;
constexpr int kHeadDim = 64;
constexpr int kPrefix = 5;
constexpr int kFF = 1536;
constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// Word 3 of a raw buffer descriptor on CDNA (gfx9 family): 32-bit data
// format (untyped buffer instructions need a nonzero one), no swizzle, no
// index stride.
constexpr int kBufferRsrcWord3 = 0x00020000;

// A 64-bit address from its two 32-bit words as __builtin_amdgcn_readfirstlane
// returns them (int). Each word is widened through uint32_t: widened as a
// signed int, a low word with bit 31 set would sign-extend and overwrite the
// high word with ones (0x80000000 -> 0xffffffff80000000), and stores through
// such a base fault.
__host__ __device__ constexpr uint64_t address_from_words(int lo, int hi) {
    return ((uint64_t)(uint32_t)hi << 32) | (uint64_t)(uint32_t)lo;
}

// Output stores that write through the L2: 16-byte buffer stores with the
// sc1 cache policy. On this multi-XCD GPU every dispatch ends by writing its
// dirty L2 lines back (the XCDs' L2s are not coherent with each other), and
// for a kernel that writes tens of MB that flush is a serial tail after its
// last workgroup; written through, the lines are already out when the
// kernel's waves finish. The descriptor covers `bytes` from `base`; both
// must be wave-uniform (they are read from the first lane, so that the
// descriptor lives in scalar registers: one the compiler cannot prove
// uniform costs a loop over the lanes' values at every store). Offsets are
// bytes from base.
struct WtOut {
    __amdgpu_buffer_rsrc_t r;
    __device__ __forceinline__ WtOut(const void* base, uint32_t bytes) {
        const uint64_t a = (uint64_t)(uintptr_t)base;
        const uint64_t u = address_from_words(__builtin_amdgcn_readfirstlane((uint32_t)a),
                                              __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)));
        r = __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)u, 0, (int)__builtin_amdgcn_readfirstlane(bytes),
                                              kBufferRsrcWord3);
    }
    template <class V>
    __device__ __forceinline__ void store(uint32_t byte_off, V v) const {
        static_assert(sizeof(V) == 16, "16-byte stores");
        constexpr int kSc1 = 16;  // cache-policy bit SC1 of gfx940-family buffer instructions
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(uint4_t, v), r, (int)byte_off, 0, kSc1);
    }
};

// v_mfma_f32_32x32x16_f16. Operand a: lane l holds row (l % 32), k-slice
// 8*(l / 32) .. +7; operand b: lane l holds column (l % 32), the same
// k-slice. The 16 results of lane l are rows 8*(r/4) + 4*(l/32) + r%4,
// column l % 32. Any permutation of k inside the instruction applies to both
// operands alike, so only the row/column placement matters to callers.
__device__ __forceinline__ float16_t mfma32x32x16(half8_t a, half8_t b, float16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

typedef short short4_t __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16 (gfx950 LDS transpose read). Within each group of 16
// lanes, lane j receives element j % 4 of the 8-byte words addressed by lanes
// j/4, j/4 + 4, j/4 + 8 and j/4 + 12, in that order. If lane i of the group
// addresses row r0 + i/4, columns c0 + 4*(i%4) .. +3 of a row-major f16
// matrix, lane j gets column c0 + j of rows r0 .. r0+3. p must be 8-byte
// aligned and point into LDS.
__device__ __forceinline__ half4_t lds_read_tr16(const half_t* p) {
    const short4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_t*)p);
    return __builtin_bit_cast(half4_t, v);
}

// Waits for this wave's LDS reads and writes, then joins the workgroup
// barrier; global loads stay in flight (__syncthreads() would also drain
// them: its workgroup release fence waits on vmcnt(0)). The memory clobber
// keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Orders this wave's earlier LDS writes before its later LDS reads (of words
// other lanes wrote): a wave's LDS instructions complete in issue order, and
// the clobber keeps the compiler from moving LDS accesses across this point.
__device__ __forceinline__ void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// x combined with the same register of lane l ^ 32 (the other half of the
// wave) by v_permlane32_swap, a VALU instruction (__shfl_xor goes through
// LDS with ds_bpermute). With both operands x, the swap returns for every
// lane the pair {x[l], x[l ^ 32]} (in lane-half order), so the sum or max
// of the two results is the pair's, bitwise the same as x + shfl_xor(x, 32).
// Written as inline assembly: this compiler folds the two results of the
// builtin into one when both operands hold the same value. The s_nop pair
// covers the VALU-write -> permlane-read hazard on either side.
__device__ __forceinline__ void half_pair(float x, float& a, float& b) {
    a = x;
    b = x;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}

__device__ __forceinline__ float half_pair_sum(float x) {
    float a, b;
    half_pair(x, a, b);
    return a + b;
}

__device__ __forceinline__ float half_pair_max(float x) {
    float a, b;
    half_pair(x, a, b);
    return fmaxf(a, b);
}

// Fragment order from a 32x32 MFMA result. Lane (l, hi) of the result holds
// row l, columns 8g + 4hi .. +3 in register group g; fragment order wants
// lane (l, hi) to hold columns 8hi .. 8hi+7 of each 16-column block. For
// the block of groups (g0, g1) = (2kk, 2kk+1) that is one exchange: the
// upper half-wave's g0 values swap with the lower half-wave's g1 values
// (v_permlane32_swap), after which every lane holds its 8 columns as
// {g0, g1}. These take the groups' values as 32-bit words (4 f32 values,
// or 4 f16 values packed in 2 words).
__device__ __forceinline__ void frag_swap(float4_t& g0, float4_t& g1) {
    float a0 = g0[0], a1 = g0[1], a2 = g0[2], a3 = g0[3], b0 = g1[0], b1 = g1[1], b2 = g1[2], b3 = g1[3];
    asm("s_nop 1\n\t"
        "v_permlane32_swap_b32 %0, %4\n\t"
        "v_permlane32_swap_b32 %1, %5\n\t"
        "v_permlane32_swap_b32 %2, %6\n\t"
        "v_permlane32_swap_b32 %3, %7\n\t"
        "s_nop 1"
        : "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3), "+v"(b0), "+v"(b1), "+v"(b2), "+v"(b3));
    g0 = float4_t{a0, a1, a2, a3};
    g1 = float4_t{b0, b1, b2, b3};
}

__device__ __forceinline__ half8_t frag_swap(half4_t g0, half4_t g1) {
    uint2_t a = __builtin_bit_cast(uint2_t, g0), b = __builtin_bit_cast(uint2_t, g1);
    uint32_t a0 = a[0], a1 = a[1], b0 = b[0], b1 = b[1];
    asm("s_nop 1\n\t"
        "v_permlane32_swap_b32 %0, %2\n\t"
        "v_permlane32_swap_b32 %1, %3\n\t"
        "s_nop 1"
        : "+v"(a0), "+v"(a1), "+v"(b0), "+v"(b1));
    return __builtin_bit_cast(half8_t, uint4_t{a0, a1, b0, b1});
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// Fragment order of an f16 activation matrix A[rows][K] (K a multiple of 16;
// rows padded to a multiple of 32): fragment (mb, ks) holds rows 32mb ..
// 32mb+31 and columns 16ks .. 16ks+15 as 64 lanes x 8 halfs, lane hi*32 + l
// holding row 32mb + l, columns 16ks + 8hi .. +7 — exactly the operand a
// lane feeds v_mfma_f32_32x32x16_f16 — and fragments are stored mb-major.
// A GEMM then loads its activation operand straight into registers, 1 KB
// contiguous per wave and fragment, with no LDS staging.
// frag_piece: element offset of the 8 halfs holding columns k8 .. k8+7
// (k8 a multiple of 8) of row m.
__device__ __forceinline__ size_t frag_piece(int m, int k8, int K) {
    return ((size_t)(m >> 5) * (K >> 4) + (k8 >> 4)) * 512 + (((k8 >> 3) & 1) * 32 + (m & 31)) * 8;
}

// LayerNorm statistics of one row from its six 64-column partials
// (mean_k, M2_k): mean = avg mean_k, M2 = sum M2_k + 64 * sum (mean_k -
// mean)^2 (Chan et al.'s pairwise combination), var = M2 / 384, eps 1e-5.
struct RowNorm {
    float mean, rstd;
};

// From a row's 12 statistics floats, loaded as three float4 (a, b, c).
__device__ __forceinline__ RowNorm row_norm(float4_t a, float4_t b, float4_t c) {
    const float mk[6] = {a[0], a[2], b[0], b[2], c[0], c[2]};
    const float m2 = (a[1] + a[3]) + (b[1] + b[3]) + (c[1] + c[3]);
    const float mean = (((mk[0] + mk[1]) + (mk[2] + mk[3])) + (mk[4] + mk[5])) * (1.0f / 6.0f);
    float dev = 0.f;
#pragma unroll
    for (int i = 0; i < 6; ++i) dev += (mk[i] - mean) * (mk[i] - mean);
    const float var = (m2 + 64.0f * dev) * (1.0f / kHidden);
    return RowNorm{mean, rsqrtf(var + 1e-5f)};
}

__device__ __forceinline__ RowNorm row_norm(const float* stats, size_t row) {
    const float4_t* p = (const float4_t*)(stats + row * 12);
    return row_norm(p[0], p[1], p[2]);
}

}  // namespace dhx
