/*
 * dinov3_engine.h -- engine-level C ABI: the thin FFI layer a Rust
 * `src/engine.rs` binds in place of the HRX runtime surface it uses today
 * (hrx::{Device, Stream, Buffer, GraphExec, Kernel, Constants} and
 * hrx::loom::{Compiler, Kernels}; engine.rs:1-3). One engine = one device,
 * one HIP stream, resident buffers, one instantiated hipGraph per batch size.
 *
 * Conventions: every function returns 0 on success and nonzero on failure;
 * the message is then available from dhx_last_error(engine) (or
 * dhx_last_error(NULL) when no engine exists yet). After any failed HIP call
 * the engine is poisoned and later calls fail with "session is unusable
 * after a GPU failure" (engine.rs:36, 93, 168-171, 192-201, 204-213).
 * An engine is not thread-safe; separate engines are independent.
 */
#ifndef DINOV3_ENGINE_H
#define DINOV3_ENGINE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct dhx_engine dhx_engine;

/* A byte range of one engine buffer; replaces engine.rs:6-20 `Region`. */
typedef struct dhx_region {
    uint32_t buffer;
    uint64_t offset;
    uint64_t bytes;
} dhx_region;

/* Kernel table; replaces the `specifications()` list (lib.rs:281-300).
 * Scalars and bindings (in order) per kernel:
 *   DHX_K_PATCH_EMBED   s = {images, grid}           b = {pixels f32 NCHW, patch_w f16 [384][768],
 *                                                          patch_b f32 [384], prefix f32 [5][384], x f16}
 *   DHX_K_LAYERNORM     s = {rows}                   b = {x f16, gamma f32, beta f32, out f16}
 *   DHX_K_LAYERNORM_F32 s = {rows}                   b = {x f16, gamma f32, beta f32, out f32}
 *   DHX_K_QKV_ROPE      s = {images, grid, tpad}     b = {h f16, qkv_w f16 [1152][384], qkv_b f32,
 *                                                          rope_cos f32 [P][64], rope_sin f32, q, k, v}
 *   DHX_K_ATTENTION     s = {images, grid, tpad}     b = {q, k, v, out f16 [rows][384]}
 *   DHX_K_RESID         s = {rows, k}                b = {a f16 [rows][k], w f16 [384][k], b f32, ls f32, x f16}
 *   DHX_K_SWIGLU        s = {rows}                   b = {h f16, gateup_w f16 [3072][384], gateup_b f32, act f16}
 *   DHX_K_SPLITK        s = {rows, k, splits}        b = {a f16, w f16 [384][k], partials f32 [splits][rows][384]}
 *   DHX_K_SPLITK_REDUCE s = {rows, splits}           b = {partials f32, b f32, ls f32, x f16}
 *   DHX_K_PATCH_EMBED_STATS   s = {images, grid}   b = {pixels, patch_w, patch_b, prefix, prefix_stats f32 [5][12],
 *                                                        x f16, stats f32 [rows][12]}
 *   DHX_K_QKV_ROPE_LN         s = {images, grid, tpad}  b = {x f16, stats, qkv_wln f16 [1152][384], qkv_wsum f32,
 *                                                        qkv_t f32, rope_cos, rope_sin, q, k, v}
 *   DHX_K_RESID_STATS         s = {rows, k}        b = {a, w, b, ls, x, stats}
 *   DHX_K_SWIGLU_LN           s = {rows}           b = {x f16, stats, gateup_wln f16 [3072][384], gateup_wsum f32,
 *                                                        gateup_t f32, act}
 *   DHX_K_SPLITK_REDUCE_STATS s = {rows, splits}   b = {partials, b, ls, x, stats}
 * The *_STATS kernels also write LayerNorm row statistics of the x they
 * produce: stats[row][slot] = (mean, M2) of the f16 values of x in columns
 * 64*slot .. 64*slot+63 (6 slots). The *_LN kernels apply LayerNorm to their
 * input algebraically from those statistics: with W' = gamma (.) W (f16),
 * wsum[n] = sum_k W'[n][k] and t = b + beta . W^T, out = rstd * (x . W'^T -
 * mean * wsum) + t equals LN(x) . W^T + b.
 * The f16 activations x (patch_embed, resid and reduce output, QKV / SwiGLU
 * input with LayerNorm folded in), h (LayerNorm output), attn (attention
 * output) and act (SwiGLU output) are in fragment order, rows padded to a
 * multiple of 32: for A[rows][K], the 8 halfs of row m, columns k8 .. k8+7
 * (k8 % 8 == 0) start at element ((m/32)*(K/16) + k8/16)*512 +
 * ((k8/8)%2*32 + m%32)*8 — each 32-row x 16-column block is the 1 KB operand
 * a wave feeds one v_mfma_f32_32x32x16_f16, so GEMMs load activations straight
 * into registers. Binding sizes count the padded rows. dhx_fragment_order and
 * dhx_row_order convert on the host. The weights of the QKV, residual, SwiGLU
 * and split-K GEMMs (qkv_w, qkv_wln, w [384][k], gateup_w, gateup_wln) are in
 * the same fragment order (their row counts are multiples of 32): the kernels
 * move them into LDS block by block with DMA loads.
 * q, k and v are [images][6] f16 matrices of [tpad][64], each in the same
 * fragment order with K = 64 (rows T .. tpad-1 are never written and must
 * hold finite values for attention: regions from dhx_allocate start zeroed),
 * tpad a multiple of 128 >= T = grid*grid + 5;
 * the RoPE tables hold one row of 64 angles per patch whose columns 32..63
 * repeat 0..31 (as DINOv3's do); the kernels read columns 0..31; k (and k / splits) a multiple
 * of 384 (the GEMM K loop runs stages of 64 six at a time). Every binding's size is
 * checked against these shapes before anything is launched or recorded. */
enum {
    DHX_K_PATCH_EMBED = 0,
    DHX_K_LAYERNORM = 1,
    DHX_K_LAYERNORM_F32 = 2,
    DHX_K_QKV_ROPE = 3,
    DHX_K_ATTENTION = 4,
    DHX_K_RESID = 5,
    DHX_K_SWIGLU = 6,
    DHX_K_SPLITK = 7,
    DHX_K_SPLITK_REDUCE = 8,
    DHX_K_PATCH_EMBED_STATS = 9,
    DHX_K_QKV_ROPE_LN = 10,
    DHX_K_RESID_STATS = 11,
    DHX_K_SWIGLU_LN = 12,
    DHX_K_SPLITK_REDUCE_STATS = 13,
    DHX_KERNEL_COUNT = 14
};

#define DHX_MAX_SCALARS 4
#define DHX_MAX_BINDINGS 12
#define DHX_MAX_BRANCHES 4

/* One dispatch; replaces engine.rs:21-27 `Launch`. The grid is derived from
 * the scalars by each kernel's launcher. */
typedef struct dhx_launch {
    uint32_t kernel;
    uint32_t scalars[DHX_MAX_SCALARS];
    uint32_t n_bindings;
    dhx_region bindings[DHX_MAX_BINDINGS];
} dhx_launch;

/* Host-clock milliseconds around submission and completion; replaces
 * engine.rs:272-284 `ForwardTimings` / `Distribution`. */
typedef struct dhx_distribution {
    double median_ms;
    double p95_ms;
} dhx_distribution;

typedef struct dhx_timings {
    uint64_t samples;
    dhx_distribution graph;
    dhx_distribution direct;
} dhx_timings;

/* engine.rs:40-59 (Engine::new): open the device and create the stream.
 * Fails unless the device is gfx950. */
int dhx_engine_open(int32_t device, dhx_engine **out);
void dhx_engine_free(dhx_engine *e);
const char *dhx_last_error(const dhx_engine *e);

/* engine.rs:60-64 (allocate): zero-initialised device buffer. */
int dhx_allocate(dhx_engine *e, uint64_t bytes, dhx_region *out);
/* engine.rs:65-70 (weight): allocate and upload. */
int dhx_weight(dhx_engine *e, const void *bytes, uint64_t n, dhx_region *out);
/* engine.rs:191-202 (upload). */
int dhx_upload(dhx_engine *e, dhx_region r, const void *bytes, uint64_t n);
/* engine.rs:87-129 (record): validate the launch list, capture it as one
 * hipGraph for `batch` and keep it with its launch list. Recording a batch
 * that already has a graph is a no-op. */
int dhx_record(dhx_engine *e, uint64_t batch, const dhx_launch *launches, uint64_t n);
/* dhx_record for a plan made of independent chains (no counterpart in the
 * reference, whose graph is one chain): launches holds `branches` lists back
 * to back, counts[i] launches each (1 <= branches <= DHX_MAX_BRANCHES). Each
 * list runs in order; different lists may run concurrently (on forked
 * streams inside the graph, and likewise for dhx_dispatch / dhx_benchmark),
 * so they must not write memory another list reads or writes. The model
 * uses this to run halves of a batch side by side, filling the last partial
 * wave of one half's kernels with the other half's work. */
int dhx_record_branches(dhx_engine *e, uint64_t batch, const dhx_launch *launches, const uint64_t *counts,
                        uint32_t branches);
int dhx_has_graph(const dhx_engine *e, uint64_t batch);
/* engine.rs:203-214 (replay): launch the graph recorded for `batch`. */
int dhx_replay(dhx_engine *e, uint64_t batch);
/* Direct dispatch of the launch list recorded for `batch` (the "direct"
 * mode of engine.rs:140-163). */
int dhx_dispatch(dhx_engine *e, uint64_t batch);
int dhx_synchronize(dhx_engine *e);
/* engine.rs:215-218 (reserve_readback): pinned host staging buffer. */
int dhx_reserve_readback(dhx_engine *e, uint64_t bytes);
/* engine.rs:219-269 (read): device -> pinned staging -> caller memory. */
int dhx_read(dhx_engine *e, dhx_region r, void *out, uint64_t n);
/* engine.rs:130-190 (benchmark): samples >= 10; samples + 10 iterations of
 * graph replay and direct dispatch in alternating order, first 10 dropped. */
int dhx_benchmark(dhx_engine *e, uint64_t batch, uint64_t samples, dhx_timings *out);

/* Host-side layout conversion for fragment-order activations (no GPU work,
 * no reference counterpart): rows x k f16 values (k a multiple of 16)
 * between row-major and fragment order; the fragment buffer holds
 * ceil(rows/32)*32*k values (padding rows zero on the way in, dropped on the
 * way out). */
int dhx_fragment_order(const uint16_t *rows_in, uint64_t rows, uint64_t k, uint16_t *frag_out);
int dhx_row_order(const uint16_t *frag_in, uint64_t rows, uint64_t k, uint16_t *rows_out);

/* Pipelined transfers (no reference counterpart; the reference uploads,
 * replays and reads back one chunk at a time, lib.rs:98-112). Two slots,
 * each with a pinned input and a pinned output staging buffer, a stream for
 * uploads and one for readbacks, so chunk i+1's host copy and upload overlap
 * chunk i's graph, and chunk i's readback overlaps chunk i+1's graph. Host
 * copies into and out of staging run on several threads. Slot s's graphs
 * must read their input from the region dhx_copy_in filled for slot s and
 * write their output to the region dhx_copy_out reads for slot s.
 *   dhx_reserve_staging: allocate the staging buffers (in_bytes / out_bytes
 *     per slot) and the streams and events.
 *   dhx_copy_in: wait until slot s's previous upload has left its staging
 *     buffer, copy n bytes from host into it, then upload them to dst once
 *     slot s's previous graph is done with dst.
 *   dhx_replay_slot: launch `batch`'s graph after slot s's upload and after
 *     slot s's previous readback (which reads the graph's output region).
 *   dhx_copy_out: read back n bytes of src into slot s's staging buffer once
 *     slot s's graph is done.
 *   dhx_copy_out_finish: wait for that readback and copy it to host memory. */
#define DHX_STAGING_SLOTS 2
int dhx_reserve_staging(dhx_engine *e, uint64_t in_bytes, uint64_t out_bytes);
int dhx_copy_in(dhx_engine *e, dhx_region dst, const void *src, uint64_t n, uint32_t slot);
int dhx_replay_slot(dhx_engine *e, uint64_t batch, uint32_t slot);
int dhx_copy_out(dhx_engine *e, dhx_region src, uint64_t n, uint32_t slot);
int dhx_copy_out_finish(dhx_engine *e, void *dst, uint64_t n, uint32_t slot);

/* No reference counterpart (measurement hook): average device time of each
 * launch of `batch`'s list, from HIP events on the engine's stream over
 * `iters` direct dispatches of that launch alone. ms_out has one slot per
 * launch; kernel_out (optional) receives each launch's kernel id. */
int dhx_launch_timings(dhx_engine *e, uint64_t batch, uint32_t iters, double *ms_out,
                       uint32_t *kernel_out, uint64_t capacity, uint64_t *count);

/* No reference counterpart (test hook): make the next HIP-facing engine call
 * fail as if the runtime had returned an error, to exercise poisoning. */
int dhx_test_fail_next_call(dhx_engine *e);

#ifdef __cplusplus
}
#endif
#endif
