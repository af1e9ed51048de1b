/*
 * dinov3.h -- model-level C ABI mirroring the public API of the crate
 * `dinov3-hrx` (src/lib.rs:11-148, 302). The C++ model behind it builds its
 * launch plan on the engine ABI in dinov3_engine.h exactly as lib.rs's
 * `prepare` builds one on the HRX engine.
 *
 * Conventions: 0 = success; on failure the message is returned by
 * dinov3_last_error(model), or dinov3_last_error(NULL) for failures that
 * happen before a model exists (load / from_pretrained / helpers). Messages
 * keep the reference's texts ("max_batch must be 1..=64", "input must contain
 * complete 3×224×224 images", "input must be finite", "tensor patch_w[0]
 * cannot be represented as finite float16: ...", "session is unusable after a
 * GPU failure", ...). A model is not thread-safe; separate models are
 * independent.
 */
#ifndef DINOV3_H
#define DINOV3_H
#include <stddef.h>
#include <stdint.h>
#include "dinov3_engine.h"

#ifdef __cplusplus
extern "C" {
#endif

/* lib.rs:11-13 */
#define DINOV3_IMAGE_ELEMENTS (3 * 224 * 224)
#define DINOV3_TOKENS 201
#define DINOV3_HIDDEN 384

typedef struct dinov3_model dinov3_model;

/* lib.rs:15-27 `Options` {device, max_batch} (default {0, 32}). image_size
 * has no reference counterpart: 0 or 224 is the reference's fixed 224x224;
 * other multiples of 16 (e.g. 512, giving 1029 tokens) select the
 * high-resolution extension with RoPE on the (image_size/16)^2 grid. */
typedef struct dinov3_options {
    int32_t device;
    uint64_t max_batch;
    uint32_t image_size;
} dinov3_options;

/* engine.rs:272-284 */
typedef dhx_distribution dinov3_distribution;
typedef dhx_timings dinov3_timings;

/* lib.rs:20-27 */
void dinov3_options_default(dinov3_options *out);

/* lib.rs:49-88 (DINOv3::load): check max_batch, validate and pack the
 * safetensors file (weights.rs:19-146) before touching the GPU, open the
 * device, upload weights, allocate resident buffers, reserve readback. */
int dinov3_load(const char *path, const dinov3_options *options, dinov3_model **out);

/* lib.rs:40-46 (DINOv3::from_pretrained) on the local Hugging Face cache
 * only (hub.rs:17-54 with downloads disabled: there is no network here). */
int dinov3_from_pretrained(const dinov3_options *options, dinov3_model **out);

/* hub.rs:17-54 (hub::weights) without the download branch: resolve the
 * pinned snapshot path in HF_HUB_CACHE / HF_HOME/hub / ~/.cache/huggingface/hub. */
int dinov3_hub_weights(char *path_out, uint64_t capacity);

/* lib.rs:90-114 (forward): any number of whole images, float32 NCHW; output
 * [images][T][384] float32 (T = 201 at 224x224). out_floats must be at
 * least images*T*384. Zero images succeed with no output. */
int dinov3_forward(dinov3_model *m, const float *pixels, uint64_t n_floats, float *out, uint64_t out_floats);
/* lib.rs:126-132 (cls): token 0 of each image, [images][384]. */
int dinov3_cls(dinov3_model *m, const float *pixels, uint64_t n_floats, float *out, uint64_t out_floats);
/* lib.rs:134-148 (patch_mean): mean of the patch tokens 5.. of each image,
 * accumulated in float32 as `+= v / 196` in token order. */
int dinov3_patch_mean(dinov3_model *m, const float *pixels, uint64_t n_floats, float *out, uint64_t out_floats);
/* lib.rs:116-124 (benchmark): one nonempty batch of at most max_batch
 * images; runs forward once, then dhx_benchmark. */
int dinov3_benchmark(dinov3_model *m, const float *pixels, uint64_t n_floats, uint64_t samples,
                     dinov3_timings *out);
/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). dinov3_forward on device memory, with every
 * intermediate buffer (residual stream, q/k/v, attention and SwiGLU outputs,
 * LayerNorm statistics, split-K slabs) in a fixed array of
 * DINOV3_NOALLOC_SCRATCH_BYTES per GPU, which the library holds from the
 * first model load on that GPU until the process ends, instead of the
 * model's own buffers. pixels: images x 3 x S x S float32 NCHW, out:
 * images x T x 384 float32, both device memory on the model's GPU, 16-byte
 * aligned. The launches (the same kernels and plan as dinov3_forward, so the
 * same results bit for bit) are queued on `stream` (a hipStream_t of that
 * GPU; NULL = the model's own stream) and the call returns without waiting:
 * synchronise the stream before reading `out`. It calls no hipMalloc,
 * hipFree or other allocating routine, records no graph and does not check
 * that the pixels are finite. A batch whose buffers do not fit the array (beyond about 43 images
 * at 224x224, 9 at 512x512) fails with an error naming the sizes, before
 * anything is queued. Every call on one GPU uses that GPU's single array and
 * leaves its data there, so calls on one GPU are run one after another:
 * each call's stream waits (hipStreamWaitEvent, no host wait) for the
 * launches of the call queued before it on that GPU, from any stream,
 * thread or model. A call made while `stream` is being captured into a HIP
 * graph is queued without that wait: replays of the graph use the same
 * array, and the caller must not let them overlap other calls on that GPU.
 * The caller's current device is left as it was. */
#define DINOV3_NOALLOC_SCRATCH_BYTES (64ull << 20)
int dinov3_forward_noalloc(dinov3_model *m, const float *pixels, uint64_t images, float *out, void *stream);
const char *dinov3_last_error(const dinov3_model *m);
void dinov3_free(dinov3_model *m);

/* Shape helpers (no reference counterpart; the reference hard-codes 224). */
uint64_t dinov3_image_elements(const dinov3_model *m);
uint64_t dinov3_tokens(const dinov3_model *m);
/* The model's engine, for callers that time or inspect launches. */
dhx_engine *dinov3_engine(dinov3_model *m);
/* Resident upload + graph replay without readback: stages `images` images
 * (recording the graph if needed) and replays it once; no reference
 * counterpart (the GPU half of forward, for timing). */
int dinov3_stage(dinov3_model *m, const float *pixels, uint64_t n_floats);
int dinov3_replay(dinov3_model *m, uint64_t images);
/* Select the down-projection variant: 0 (default) = residual GEMM at every
 * batch size (the reference's choice for b > 1, lib.rs:226-232; at b = 1 the
 * reference takes split-K, lib.rs:218-225, but here the residual GEMM is
 * faster there too and gives each image the same bits at every batch size),
 * 1 = split-K slabs + reduce at every batch size. Graphs are kept per
 * (batch, variant). */
int dinov3_set_splitk(dinov3_model *m, int mode);
/* LayerNorm plan (no reference counterpart): 1 (default) folds LayerNorm
 * into the QKV and gate/up GEMMs from row statistics written by the kernels
 * that produce the residual stream (62 launches per forward at b > 1);
 * 0 runs separate LayerNorm kernels as the reference does (86 launches).
 * Graphs are kept per (batch, variant). */
int dinov3_set_layernorm_fusion(dinov3_model *m, int on);
/* Image groups run side by side (no reference counterpart): batches of at
 * least 4*n images are cut into n groups (1 <= n <= DHX_MAX_BRANCHES,
 * default 2) recorded as concurrent branches of one graph, so one group's
 * kernels fill the last partial wave of workgroups of the other's. Results
 * are bitwise the same for every n. Graphs are kept per (batch, variant). */
int dinov3_set_branches(dinov3_model *m, uint32_t n);
/* dhx_launch_timings for the plan the model would replay for `images`. */
int dinov3_launch_timings(dinov3_model *m, uint64_t images, uint32_t iters, double *ms_out, uint32_t *kernel_out,
                          uint64_t capacity, uint64_t *count);

/* Seeded random-init weights (no reference counterpart): writes an
 * HF-named float32 safetensors file with every tensor the loader and the
 * oracle read. preset 0 = the BASELINE config (trunc-normal std 0.02 for
 * weights and CLS/register tokens, zero biases, LN gamma 1 beta 0,
 * layerscale 1e-5); preset 1 = stress (nonzero biases, layerscale 1,
 * perturbed LN affine, larger q/k weights). */
int dinov3_write_random_weights(const char *path, uint64_t seed, int preset);
/* Seeded i.i.d. N(0,1) float32 NCHW pixels (no reference counterpart). */
int dinov3_random_pixels(uint64_t seed, uint64_t images, uint32_t image_size, float *out);
/* lib.rs:265-280 (patchify) on the host, for the reference's KAT. */
int dinov3_patchify(const float *pixels, uint64_t images, uint32_t image_size, float *out);
/* weights.rs:6-17 (pack_f16): float32 -> float16 bits with the reference's
 * finite-value check and error text. */
int dinov3_pack_f16(const char *name, const float *values, uint64_t n, uint16_t *out);

#ifdef __cplusplus
}
#endif
#endif
