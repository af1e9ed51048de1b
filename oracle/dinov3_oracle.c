/*
 * dinov3_oracle.c -- TEST INFRASTRUCTURE ONLY (the checker, never the product).
 *
 * A float64 CPU restatement of the reference's numerical oracle
 * (tests/support/reference.rs:1-192 in zacharydenton/dinov3-loom) and of the
 * small host-side algorithms the forward path depends on:
 *   - patchify                 lib.rs:265-280
 *   - float16 packing (RNE)    weights.rs:6-17 (the `half` crate's f16::from_f32)
 *   - RoPE cos/sin tables      weights.rs:127-144
 *   - linear / LayerNorm / 2D axial RoPE / exact softmax attention / SwiGLU /
 *     layerscale residuals / final norm   reference.rs:5-192
 * The 224x224 constants of the reference (14x14 grid, 201 tokens) are
 * generalised to a G x G patch grid (T = G*G + 5 tokens); G = 14 reproduces the
 * reference exactly, G = 32 is the 512x512 configuration.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library. Nothing under dinov3-loom_amd/ links or calls it.
 *
 * How each function is pinned (not by retyping it in a test):
 *   patchify      reference KAT lib.rs:307-327 (ramp input, exact permutation)
 *   f16 packing   reference KAT weights.rs:152-169 + numpy.float16 over random
 *                 bit patterns (independent IEEE RNE implementation)
 *   rope tables   transformers' DINOv3ViTRopePositionEmbedding (third party)
 *   linear / norm / attention / forward
 *                 closed forms and brute force on tiny inputs (constant rows,
 *                 q = 0 gives the mean of V, a single key gives V), plus
 *                 golden vectors from transformers' DINOv3ViTModel in float64
 *                 (tests/golden/make_golden.py).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define H 384
#define HEADS 6
#define HD 64
#define PREFIX 5
#define FF 1536
#define LAYERS 12
#define PATCH_K 768

/* Canonical tensor order of oracle_forward's `tensors` argument (HF names). */
enum {
    T_PATCH_W, T_PATCH_B, T_CLS, T_REG, T_LAYER0,
    L_N1W = 0, L_N1B, L_QW, L_QB, L_KW, L_VW, L_VB, L_OW, L_OB, L_LS1,
    L_N2W, L_N2B, L_GW, L_GB, L_UW, L_UB, L_DW, L_DB, L_LS2, L_COUNT
};
#define T_NORM_W (T_LAYER0 + LAYERS * L_COUNT)
#define T_NORM_B (T_NORM_W + 1)
#define T_COUNT (T_NORM_B + 1)

int oracle_tensor_count(void) { return T_COUNT; }
int oracle_layer_tensor_count(void) { return L_COUNT; }

void oracle_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

int oracle_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* lib.rs:265-280: per image, patches in (gy, gx) order, each patch laid out
 * as (c, dy, dx) = 3 x 16 x 16 floats. The image side is 16*G. */
void oracle_patchify(const float *images, int n_images, int G, float *out) {
    const int S = 16 * G;
    size_t o = 0;
    for (int n = 0; n < n_images; ++n) {
        const float *img = images + (size_t)n * 3 * S * S;
        for (int gy = 0; gy < G; ++gy)
            for (int gx = 0; gx < G; ++gx)
                for (int c = 0; c < 3; ++c)
                    for (int dy = 0; dy < 16; ++dy) {
                        const float *src = img + (size_t)c * S * S + (size_t)(gy * 16 + dy) * S + gx * 16;
                        memcpy(out + o, src, 16 * sizeof(float));
                        o += 16;
                    }
    }
}

/* IEEE 754 binary32 -> binary16, round to nearest, ties to even; the
 * conversion weights.rs:10 performs through half::f16::from_f32. */
static uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t exp = (x >> 23) & 0xffu;
    const uint32_t mant = x & 0x7fffffu;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u | (mant >> 13) : 0u));
    const int e = (int)exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        /* f16 subnormal: m * 2^-24 with m = round(full24 * 2^(exp-126)). */
        const int shift = 126 - (int)exp;
        if (shift > 24) return (uint16_t)sign;
        const uint32_t full = mant | 0x800000u;
        uint32_t m = full >> shift;
        const uint32_t rem = full & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (m & 1u))) ++m;
        return (uint16_t)(sign | m); /* m == 0x400 is the smallest normal */
    }
    uint32_t m = mant >> 13;
    const uint32_t rem = mant & 0x1fffu;
    uint32_t ee = (uint32_t)e;
    if (rem > 0x1000u || (rem == 0x1000u && (m & 1u))) {
        ++m;
        if (m == 0x400u) {
            m = 0;
            ++ee;
            if (ee >= 0x1f) return (uint16_t)(sign | 0x7c00u);
        }
    }
    return (uint16_t)(sign | (ee << 10) | m);
}

static float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    const uint32_t mant = h & 0x3ffu;
    float f;
    if (exp == 0) {
        f = ldexpf((float)mant, -24);
        uint32_t x;
        memcpy(&x, &f, 4);
        x |= sign;
        memcpy(&f, &x, 4);
        return f;
    }
    uint32_t x;
    if (exp == 0x1f) x = sign | 0x7f800000u | (mant << 13);
    else x = sign | ((exp - 15 + 127) << 23) | (mant << 13);
    memcpy(&f, &x, 4);
    return f;
}

void oracle_f32_to_f16(const float *in, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = f32_to_f16(in[i]);
}

void oracle_f16_to_f32(const uint16_t *in, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = f16_to_f32(in[i]);
}

/* weights.rs:127-144 with 14 -> G: per patch (gy, gx), 64 entries laid out as
 * [y x16, x x16, y x16, x x16]; angle = 2*pi*(2(pos+0.5)/G - 1) / 100^(j/16),
 * evaluated in float64 and stored as float32. */
void oracle_rope_tables(int G, float *cos_out, float *sin_out) {
    size_t o = 0;
    for (int y = 0; y < G; ++y)
        for (int x = 0; x < G; ++x)
            for (int rep = 0; rep < 2; ++rep)
                for (int axis = 0; axis < 2; ++axis) {
                    const int pos = axis == 0 ? y : x;
                    for (int j = 0; j < 16; ++j) {
                        const double coord = 2.0 * ((double)pos + 0.5) / (double)G - 1.0;
                        const double a = 2.0 * M_PI * coord / pow(100.0, (double)j / 16.0);
                        cos_out[o] = (float)cos(a);
                        sin_out[o] = (float)sin(a);
                        ++o;
                    }
                }
}

/* reference.rs:5-37: out[m][n] = sum_k x[m][k] * w[n][k] (+ bias[n]).
 * Four rows share each weight row; rows are independent across threads. */
void oracle_linear(const double *x, const double *w, const double *bias, int m, int k, int n, double *out) {
#pragma omp parallel for schedule(static)
    for (int i0 = 0; i0 < m; i0 += 4) {
        const int rows = m - i0 < 4 ? m - i0 : 4;
        for (int j = 0; j < n; ++j) {
            const double *wr = w + (size_t)j * k;
            double acc[4][4] = {{0}};
            int kk = 0;
            for (; kk + 4 <= k; kk += 4)
                for (int r = 0; r < rows; ++r) {
                    const double *xr = x + (size_t)(i0 + r) * k + kk;
                    acc[r][0] += xr[0] * wr[kk];
                    acc[r][1] += xr[1] * wr[kk + 1];
                    acc[r][2] += xr[2] * wr[kk + 2];
                    acc[r][3] += xr[3] * wr[kk + 3];
                }
            for (int r = 0; r < rows; ++r) {
                double s = (acc[r][0] + acc[r][1]) + (acc[r][2] + acc[r][3]);
                for (int t = kk; t < k; ++t) s += x[(size_t)(i0 + r) * k + t] * wr[t];
                out[(size_t)(i0 + r) * n + j] = s + (bias ? bias[j] : 0.0);
            }
        }
    }
}

/* reference.rs:38-48: two-pass mean / biased variance over 384 channels,
 * eps 1e-5, then * gamma + beta. */
void oracle_layernorm(const double *x, const double *g, const double *b, int rows, double *out) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const double *src = x + (size_t)r * H;
        double *dst = out + (size_t)r * H;
        double mean = 0.0;
        for (int c = 0; c < H; ++c) mean += src[c];
        mean /= H;
        double var = 0.0;
        for (int c = 0; c < H; ++c) var += (src[c] - mean) * (src[c] - mean);
        var /= H;
        const double inv = 1.0 / sqrt(var + 1e-5);
        for (int c = 0; c < H; ++c) dst[c] = (src[c] - mean) * inv * g[c] + b[c];
    }
}

/* reference.rs:108-128 with 14 -> G: for patch tokens t >= 5 of one image,
 * channel c of each 64-wide head uses pos = (c%32 < 16) ? patch/G : patch%G,
 * angle = 2*pi*(2(pos+0.5)/G - 1) / 100^((c%16)/16), and
 * out[c] = v[c]*cos + rot[c]*sin with rot[c] = -v[c+32] (c < 32), v[c-32] (c >= 32). */
void oracle_rope(double *values, int T, int G) {
    double buf[HD];
    for (int t = PREFIX; t < T; ++t) {
        const int patch = t - PREFIX;
        for (int head = 0; head < HEADS; ++head) {
            double *v = values + (size_t)t * H + head * HD;
            memcpy(buf, v, sizeof buf);
            for (int c = 0; c < HD; ++c) {
                const int pos = (c % 32 < 16) ? patch / G : patch % G;
                const double angle = 2.0 * M_PI * (2.0 * ((double)pos + 0.5) / (double)G - 1.0) /
                                     pow(100.0, (double)(c % 16) / 16.0);
                const double rot = c < 32 ? -buf[c + 32] : buf[c - 32];
                v[c] = buf[c] * cos(angle) + rot * sin(angle);
            }
        }
    }
}

/* reference.rs:129-151: exact softmax(q k^T * 0.125) v per head and row,
 * over all T keys of the image. q, k, v, ctx are [T][384]. */
void oracle_attention(const double *q, const double *k, const double *v, int T, double *ctx) {
    memset(ctx, 0, sizeof(double) * (size_t)T * H);
#pragma omp parallel
    {
        double *scores = (double *)malloc(sizeof(double) * (size_t)T);
#pragma omp for schedule(static) collapse(2)
        for (int head = 0; head < HEADS; ++head)
            for (int row = 0; row < T; ++row) {
                const double *qr = q + (size_t)row * H + head * HD;
                double mx = -INFINITY;
                for (int col = 0; col < T; ++col) {
                    const double *kr = k + (size_t)col * H + head * HD;
                    double s = 0.0;
                    for (int c = 0; c < HD; ++c) s += qr[c] * kr[c];
                    scores[col] = s * 0.125;
                    if (scores[col] > mx) mx = scores[col];
                }
                double sum = 0.0;
                for (int col = 0; col < T; ++col) {
                    scores[col] = exp(scores[col] - mx);
                    sum += scores[col];
                }
                double *out = ctx + (size_t)row * H + head * HD;
                for (int col = 0; col < T; ++col) {
                    const double a = scores[col] / sum;
                    const double *vr = v + (size_t)col * H + head * HD;
                    for (int c = 0; c < HD; ++c) out[c] += a * vr[c];
                }
            }
        free(scores);
    }
}

/* reference.rs:177-179: silu(g) * u, with silu(g) = g / (1 + exp(-g)). */
void oracle_swiglu(const double *gate, const double *up, size_t n, double *out) {
    for (size_t i = 0; i < n; ++i) out[i] = gate[i] / (1.0 + exp(-gate[i])) * up[i];
}

/* reference.rs:152-161 and 180-189: x[i] += y[i] * ls[i % 384]. */
void oracle_layerscale_residual(double *x, const double *y, const double *ls, int rows) {
    for (size_t i = 0; i < (size_t)rows * H; ++i) x[i] += y[i] * ls[i % H];
}

/* One transformer block of reference.rs:89-190, in place on x [T][384]. */
void oracle_block(double *x, const double *const *lt, int T, int G) {
    const size_t th = (size_t)T * H, tf = (size_t)T * FF;
    double *h = malloc(sizeof(double) * th), *q = malloc(sizeof(double) * th);
    double *k = malloc(sizeof(double) * th), *v = malloc(sizeof(double) * th);
    double *ctx = malloc(sizeof(double) * th), *o = malloc(sizeof(double) * th);
    double *gate = malloc(sizeof(double) * tf), *up = malloc(sizeof(double) * tf);
    oracle_layernorm(x, lt[L_N1W], lt[L_N1B], T, h);
    oracle_linear(h, lt[L_QW], lt[L_QB], T, H, H, q);
    oracle_linear(h, lt[L_KW], NULL, T, H, H, k);
    oracle_linear(h, lt[L_VW], lt[L_VB], T, H, H, v);
    oracle_rope(q, T, G);
    oracle_rope(k, T, G);
    oracle_attention(q, k, v, T, ctx);
    oracle_linear(ctx, lt[L_OW], lt[L_OB], T, H, H, o);
    oracle_layerscale_residual(x, o, lt[L_LS1], T);
    oracle_layernorm(x, lt[L_N2W], lt[L_N2B], T, h);
    oracle_linear(h, lt[L_GW], lt[L_GB], T, H, FF, gate);
    oracle_linear(h, lt[L_UW], lt[L_UB], T, H, FF, up);
    oracle_swiglu(gate, up, tf, gate);
    oracle_linear(gate, lt[L_DW], lt[L_DB], T, FF, H, o);
    oracle_layerscale_residual(x, o, lt[L_LS2], T);
    free(h); free(q); free(k); free(v); free(ctx); free(o); free(gate); free(up);
}

/* reference.rs:49-192 for one image of side 16*G: tensors in the canonical
 * order above (float64), image float32 NCHW [3][16G][16G], out [T][384]. */
void oracle_forward(const double *const *tensors, const float *image, int G, double *out) {
    const int P = G * G, T = P + PREFIX;
    float *pf = malloc(sizeof(float) * (size_t)P * PATCH_K);
    double *patches = malloc(sizeof(double) * (size_t)P * PATCH_K);
    double *x = malloc(sizeof(double) * (size_t)T * H);
    oracle_patchify(image, 1, G, pf);
    for (size_t i = 0; i < (size_t)P * PATCH_K; ++i) patches[i] = pf[i];
    memcpy(x, tensors[T_CLS], sizeof(double) * H);
    memcpy(x + H, tensors[T_REG], sizeof(double) * 4 * H);
    oracle_linear(patches, tensors[T_PATCH_W], tensors[T_PATCH_B], P, PATCH_K, H, x + (size_t)PREFIX * H);
    for (int layer = 0; layer < LAYERS; ++layer)
        oracle_block(x, tensors + T_LAYER0 + layer * L_COUNT, T, G);
    oracle_layernorm(x, tensors[T_NORM_W], tensors[T_NORM_B], T, out);
    free(pf); free(patches); free(x);
}
