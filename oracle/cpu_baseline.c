/*
 * CPU BASELINE -- benchmark infrastructure, not the oracle and not product code.
 *
 * bench.py's CPU-baseline leg times this file on the host cores: one decode token through one
 * routed-expert MoE layer, written as a CPU implementation would be, not as a checker:
 *   - router: logits = x . W_r^T (+ bias) in fp32, softmax over the experts, top-k,
 *     renormalised or not (the rule the reference restates at bigrig_engine/stream.py:895,
 *     1436-1439 and adapter.py:75-93);
 *   - each selected expert: gate/up and down as fp32 GEMVs that dequantize MLX affine 4-bit
 *     (group 64, bf16 or fp16 scale + bias) on the fly, folding each group's affine map into the
 *     dot product: sum_i (s q_i + b) x_i = s sum_i q_i x_i + b sum_i x_i, with the group sums of
 *     x computed once per input (bigrig_engine/stream.py:1605-1631, precision.py:186-189);
 *   - SwiGLU h = silu(gate) * up, down, then out = sum_j w_j y_j (stream.py:1164-1166,
 *     1523-1525).
 * Accumulation is fp32 throughout; output rows are rounded to bf16 once, at the end. The
 * loops are written so gcc vectorizes them (AVX2 + FMA) and OpenMP splits the output rows of
 * all selected experts over the threads.
 *
 * The oracle (moe_oracle.c) is the reference result the tests compare against; this file is
 * only timed. Its output is checked against the oracle in tests/test_cpu_baseline.py so the
 * timed work is the real layer.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float cb_bf2f(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline float cb_h2f(uint16_t h) {
    const uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(m | 0x400u), (int)e - 25);
    return s ? -v : v;
}

static inline uint16_t cb_f2bf(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* One projection of an expert in blob layout: weight [n_out, n_in / 2] bytes (two codes per
 * byte, low nibble first), then scales [n_out, n_in / 64] and biases [n_out, n_in / 64] (16-bit). */
typedef struct {
    const uint8_t* w;
    const uint16_t* s;
    const uint16_t* b;
} cb_proj;

static cb_proj cb_projection(const uint8_t* expert, int64_t off, int n_out, int n_in) {
    cb_proj p;
    const int64_t G = n_in / 64;
    p.w = expert + off;
    p.s = (const uint16_t*)(expert + off + (int64_t)n_out * n_in / 2);
    p.b = p.s + (int64_t)n_out * G;
    return p;
}

/* x split by parity for each group of 64: xe[g][j] = x[64 g + 2 j], xo[g][j] = x[64 g + 2 j + 1],
 * so byte j of a group's 32 weight bytes meets (xe[j], xo[j]); xs[g] = the group's sum. */
static void cb_prep(const float* x, int n_in, float* xe, float* xo, float* xs) {
    const int G = n_in / 64;
    for (int g = 0; g < G; ++g) {
        float s = 0.0f;
        for (int j = 0; j < 32; ++j) {
            xe[g * 32 + j] = x[64 * g + 2 * j];
            xo[g * 32 + j] = x[64 * g + 2 * j + 1];
            s += x[64 * g + 2 * j] + x[64 * g + 2 * j + 1];
        }
        xs[g] = s;
    }
}

/* row n of a 4-bit affine projection . x (prepared by cb_prep) */
static inline float cb_row(const cb_proj* p, int n, int n_in, int f16, const float* xe, const float* xo,
                           const float* xs) {
    const int G = n_in / 64;
    const uint8_t* wr = p->w + (int64_t)n * n_in / 2;
    float acc = 0.0f;
    for (int g = 0; g < G; ++g) {
        const uint8_t* wb = wr + 32 * g;
        const float* e = xe + 32 * g;
        const float* o = xo + 32 * g;
        float d = 0.0f;
        for (int j = 0; j < 32; ++j) d += (float)(wb[j] & 15) * e[j] + (float)(wb[j] >> 4) * o[j];
        const uint16_t sv = p->s[(int64_t)n * G + g], bv = p->b[(int64_t)n * G + g];
        const float s = f16 ? cb_h2f(sv) : cb_bf2f(sv), b = f16 ? cb_h2f(bv) : cb_bf2f(bv);
        acc += s * d + b * xs[g];
    }
    return acc;
}

/*
 * One decode token through one layer. x [H] bf16; w_router [E, H] bf16; bias [E] fp32 or NULL;
 * expert e's bytes at experts + e * stride (gate, up, down projections in blob order);
 * renorm: divide the k weights by their sum; out [H] bf16. Only 4-bit affine group-64 SwiGLU
 * layers (the configuration the baseline is timed on): returns -1 for anything else.
 */
int cpb_decode_layer(const uint16_t* x, const uint16_t* w_router, const float* bias, int H, int I, int E,
                     int k, int renorm, int scale_f16, const uint8_t* experts, int64_t stride,
                     uint16_t* out, int nthreads) {
    if (H % 64 || I % 64 || k < 1 || k > E || k > 64) return -1;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#endif
    float* xf = (float*)malloc(sizeof(float) * H);
    float* logits = (float*)malloc(sizeof(float) * E);
    float* xe = (float*)malloc(sizeof(float) * H / 2);
    float* xo = (float*)malloc(sizeof(float) * H / 2);
    float* xs = (float*)malloc(sizeof(float) * H / 64);
    float* gu = (float*)malloc(sizeof(float) * 2 * (size_t)k * I);
    float* h = (float*)malloc(sizeof(float) * (size_t)k * I);
    float* he = (float*)malloc(sizeof(float) * (size_t)k * I / 2);
    float* ho = (float*)malloc(sizeof(float) * (size_t)k * I / 2);
    float* hs = (float*)malloc(sizeof(float) * (size_t)k * I / 64);
    float* y = (float*)malloc(sizeof(float) * (size_t)k * H);
    int sel[64];
    float wsel[64];
    for (int i = 0; i < H; ++i) xf[i] = cb_bf2f(x[i]);
    /* router */
#pragma omp parallel for schedule(static)
    for (int e = 0; e < E; ++e) {
        const uint16_t* wr = w_router + (int64_t)e * H;
        float acc = 0.0f;
        for (int i = 0; i < H; ++i) acc += xf[i] * cb_bf2f(wr[i]);
        logits[e] = acc + (bias ? bias[e] : 0.0f);
    }
    float mx = logits[0];
    for (int e = 1; e < E; ++e) mx = logits[e] > mx ? logits[e] : mx;
    float den = 0.0f;
    for (int e = 0; e < E; ++e) den += expf(logits[e] - mx);
    for (int j = 0; j < k; ++j) {
        int best = -1;
        for (int e = 0; e < E; ++e) {
            int taken = 0;
            for (int q = 0; q < j; ++q) taken |= sel[q] == e;
            if (!taken && (best < 0 || logits[e] > logits[best])) best = e;
        }
        sel[j] = best;
        wsel[j] = expf(logits[best] - mx) / den;
    }
    if (renorm) {
        float s = 0.0f;
        for (int j = 0; j < k; ++j) s += wsel[j];
        for (int j = 0; j < k; ++j) wsel[j] /= s;
    }
    /* gate/up of every selected expert: rows (j, n) of gate then up, all in one parallel loop */
    cb_prep(xf, H, xe, xo, xs);
    const int64_t gate_off = 0;
    const int64_t proj_gu = (int64_t)I * H / 2 + 2 * (int64_t)I * (H / 64) * 2;
    const int64_t down_off = 2 * proj_gu;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < 2 * k * I; ++r) {
        const int j = r / (2 * I), rem = r % (2 * I), which = rem / I, n = rem % I;
        const uint8_t* ex = experts + (int64_t)sel[j] * stride;
        const cb_proj p = cb_projection(ex, gate_off + which * proj_gu, I, H);
        gu[r] = cb_row(&p, n, H, scale_f16, xe, xo, xs);
    }
    for (int j = 0; j < k; ++j)
        for (int n = 0; n < I; ++n) {
            const float g = gu[(size_t)j * 2 * I + n], u = gu[(size_t)j * 2 * I + I + n];
            h[(size_t)j * I + n] = g / (1.0f + expf(-g)) * u;
        }
    for (int j = 0; j < k; ++j)
        cb_prep(h + (size_t)j * I, I, he + (size_t)j * I / 2, ho + (size_t)j * I / 2, hs + (size_t)j * I / 64);
    /* down of every selected expert */
#pragma omp parallel for schedule(static)
    for (int r = 0; r < k * H; ++r) {
        const int j = r / H, n = r % H;
        const uint8_t* ex = experts + (int64_t)sel[j] * stride;
        const cb_proj p = cb_projection(ex, down_off, H, I);
        y[r] = cb_row(&p, n, I, scale_f16, he + (size_t)j * I / 2, ho + (size_t)j * I / 2, hs + (size_t)j * I / 64);
    }
    for (int n = 0; n < H; ++n) {
        float acc = 0.0f;
        for (int j = 0; j < k; ++j) acc += wsel[j] * y[(size_t)j * H + n];
        out[n] = cb_f2bf(acc);
    }
    free(xf); free(logits); free(xe); free(xo); free(xs); free(gu); free(h); free(he); free(ho);
    free(hs); free(y);
    return 0;
}

int cpb_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
