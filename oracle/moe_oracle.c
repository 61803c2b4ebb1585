/*
 * ORACLE -- test infrastructure, never product code.
 *
 * A plain-C restatement of the routed-expert MoE layer the reference computes through MLX:
 * the router of the MoE block (softmax over experts, top-k, optional renormalisation, as the
 * reference restates it at bigrig_engine/stream.py:895 and 1436-1439 and describes the rule
 * at bigrig_engine/adapter.py:75-93), MLX affine / MXFP4 dequantization (`mx.dequantize`,
 * bigrig_engine/precision.py:186-189) at any affine width MLX packs, the per-(token, expert)
 * SwitchGLU arithmetic `down(act(up, gate))` or the two-layer SwitchMLP `fc2(silu(fc1 x))`
 * (stream.py:1164-1169, 1270-1271; by-hand oracle
 * tests/test_plan_invariance.py:148-163) and the caller's router-weighted combine
 * (stream.py:1523-1525).
 *
 * Only tests/, the smoke check and bench.py's CPU-baseline leg load this file's library.
 *
 * Bit-exactness contract with the HIP kernels:
 *   - router logits: lane l of a 64-wide wave accumulates chunks c = l, l+64, ... of 8
 *     elements with fmaf in element order; the 64 partials are then summed pairwise
 *     a[i] += a[i+s] for s = 32, 16, ..., 1 (the result of an xor butterfly). Top-k is taken
 *     on the logits, descending, ties to the lower expert id. Indices are therefore identical
 *     bit for bit; routing weights use expf and agree to a few ulps.
 *   - dequant: s*q is exact in fp32, so s*q + b has a single rounding: bit-exact.
 *   - layer outputs: fp32 accumulation in a different order than the kernels; compared at a
 *     relative L2 tolerance. Rounding points mirrored: h = act(...) stored as bf16, y rows
 *     rounded to bf16, out = bf16(sum_j w_j * y_j (+ shared)).
 *
 * Built with -ffp-contract=off so that fmaf() is the only fused operation.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bf2f(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline uint16_t f2bf(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static inline float h2f(uint16_t h) {
    uint32_t s = (h >> 15) & 1u, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexpf((float)(m | 0x400u), (int)e - 25);
    return s ? -v : v;
}

static const float E2M1[16] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
                               -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

/* ------------------------------------------------------------------ router */

/* x [H] bf16 . w [H] (fp32 if w_f32 else bf16) in the kernels' order. H % 8 == 0. */
float orc_dot_lane_tree(const uint16_t* x, const void* w, int w_f32, int H) {
    float a[64];
    int nch = H / 8;
    for (int l = 0; l < 64; ++l) {
        float acc = 0.0f;
        for (int c = l; c < nch; c += 64) {
            for (int i = 0; i < 8; ++i) {
                int h = 8 * c + i;
                float wv = w_f32 ? ((const float*)w)[h] : bf2f(((const uint16_t*)w)[h]);
                acc = fmaf(bf2f(x[h]), wv, acc);
            }
        }
        a[l] = acc;
    }
    for (int s = 32; s >= 1; s >>= 1)
        for (int i = 0; i < s; ++i) a[i] = a[i] + a[i + s];
    return a[0];
}

/* e^x as x = n ln2 + r (|r| <= ln2 / 2; ln2 split into a 12-bit head and a tail, Cody-Waite),
 * e^r by its Taylor polynomial of degree 7 in Horner form with fused multiply-adds, scaled by
 * 2^n. Every step is one correctly rounded operation, so the kernels' copy of this function
 * gives the same bits; within 2 ulp of e^x. Used for the sigmoid routing scores, whose
 * ordering must agree bit for bit. */
float orc_exp_rt(float x) {
    if (x > 88.5f) return INFINITY;
    if (x < -104.0f) return 0.0f;
    const float n = rintf(x * 1.44269502f);
    float r = fmaf(-n, 0.693115234375f, x);
    r = fmaf(-n, 3.19461833e-05f, r);
    float p = 1.98412701e-04f;
    p = fmaf(p, r, 1.38888892e-03f);
    p = fmaf(p, r, 8.33333377e-03f);
    p = fmaf(p, r, 4.16666679e-02f);
    p = fmaf(p, r, 1.66666672e-01f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)n);
}

static float sigmoid_rt(float v) { return 1.0f / (1.0f + orc_exp_rt(-v)); }

/* Selection values of one token (mode 3/4: sigmoid(logit) + bias; else the logit), with the
 * experts outside the topk_group best of n_group contiguous groups taken out (sigmoid: 0;
 * softmax: never picked, marked in `out`). A group scores its largest logit (softmax) or the
 * sum of its two largest selection values (sigmoid), following mlx_lm's group_expert_select /
 * group_limited_greedy (DeepSeek-V3 / V2 routers; the rule adapter.py:75-93 names). Group ties
 * go to the lower group. */
static void orc_select_values(const float* lg, const float* bias, int E, int mode, int n_group,
                              int topk_group, float* c, unsigned char* out) {
    const int sig = mode >= 3;
    for (int e = 0; e < E; ++e) {
        c[e] = sig ? sigmoid_rt(lg[e]) + (bias ? bias[e] : 0.0f) : lg[e];
        out[e] = 0;
    }
    if (n_group <= 1) return;
    const int G = E / n_group;
    float gs[64];
    for (int g = 0; g < n_group; ++g) {
        /* the largest value and the largest of the rest (one holder of the maximum set aside) */
        int i1 = -1;
        for (int e = g * G; e < (g + 1) * G; ++e)
            if (i1 < 0 || c[e] > c[i1]) i1 = e;
        float second = -INFINITY;
        for (int e = g * G; e < (g + 1) * G; ++e)
            if (e != i1 && c[e] > second) second = c[e];
        gs[g] = sig ? c[i1] + second : c[i1];
    }
    unsigned char keep[64] = {0};
    for (int r = 0; r < topk_group; ++r) {
        int best = -1;
        for (int g = 0; g < n_group; ++g)
            if (!keep[g] && (best < 0 || gs[g] > gs[best])) best = g;
        keep[best] = 1;
    }
    for (int e = 0; e < E; ++e)
        if (!keep[e / G]) {
            if (sig) c[e] = 0.0f;
            else out[e] = 1;
        }
}

/* logits [T, E]; idx [T, k]; wts [T, k]; mode 0 softmax-topk, 1 + renorm, 2 topk-softmax,
 * 3 sigmoid-topk (select on sigmoid + bias, weigh sigmoid), 4 + renorm. Softmax modes add `bias`
 * to the logits; sigmoid modes use it for selection only. n_group > 1 limits the top-k to the
 * topk_group best groups; every weight is multiplied by `scale`.
 * shared_gate_w [H] bf16 or NULL -> sgate [T] = sigmoid(dot). Returns 0, or -1 on bad args. */
int orc_router(const uint16_t* x, const void* w, int w_f32, const float* bias,
               const uint16_t* shared_gate_w, int T, int H, int E, int k, int mode,
               int n_group, int topk_group, float scale,
               float* logits, int32_t* idx, float* wts, float* sgate) {
    if (H % 8 || k < 1 || k > E || E < 1 || mode < 0 || mode > 4) return -1;
    if (n_group > 1 && (n_group > 64 || E % n_group || topk_group < 1 || topk_group > n_group ||
                        k > topk_group * (E / n_group)))
        return -1;
    const int sig = mode >= 3;
    float* c = (float*)malloc(sizeof(float) * (size_t)E);
    unsigned char* taken = (unsigned char*)malloc((size_t)E);
    for (int t = 0; t < T; ++t) {
        const uint16_t* xt = x + (size_t)t * H;
        float* lg = logits + (size_t)t * E;
        for (int e = 0; e < E; ++e) {
            const void* we = w_f32 ? (const void*)((const float*)w + (size_t)e * H)
                                   : (const void*)((const uint16_t*)w + (size_t)e * H);
            float v = orc_dot_lane_tree(xt, we, w_f32, H);
            if (bias && !sig) v = v + bias[e];
            lg[e] = v;
        }
        orc_select_values(lg, sig ? bias : NULL, E, mode, n_group, topk_group, c, taken);
        for (int r = 0; r < k; ++r) {
            int best = -1;
            for (int e = 0; e < E; ++e)
                if (!taken[e] && (best < 0 || c[e] > c[best])) best = e;
            taken[best] = 1;
            idx[(size_t)t * k + r] = best;
        }
        float* wt = wts + (size_t)t * k;
        const int32_t* it = idx + (size_t)t * k;
        if (sig) {
            for (int r = 0; r < k; ++r) wt[r] = sigmoid_rt(lg[it[r]]);
            if (mode == 4) {
                float z = 0.0f;
                for (int r = 0; r < k; ++r) z += wt[r];
                for (int r = 0; r < k; ++r) wt[r] = wt[r] / z;
            }
        } else {
            float m = lg[it[0]];
            if (mode == 2) {
                float s = 0.0f;
                for (int r = 0; r < k; ++r) s += expf(lg[it[r]] - m);
                for (int r = 0; r < k; ++r) wt[r] = expf(lg[it[r]] - m) / s;
            } else {
                float s = 0.0f;
                for (int e = 0; e < E; ++e) s += expf(lg[e] - m);
                for (int r = 0; r < k; ++r) wt[r] = expf(lg[it[r]] - m) / s;
                if (mode == 1) {
                    float z = 0.0f;
                    for (int r = 0; r < k; ++r) z += wt[r];
                    for (int r = 0; r < k; ++r) wt[r] = wt[r] / z;
                }
            }
        }
        for (int r = 0; r < k; ++r) wt[r] = wt[r] * scale;
        if (shared_gate_w && sgate) {
            float d = orc_dot_lane_tree(xt, shared_gate_w, 0, H);
            sgate[t] = 1.0f / (1.0f + expf(-d));
        }
    }
    free(c);
    free(taken);
    return 0;
}

/* ------------------------------------------------------------------ layout + dequant */

typedef struct {
    int H, I, quant_mode, bits, gs, scale_f16, has_bias, act;
    float alpha, limit;
} orc_layer;

/* component offsets of one expert with intermediate width `inter` */
typedef struct { int64_t w[3], s[3], b[3], bias[3], total; } orc_off;

static void proj_dims(const orc_layer* L, int inter, int p, int* n_out, int* n_in) {
    if (p < 2) { *n_out = inter; *n_in = L->H; }
    else { *n_out = L->H; *n_in = inter; }
}

/* act 2 (a plain two-layer expert) packs fc1 then fc2: projection slots 0 and 2, slot 1 absent */
void orc_offsets(const orc_layer* L, int inter, orc_off* o) {
    int64_t pos = 0;
    for (int p = 0; p < 3; ++p) {
        if (p == 1 && L->act == 2) {
            o->w[1] = o->s[1] = o->b[1] = o->bias[1] = -1;
            continue;
        }
        int n_out, n_in;
        proj_dims(L, inter, p, &n_out, &n_in);
        int64_t G = n_in / L->gs;
        o->w[p] = pos; pos += (int64_t)n_out * n_in * L->bits / 8;
        if (L->quant_mode == 2) {            /* unquantized bf16: the weight alone */
            o->s[p] = o->b[p] = -1;
        } else if (L->quant_mode == 0) {
            o->s[p] = pos; pos += (int64_t)n_out * G * 2;
            o->b[p] = pos; pos += (int64_t)n_out * G * 2;
        } else {
            o->s[p] = pos; pos += (int64_t)n_out * G;
            o->b[p] = -1;
        }
        if (L->has_bias) { o->bias[p] = pos; pos += (int64_t)n_out * 2; }
        else o->bias[p] = -1;
    }
    o->total = pos;
}

static inline float scale_val(const orc_layer* L, const uint8_t* base, int64_t off, int64_t i) {
    uint16_t v;
    memcpy(&v, base + off + 2 * i, 2);
    return L->scale_f16 ? h2f(v) : bf2f(v);
}

/* Code k of a packed row: MLX packs every width least significant bit first, whole uint32
 * words for 2/4/8 bits and byte-aligned runs for 3/5/6 (8 values in 3 bytes for 3 bits), so in
 * both cases code k occupies bits [bits*k, bits*k + bits) of the row's little-endian bytes. */
static inline uint32_t qcode(const uint8_t* wrow, int k, int bits) {
    const int64_t pos = (int64_t)bits * k;
    const int sh = (int)(pos & 7);
    uint32_t v = wrow[pos >> 3];
    if (sh + bits > 8) v |= (uint32_t)wrow[(pos >> 3) + 1] << 8;
    return (v >> sh) & ((1u << bits) - 1u);
}

static inline int64_t row_bytes(const orc_layer* L, int n_in) { return (int64_t)n_in * L->bits / 8; }

/* The layer's quantization is one this restatement takes: affine 2-8 bits, MXFP4 (4 bits), or
 * unquantized bf16 (mode 2, 16 bits). */
static int orc_quant_ok(const orc_layer* L) {
    if (L->quant_mode == 2) return L->bits == 16;
    return L->bits >= 2 && L->bits <= 8 && (L->quant_mode == 0 || L->bits == 4);
}

/* fp32 dequantized projection p: out [n_out, n_in] (unquantized: the bf16 values). */
int orc_dequant(const orc_layer* L, const uint8_t* expert, int inter, int p, float* out) {
    if (!orc_quant_ok(L)) return -1;
    orc_off o;
    orc_offsets(L, inter, &o);
    if (o.w[p] < 0) return -1;
    int n_out, n_in;
    proj_dims(L, inter, p, &n_out, &n_in);
    int G = n_in / L->gs;
    for (int n = 0; n < n_out; ++n) {
        const uint8_t* wrow = expert + o.w[p] + (int64_t)n * row_bytes(L, n_in);
        if (L->quant_mode == 2) {
            for (int k = 0; k < n_in; ++k) {
                uint16_t v;
                memcpy(&v, wrow + 2 * k, 2);
                out[(int64_t)n * n_in + k] = bf2f(v);
            }
            continue;
        }
        for (int k = 0; k < n_in; ++k) {
            uint32_t q = qcode(wrow, k, L->bits);
            int g = k / L->gs;
            float v;
            if (L->quant_mode == 0) {
                float s = scale_val(L, expert, o.s[p], (int64_t)n * G + g);
                float b = scale_val(L, expert, o.b[p], (int64_t)n * G + g);
                v = s * (float)q + b;
            } else {
                uint8_t e = expert[o.s[p] + (int64_t)n * G + g];
                v = (e == 255) ? NAN : E2M1[q] * ldexpf(1.0f, (int)e - 127);
            }
            out[(int64_t)n * n_in + k] = v;
        }
    }
    return 0;
}

/* y[n] = sum_k W[n,k] x[k] (+ bias[n]) with on-the-fly dequant, fp32 accumulation per group
 * (affine as s*sum(q x) + b*sum(x)) and a double accumulator across groups. */
static void orc_gemv(const orc_layer* L, const uint8_t* expert, const orc_off* o, int inter,
                     int p, const float* x, float* y) {
    int n_out, n_in;
    proj_dims(L, inter, p, &n_out, &n_in);
    int G = n_in / L->gs, gs = L->gs;
    for (int n = 0; n < n_out; ++n) {
        const uint8_t* wrow = expert + o->w[p] + (int64_t)n * row_bytes(L, n_in);
        double acc = 0.0;
        for (int g = 0; g < G; ++g) {
            const float* xg = x + (int64_t)g * gs;
            const uint8_t* wg = wrow + (int64_t)g * gs / 2;
            if (L->quant_mode == 2) {
                /* unquantized bf16: fp32 sum per chunk of gs, like the scaled modes */
                float sw = 0.0f;
                for (int i = 0; i < gs; ++i) {
                    uint16_t v;
                    memcpy(&v, wrow + 2 * ((int64_t)g * gs + i), 2);
                    sw += bf2f(v) * xg[i];
                }
                acc += (double)sw;
            } else if (L->quant_mode == 0) {
                float sqx = 0.0f, sx = 0.0f;
                for (int i = 0; i < gs / 2; ++i) {
                    const int k = g * gs + 2 * i;
                    float q0 = (float)qcode(wrow, k, L->bits), q1 = (float)qcode(wrow, k + 1, L->bits);
                    sqx += q0 * xg[2 * i] + q1 * xg[2 * i + 1];
                    sx += xg[2 * i] + xg[2 * i + 1];
                }
                float s = scale_val(L, expert, o->s[p], (int64_t)n * G + g);
                float b = scale_val(L, expert, o->b[p], (int64_t)n * G + g);
                acc += (double)s * sqx + (double)b * sx;
            } else {
                float sv = 0.0f;
                for (int i = 0; i < gs / 2; ++i) {
                    uint8_t byte = wg[i];
                    sv += E2M1[byte & 0xF] * xg[2 * i] + E2M1[byte >> 4] * xg[2 * i + 1];
                }
                uint8_t e = expert[o->s[p] + (int64_t)n * G + g];
                acc += (double)sv * ldexp(1.0, (int)e - 127);
            }
        }
        if (o->bias[p] >= 0) {
            uint16_t bv;
            memcpy(&bv, expert + o->bias[p] + 2 * n, 2);
            acc += bf2f(bv);
        }
        y[n] = (float)acc;
    }
}

static inline float act_fn(const orc_layer* L, float g, float u) {
    if (L->act == 0) return g / (1.0f + expf(-g)) * u;
    if (L->act == 2) return g / (1.0f + expf(-g));
    g = fminf(g, L->limit);
    u = fminf(fmaxf(u, -L->limit), L->limit);
    return g / (1.0f + expf(-L->alpha * g)) * (u + 1.0f);
}

/* One (token, expert) row: y [H] fp32 (before bf16 rounding). h is bf16-rounded. */
static void orc_expert_row(const orc_layer* L, const uint8_t* expert, int inter,
                           const float* x, float* y, float* scratch) {
    orc_off o;
    orc_offsets(L, inter, &o);
    float* g = scratch;
    float* u = scratch + inter;
    float* h = scratch + 2 * inter;
    orc_gemv(L, expert, &o, inter, 0, x, g);
    if (L->act == 2) {
        for (int i = 0; i < inter; ++i) u[i] = 0.0f;     /* fc2(silu(fc1 x)): no up projection */
    } else {
        orc_gemv(L, expert, &o, inter, 1, x, u);
    }
    for (int i = 0; i < inter; ++i) h[i] = bf2f(f2bf(act_fn(L, g[i], u[i])));
    orc_gemv(L, expert, &o, inter, 2, h, y);
}

/* The MoE layer for T tokens. experts[e] -> packed bytes of expert e (host). out [T,H] bf16
 * or NULL; yun [T,k,H] bf16 or NULL. nthreads <= 0: OpenMP default. */
int orc_moe_forward(const orc_layer* L, const uint8_t* const* experts, int k,
                    const uint8_t* shared, int shared_inter, const uint16_t* x,
                    const int32_t* idx, const float* w, const float* sgate, int T,
                    uint16_t* out, uint16_t* yun, int nthreads) {
    if (!orc_quant_ok(L)) return -1;
    int H = L->H;
    int maxI = L->I > shared_inter ? L->I : shared_inter;
    int P = T * k;
    float* ybuf = (float*)malloc(sizeof(float) * (size_t)(P + T) * H);
    if (!ybuf) return -2;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#endif
#pragma omp parallel
    {
        float* xf = (float*)malloc(sizeof(float) * (size_t)H);
        float* scr = (float*)malloc(sizeof(float) * (size_t)3 * maxI);
#pragma omp for schedule(dynamic, 1)
        for (int pi = 0; pi < P + (shared ? T : 0); ++pi) {
            int t = pi < P ? pi / k : pi - P;
            for (int h = 0; h < H; ++h) xf[h] = bf2f(x[(size_t)t * H + h]);
            float* y = ybuf + (size_t)pi * H;
            if (pi < P) {
                orc_expert_row(L, experts[idx[pi]], L->I, xf, y, scr);
            } else if (shared) {
                orc_expert_row(L, shared, shared_inter, xf, y, scr);
            }
            for (int h = 0; h < H; ++h) y[h] = bf2f(f2bf(y[h]));
        }
        free(xf);
        free(scr);
    }
    for (int t = 0; t < T; ++t) {
        for (int h = 0; h < H; ++h) {
            float acc = 0.0f;
            for (int j = 0; j < k; ++j)
                acc = fmaf(w[(size_t)t * k + j], ybuf[((size_t)t * k + j) * H + h], acc);
            if (shared && sgate) acc = fmaf(sgate[t], ybuf[((size_t)P + t) * H + h], acc);
            if (out) out[(size_t)t * H + h] = f2bf(acc);
        }
    }
    if (yun)
        for (size_t i = 0; i < (size_t)P * H; ++i) yun[i] = f2bf(ybuf[i]);
    free(ybuf);
    return 0;
}

/* Stable bucketing of pairs by expert: np.argsort(idx.reshape(-1), kind="stable")
 * (stream.py:1526-1530) and the start of each expert's run. */
int orc_sort_pairs(const int32_t* idx, int P, int E, int32_t* order, int32_t* offsets) {
    int32_t* cnt = (int32_t*)calloc((size_t)E + 1, sizeof(int32_t));
    if (!cnt) return -2;
    for (int i = 0; i < P; ++i) {
        if (idx[i] < 0 || idx[i] >= E) { free(cnt); return -1; }
        cnt[idx[i] + 1]++;
    }
    for (int e = 0; e < E; ++e) cnt[e + 1] += cnt[e];
    memcpy(offsets, cnt, sizeof(int32_t) * ((size_t)E + 1));
    for (int i = 0; i < P; ++i) order[cnt[idx[i]]++] = i;
    free(cnt);
    return 0;
}

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
