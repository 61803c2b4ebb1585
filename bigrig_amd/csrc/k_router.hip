// Router top-k: logits = x . W_r^T (+ bias), top-k by logit, routing weights.
//
// Replaces the MoE block's `gate(x)` + softmax + argpartition + take (+ renorm) that the
// reference restates at bigrig_engine/stream.py:895 and 1436-1439 (rule: adapter.py:75-93).
//
// Reduction order (the contract that makes indices reproducible bit for bit): lane l of a
// wave accumulates the 8-element chunks c = l, l+64, ... with fmaf in element order, then the
// 64 partials are combined by an xor butterfly (offsets 32, 16, ..., 1). Top-k is selected
// on the logits, descending, ties to the lower expert id; softmax is monotonic, so this is the
// top-k of the probabilities except at exact fp32 probability ties, where the order is
// defined here rather than left to argpartition.
#include "brx_internal.h"

namespace brx {
namespace {

constexpr int kRouterThreads = 256;
constexpr int kMaxE = 512;
constexpr int kMaxK = 64;  // top-k is held one rank per lane
constexpr int kSmallT = 64;  // up to this many tokens: logits kernel + top-k kernel

__device__ __forceinline__ float wave_sum_xor(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

template <bool WF32>
__device__ __forceinline__ void load_w8(const void* w, int64_t row, int H, int c, float out[8]) {
    if constexpr (WF32) {
        const float4* p = reinterpret_cast<const float4*>(
            reinterpret_cast<const float*>(w) + row * H + 8 * c);
        float4 a = p[0], b = p[1];
        out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
        out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
    } else {
        uint4 v = *reinterpret_cast<const uint4*>(
            reinterpret_cast<const uint16_t*>(w) + row * H + 8 * c);
        uint32_t u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            out[2 * i] = bf2f(u[i] & 0xFFFFu);
            out[2 * i + 1] = bf2f(u[i] >> 16);
        }
    }
}

// One block: TPB tokens, all E (+1 shared-gate) rows. x staged in LDS as fp32.
template <bool WF32, int TPB>
__global__ __launch_bounds__(kRouterThreads) void k_router(
    const uint16_t* __restrict__ x, const void* __restrict__ w, const float* __restrict__ bias,
    const uint16_t* __restrict__ sgw, int T, int H, int E, int k, int mode,
    int32_t* __restrict__ out_idx, float* __restrict__ out_w, float* __restrict__ out_sg) {
    extern __shared__ float smem[];
    float* xs = smem;                              // [TPB][H]
    float* lg = smem + (size_t)TPB * H;            // [TPB][E + 1]
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int t0 = blockIdx.x * TPB;
    const int nt = min(TPB, T - t0);
    const int nch = H / 8;

    for (int i = tid; i < TPB * H; i += kRouterThreads) {
        int t = i / H, h = i - t * H;
        xs[i] = t < nt ? bf2f(x[(int64_t)(t0 + t) * H + h]) : 0.0f;
    }
    __syncthreads();

    const int rows = E + (sgw ? 1 : 0);
    for (int r = wv; r < rows; r += kRouterThreads / kWave) {
        float acc[TPB];
#pragma unroll
        for (int t = 0; t < TPB; ++t) acc[t] = 0.0f;
        for (int c = lane; c < nch; c += kWave) {
            float wv8[8];
            if (r < E) load_w8<WF32>(w, r, H, c, wv8);
            else load_w8<false>(sgw, 0, H, c, wv8);
#pragma unroll
            for (int t = 0; t < TPB; ++t) {
                const float* xt = xs + t * H + 8 * c;
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[t] = fmaf(xt[i], wv8[i], acc[t]);
            }
        }
#pragma unroll
        for (int t = 0; t < TPB; ++t) {
            float s = wave_sum_xor(acc[t]);
            if (lane == 0) lg[t * (E + 1) + r] = (r < E && bias) ? s + bias[r] : s;
        }
    }
    __syncthreads();

    // one wave per token: top-k on logits, then the routing weights
    constexpr int kPer = kMaxE / kWave;
    for (int t = wv; t < nt; t += kRouterThreads / kWave) {
        const float* l = lg + t * (E + 1);
        float v[kPer];
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            int e = lane + kWave * i;
            v[i] = e < E ? l[e] : 0.0f;
        }
        int my_id;
        float my_v;
        wave_topk<kPer>(v, E, k, my_id, my_v);
        const float wt = wave_route_weight<kPer>(v, E, k, mode, my_v);
        const int64_t tt = t0 + t;
        if (lane < k) {
            out_idx[tt * k + lane] = my_id;
            out_w[tt * k + lane] = wt;
        }
        if (lane == 0 && sgw && out_sg) out_sg[tt] = 1.0f / (1.0f + expf(-l[E]));
    }
}

// ---------------------------------------------------------------- small T
// k_router_logits: one wave per (expert row, tile of TT tokens), WPB waves per block; every
// load of the wave is issued before the first FMA. Same per-lane chain and butterfly as
// k_router, so the logits are the same bits.
template <bool WF32, int TT, int WPB>
__global__ __launch_bounds__(WPB * kWave) void k_router_logits(
    const uint16_t* __restrict__ x, const void* __restrict__ w, const float* __restrict__ bias,
    const uint16_t* __restrict__ sgw, int T, int H, int E, float* __restrict__ logits) {
    constexpr int kNJ = 6;                      // chunks per lane: H <= 64 * 8 * 6 = 3072
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * WPB + (threadIdx.x >> 6);
    const int rows = E + (sgw ? 1 : 0);
    const int t0 = blockIdx.y * TT;
    const int nt = min(TT, T - t0);
    const int nch = H / 8;
    if (r >= rows) return;
    const bool wf32 = WF32 && r < E;
    uint4 wv[kNJ][2];
    uint4 xv[TT][kNJ];
#pragma unroll
    for (int j = 0; j < kNJ; ++j) {
        const int c = lane + kWave * j;
        if (c < nch) {
            if (wf32) {
                const uint4* p = reinterpret_cast<const uint4*>(
                    reinterpret_cast<const float*>(w) + (int64_t)r * H + 8 * c);
                wv[j][0] = p[0];
                wv[j][1] = p[1];
            } else {
                const uint16_t* src = r < E ? reinterpret_cast<const uint16_t*>(w) + (int64_t)r * H : sgw;
                wv[j][0] = *reinterpret_cast<const uint4*>(src + 8 * c);
            }
#pragma unroll
            for (int t = 0; t < TT; ++t)
                if (t < nt) xv[t][j] = *reinterpret_cast<const uint4*>(x + (int64_t)(t0 + t) * H + 8 * c);
        }
    }
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < kNJ; ++j) {
            const int c = lane + kWave * j;
            if (c < nch && t < nt) {
                uint32_t xw[4] = {xv[t][j].x, xv[t][j].y, xv[t][j].z, xv[t][j].w};
                float wf[8];
                if (wf32) {
                    wf[0] = __uint_as_float(wv[j][0].x); wf[1] = __uint_as_float(wv[j][0].y);
                    wf[2] = __uint_as_float(wv[j][0].z); wf[3] = __uint_as_float(wv[j][0].w);
                    wf[4] = __uint_as_float(wv[j][1].x); wf[5] = __uint_as_float(wv[j][1].y);
                    wf[6] = __uint_as_float(wv[j][1].z); wf[7] = __uint_as_float(wv[j][1].w);
                } else {
                    uint32_t ww[4] = {wv[j][0].x, wv[j][0].y, wv[j][0].z, wv[j][0].w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        wf[2 * i] = bf2f(ww[i] & 0xFFFFu);
                        wf[2 * i + 1] = bf2f(ww[i] >> 16);
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    acc = fmaf(bf2f(xw[i] & 0xFFFFu), wf[2 * i], acc);
                    acc = fmaf(bf2f(xw[i] >> 16), wf[2 * i + 1], acc);
                }
            }
        }
        float s = wave_sum_xor(acc);
        if (lane == 0 && t < nt) logits[(int64_t)(t0 + t) * (E + 1) + r] = (r < E && bias) ? s + bias[r] : s;
    }
}

// Top-k of one token's logits row `l` ([E + 1], the last entry the shared-gate logit) and its
// routing weights, by the calling wave.
template <int kPer>
__device__ __forceinline__ void topk_row(const float* __restrict__ l, int t, int E, int k, int mode,
                                         int has_sg, int32_t* __restrict__ out_idx,
                                         float* __restrict__ out_w, float* __restrict__ out_sg) {
    const int lane = threadIdx.x & 63;
    float v[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int e = lane + kWave * i;
        v[i] = e < E ? l[e] : 0.0f;
    }
    int my_id;
    float my_v;
    wave_topk<kPer>(v, E, k, my_id, my_v);
    const float wt = wave_route_weight<kPer>(v, E, k, mode, my_v);
    if (lane < k) {
        out_idx[(int64_t)t * k + lane] = my_id;
        out_w[(int64_t)t * k + lane] = wt;
    }
    if (lane == 0 && has_sg && out_sg) out_sg[t] = 1.0f / (1.0f + expf(-l[E]));
}

// One wave per token over logits [T][E + 1].
template <int kPer>
__global__ __launch_bounds__(kRouterThreads) void k_router_topk(
    const float* __restrict__ logits, int T, int E, int k, int mode, int has_sg,
    int32_t* __restrict__ out_idx, float* __restrict__ out_w, float* __restrict__ out_sg) {
    const int t = blockIdx.x * (kRouterThreads / kWave) + (threadIdx.x >> 6);
    if (t >= T) return;
    topk_row<kPer>(logits + (int64_t)t * (E + 1), t, E, k, mode, has_sg, out_idx, out_w, out_sg);
}

template <bool WF32, int TPB>
hipError_t launch_tpb(const brx_layer_desc& d, const void* x, const void* w, const float* bias,
                      const void* sgw, int T, int32_t* out_idx, float* out_w, float* out_sg,
                      hipStream_t s) {
    size_t lds = sizeof(float) * ((size_t)TPB * d.hidden + (size_t)TPB * (d.n_experts + 1));
    dim3 grid((T + TPB - 1) / TPB);
    hipLaunchKernelGGL((k_router<WF32, TPB>), grid, dim3(kRouterThreads), lds, s,
                       (const uint16_t*)x, w, bias, (const uint16_t*)sgw, T, d.hidden,
                       d.n_experts, d.top_k, d.route_mode, out_idx, out_w, out_sg);
    return hipGetLastError();
}

template <bool WF32>
hipError_t logits_launch(const brx_layer_desc& d, const void* x, const void* w_router, const float* bias,
                         const void* sgw, int T, float* logits, hipStream_t s) {
    constexpr int TT = 4, WPB = 1;
    const int rows = d.n_experts + (sgw ? 1 : 0);
    dim3 grid((rows + WPB - 1) / WPB, (T + TT - 1) / TT);
    hipLaunchKernelGGL((k_router_logits<WF32, TT, WPB>), grid, dim3(WPB * kWave), 0, s,
                       (const uint16_t*)x, w_router, bias, (const uint16_t*)sgw, T, d.hidden,
                       d.n_experts, logits);
    return hipGetLastError();
}

hipError_t topk_launch(const brx_layer_desc& d, int T, int has_sg, const float* logits,
                       int32_t* out_idx, float* out_w, float* out_sg, hipStream_t s) {
    const int E = d.n_experts;
    dim3 grid((T + 3) / 4), block(kRouterThreads);
#define BRX_TOPK(KP) hipLaunchKernelGGL(k_router_topk<KP>, grid, block, 0, s, logits, T, E, d.top_k, \
                                        d.route_mode, has_sg, out_idx, out_w, out_sg)
    if (E <= 64) BRX_TOPK(1);
    else if (E <= 128) BRX_TOPK(2);
    else if (E <= 256) BRX_TOPK(4);
    else BRX_TOPK(8);
#undef BRX_TOPK
    return hipGetLastError();
}

}  // namespace

size_t router_workspace_bytes(const brx_layer_desc& d, int T) {
    return T <= kSmallT ? sizeof(float) * (size_t)T * (d.n_experts + 1) : 0;
}

hipError_t launch_router_logits(const brx_layer_desc& d, const void* x, const void* w_router,
                                const float* bias, const void* sgw, int T, float* logits,
                                hipStream_t s) {
    return d.router_dtype == BRX_DT_F32 ? logits_launch<true>(d, x, w_router, bias, sgw, T, logits, s)
                                        : logits_launch<false>(d, x, w_router, bias, sgw, T, logits, s);
}

hipError_t launch_router(const brx_layer_desc& d, const void* x, const void* w_router,
                         const float* bias, const void* sgw, int T, int32_t* out_idx,
                         float* out_w, float* out_sg, float* ws_logits, hipStream_t s) {
    if (T <= 0) return hipSuccess;
    const bool f32 = d.router_dtype == BRX_DT_F32;
    if (T <= kSmallT) {
        hipError_t e = launch_router_logits(d, x, w_router, bias, sgw, T, ws_logits, s);
        if (e != hipSuccess) return e;
        return topk_launch(d, T, sgw ? 1 : 0, ws_logits, out_idx, out_w, out_sg, s);
    }
    // x staged as fp32: keep TPB * H * 4 within 48 KB of LDS
    if (d.hidden <= 2880) {
        return f32 ? launch_tpb<true, 4>(d, x, w_router, bias, sgw, T, out_idx, out_w, out_sg, s)
                   : launch_tpb<false, 4>(d, x, w_router, bias, sgw, T, out_idx, out_w, out_sg, s);
    }
    return f32 ? launch_tpb<true, 1>(d, x, w_router, bias, sgw, T, out_idx, out_w, out_sg, s)
               : launch_tpb<false, 1>(d, x, w_router, bias, sgw, T, out_idx, out_w, out_sg, s);
}

}  // namespace brx
