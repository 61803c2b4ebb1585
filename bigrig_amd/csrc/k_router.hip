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
        bool taken[kPer];
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            int e = lane + kWave * i;
            v[i] = e < E ? l[e] : 0.0f;
            taken[i] = e >= E;
        }
        // rank r's (id, logit) ends up in lane r
        int my_id = -1;
        float my_v = 0.0f;
        for (int r = 0; r < k; ++r) {
            float bv = 0.0f;
            int bid = 0x7fffffff;
#pragma unroll
            for (int i = 0; i < kPer; ++i) {
                int e = lane + kWave * i;
                if (!taken[i] && (bid == 0x7fffffff || v[i] > bv)) { bv = v[i]; bid = e; }
            }
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) {
                float ov = __shfl_xor(bv, off, kWave);
                int oid = __shfl_xor(bid, off, kWave);
                bool better = (oid != 0x7fffffff) &&
                              (bid == 0x7fffffff || ov > bv || (ov == bv && oid < bid));
                if (better) { bv = ov; bid = oid; }
            }
            if (lane == r) { my_id = bid; my_v = bv; }
#pragma unroll
            for (int i = 0; i < kPer; ++i)
                if (lane + kWave * i == bid) taken[i] = true;
        }
        const float m = __shfl(my_v, 0, kWave);
        float wt;
        if (mode == BRX_ROUTE_TOPK_SOFTMAX) {
            float ex = lane < k ? expf(my_v - m) : 0.0f;
            wt = ex / wave_sum_xor(ex);
        } else {
            float part = 0.0f;
#pragma unroll
            for (int i = 0; i < kPer; ++i)
                if (lane + kWave * i < E) part += expf(v[i] - m);
            float s = wave_sum_xor(part);
            wt = lane < k ? expf(my_v - m) / s : 0.0f;
            if (mode == BRX_ROUTE_SOFTMAX_TOPK_RENORM) wt = wt / wave_sum_xor(wt);
        }
        const int64_t tt = t0 + t;
        if (lane < k) {
            out_idx[tt * k + lane] = my_id;
            out_w[tt * k + lane] = wt;
        }
        if (lane == 0 && sgw && out_sg) out_sg[tt] = 1.0f / (1.0f + expf(-l[E]));
    }
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

}  // namespace

hipError_t launch_router(const brx_layer_desc& d, const void* x, const void* w_router,
                         const float* bias, const void* sgw, int T, int32_t* out_idx,
                         float* out_w, float* out_sg, hipStream_t s) {
    if (T <= 0) return hipSuccess;
    // x staged as fp32: keep TPB * H * 4 within 48 KB of LDS
    bool f32 = d.router_dtype == BRX_DT_F32;
    if (T >= 64 && d.hidden <= 2880) {
        return f32 ? launch_tpb<true, 4>(d, x, w_router, bias, sgw, T, out_idx, out_w, out_sg, s)
                   : launch_tpb<false, 4>(d, x, w_router, bias, sgw, T, out_idx, out_w, out_sg, s);
    }
    return f32 ? launch_tpb<true, 1>(d, x, w_router, bias, sgw, T, out_idx, out_w, out_sg, s)
               : launch_tpb<false, 1>(d, x, w_router, bias, sgw, T, out_idx, out_w, out_sg, s);
}

}  // namespace brx
