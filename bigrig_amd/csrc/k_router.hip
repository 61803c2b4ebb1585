// Router top-k: logits = x . W_r^T (+ bias), top-k by logit (or by the sigmoid rules'
// selection values), routing weights.
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
constexpr int kSmallT = 64;  // up to this many tokens: one wave per (row, 4 tokens); above: token tiles
constexpr size_t kMaxBlockLds = 160 * 1024;   // LDS one gfx950 block may allocate

// ---------------------------------------------------------------- many tokens
// k_router_tiled: a block takes a tile of TT tokens (staged in LDS as bf16) and a group of
// rows; each row's weights are loaded once per block and used for all TT tokens, and a wave
// works on two rows at once so each token's activations are converted once for both. Per
// token the lane partials follow the same fmaf chain as k_router_logits; the TT partials are
// reduced by a transposed butterfly that forms exactly the sums of the xor butterfly
// (strides 32, 16, ..., 1; fp32 addition is commutative, so a[i] + a[i^s] is the same value on
// both lanes): at stride 32 a lane keeps half of the tokens and sends the other half, at 16 a
// quarter, and so on, so 16 tokens take 17 exchanges instead of 96. Token tau ends on lanes
// 4 tau .. 4 tau + 3.
template <bool WF32, int TT>
__global__ __launch_bounds__(kRouterThreads) void k_router_tiled(
    const uint16_t* __restrict__ x, const void* __restrict__ w, const float* __restrict__ bias,
    const uint16_t* __restrict__ sgw, int T, int H, int E, int rows_per_block, float* __restrict__ logits) {
    static_assert(TT == 16, "the exchange pattern below is written for 16 tokens");
    constexpr int kNJ = 6;                      // chunks per lane per pass (one pass: H <= 3072)
    constexpr int RW = WF32 ? 2 : 4;            // rows a wave works on at once (sharing x)
    extern __shared__ uint4 xs4[];              // [TT][H / 8] chunks of 8 bf16
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int t0 = blockIdx.x * TT;
    const int nt = min(TT, T - t0);
    const int nch = H / 8;
    const uint4* x4 = reinterpret_cast<const uint4*>(x);
    // kSt chunks a thread in flight at once (token rows clamped into the tile, so every load is
    // unconditional), then the stores: a load and its store per iteration would make each of the
    // TT * nch / kRouterThreads chunks a round trip of its own
    {
        constexpr int kSt = 16;
        const int nall = TT * nch;
        for (int i0 = 0; i0 < nall; i0 += kSt * kRouterThreads) {
            uint4 v[kSt];
#pragma unroll
            for (int b = 0; b < kSt; ++b) {
                const int i = min(i0 + b * kRouterThreads + tid, nall - 1);
                const int t = i / nch, c = i - t * nch;
                v[b] = x4[(int64_t)(t0 + min(t, nt - 1)) * nch + c];
            }
#pragma unroll
            for (int b = 0; b < kSt; ++b) {
                const int i = i0 + b * kRouterThreads + tid;
                if (i < nall) xs4[i] = i / nch < nt ? v[b] : make_uint4(0, 0, 0, 0);
            }
        }
    }
    __syncthreads();
    const int rows = E + (sgw ? 1 : 0);
    const int r_end = min(rows, (int)(blockIdx.y + 1) * rows_per_block);
    constexpr int kWaves = kRouterThreads / kWave;
    for (int r0 = blockIdx.y * rows_per_block + wv * RW; r0 < r_end; r0 += kWaves * RW) {
        // the wave's rows r0, r0 + 1 (a row past the block's range repeats the last one and is
        // not stored)
        float acc[RW][TT];
#pragma unroll
        for (int rr = 0; rr < RW; ++rr)
#pragma unroll
            for (int t = 0; t < TT; ++t) acc[rr][t] = 0.0f;
        bool wf32[RW];
#pragma unroll
        for (int rr = 0; rr < RW; ++rr) wf32[rr] = WF32 && min(r0 + rr, r_end - 1) < E;
        // passes of kNJ chunks per lane continue each lane's chain in chunk order
        for (int jb = 0; jb < nch; jb += kWave * kNJ) {
            uint4 wv4[RW][kNJ][2];
#pragma unroll
            for (int rr = 0; rr < RW; ++rr) {
                const int r = min(r0 + rr, r_end - 1);
#pragma unroll
                for (int j = 0; j < kNJ; ++j) {
                    const int c = min(jb + lane + kWave * j, nch - 1);
                    if (wf32[rr]) {
                        const uint4* p = reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(w) + (int64_t)r * H + 8 * c);
                        wv4[rr][j][0] = p[0];
                        wv4[rr][j][1] = p[1];
                    } else {
                        const uint16_t* src = r < E ? reinterpret_cast<const uint16_t*>(w) + (int64_t)r * H : sgw;
                        wv4[rr][j][0] = *reinterpret_cast<const uint4*>(src + 8 * c);
                        wv4[rr][j][1] = make_uint4(0, 0, 0, 0);
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < kNJ; ++j) {
                const int c = jb + lane + kWave * j;
                if (c >= nch) continue;
                float wf[RW][8];
#pragma unroll
                for (int rr = 0; rr < RW; ++rr) {
                    if (wf32[rr]) {
                        wf[rr][0] = __uint_as_float(wv4[rr][j][0].x); wf[rr][1] = __uint_as_float(wv4[rr][j][0].y);
                        wf[rr][2] = __uint_as_float(wv4[rr][j][0].z); wf[rr][3] = __uint_as_float(wv4[rr][j][0].w);
                        wf[rr][4] = __uint_as_float(wv4[rr][j][1].x); wf[rr][5] = __uint_as_float(wv4[rr][j][1].y);
                        wf[rr][6] = __uint_as_float(wv4[rr][j][1].z); wf[rr][7] = __uint_as_float(wv4[rr][j][1].w);
                    } else {
                        const uint32_t ww[4] = {wv4[rr][j][0].x, wv4[rr][j][0].y, wv4[rr][j][0].z, wv4[rr][j][0].w};
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            wf[rr][2 * i] = bf2f(ww[i] & 0xFFFFu);
                            wf[rr][2 * i + 1] = bf2f(ww[i] >> 16);
                        }
                    }
                }
                // one conversion of the token's 8 activations serves every row of the wave
#pragma unroll
                for (int t = 0; t < TT; ++t) {
                    const uint4 xv = xs4[t * nch + c];
                    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
                    float xf[8];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        xf[2 * i] = bf2f(xw[i] & 0xFFFFu);
                        xf[2 * i + 1] = bf2f(xw[i] >> 16);
                    }
#pragma unroll
                    for (int rr = 0; rr < RW; ++rr)
#pragma unroll
                        for (int i = 0; i < 8; ++i) acc[rr][t] = fmaf(xf[i], wf[rr][i], acc[rr][t]);
                }
            }
        }
#pragma unroll
        for (int rr = 0; rr < RW; ++rr) {
            const int r = r0 + rr;
            // transposed butterfly: strides 32, 16, 8, 4 halve the tokens a lane keeps
            const bool b5 = lane & 32, b4 = lane & 16, b3 = lane & 8, b2 = lane & 4;
            float v8[8], v4[4], v2[2];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float mine = b5 ? acc[rr][8 + i] : acc[rr][i], other = b5 ? acc[rr][i] : acc[rr][8 + i];
                v8[i] = mine + __shfl_xor(other, 32, kWave);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float mine = b4 ? v8[4 + i] : v8[i], other = b4 ? v8[i] : v8[4 + i];
                v4[i] = mine + __shfl_xor(other, 16, kWave);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const float mine = b3 ? v4[2 + i] : v4[i], other = b3 ? v4[i] : v4[2 + i];
                v2[i] = mine + __shfl_xor(other, 8, kWave);
            }
            float v1;
            {
                const float mine = b2 ? v2[1] : v2[0], other = b2 ? v2[0] : v2[1];
                v1 = mine + __shfl_xor(other, 4, kWave);
            }
            v1 += __shfl_xor(v1, 2, kWave);
            v1 += __shfl_xor(v1, 1, kWave);
            const int tau = lane >> 2;
            if ((lane & 3) == 0 && tau < nt && r < r_end)
                logits[(int64_t)(t0 + tau) * (E + 1) + r] = (r < E && bias) ? v1 + bias[r] : v1;
        }
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
    constexpr int kNJ = 6;                      // chunks per lane per pass (one pass: H <= 3072)
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * WPB + (threadIdx.x >> 6);
    const int rows = E + (sgw ? 1 : 0);
    const int t0 = blockIdx.y * TT;
    const int nt = min(TT, T - t0);
    const int nch = H / 8;
    if (r >= rows) return;
    const bool wf32 = WF32 && r < E;
    float acc[TT];
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[t] = 0.0f;
    // passes of kNJ chunks per lane continue each lane's chain in chunk order; every load of a
    // pass is issued before its first FMA
    for (int jb = 0; jb < nch; jb += kWave * kNJ) {
        uint4 wv[kNJ][2];
        uint4 xv[TT][kNJ];
#pragma unroll
        for (int j = 0; j < kNJ; ++j) {
            const int c = jb + lane + kWave * j;
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
#pragma unroll
            for (int j = 0; j < kNJ; ++j) {
                const int c = jb + lane + kWave * j;
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
                        acc[t] = fmaf(bf2f(xw[i] & 0xFFFFu), wf[2 * i], acc[t]);
                        acc[t] = fmaf(bf2f(xw[i] >> 16), wf[2 * i + 1], acc[t]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < TT; ++t) {
        if (t >= nt) break;   // uniform
        float s = wave_sum_xor(acc[t]);
        if (lane == 0) logits[(int64_t)(t0 + t) * (E + 1) + r] = (r < E && bias) ? s + bias[r] : s;
    }
}

// Top-k of one token's logits row `l` ([E + 1], the last entry the shared-gate logit) and its
// routing weights, by the calling wave.
template <int kPer>
__device__ __forceinline__ void topk_row(const float* __restrict__ l, int t, int E, int k, const RouteRule& rr,
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
    wave_select<kPer>(v, rr, E, k, my_id, my_v);
    const float wt = wave_weight<kPer>(v, rr, E, k, my_id, my_v);
    if (lane < k) {
        out_idx[(int64_t)t * k + lane] = my_id;
        out_w[(int64_t)t * k + lane] = wt;
    }
    if (lane == 0 && has_sg && out_sg) out_sg[t] = 1.0f / (1.0f + expf(-l[E]));
}

// One wave per token over logits [T][E + 1].
template <int kPer>
__global__ __launch_bounds__(kRouterThreads) void k_router_topk(
    const float* __restrict__ logits, int T, int E, int k, RouteRule rr, int has_sg,
    int32_t* __restrict__ out_idx, float* __restrict__ out_w, float* __restrict__ out_sg) {
    const int t = blockIdx.x * (kRouterThreads / kWave) + (threadIdx.x >> 6);
    if (t >= T) return;
    topk_row<kPer>(logits + (int64_t)t * (E + 1), t, E, k, rr, has_sg, out_idx, out_w, out_sg);
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

hipError_t topk_launch(const brx_layer_desc& d, int T, int has_sg, const float* logits, const float* bias,
                       int32_t* out_idx, float* out_w, float* out_sg, hipStream_t s) {
    const int E = d.n_experts;
    const RouteRule rr = route_rule(d, bias);
    dim3 grid((T + 3) / 4), block(kRouterThreads);
#define BRX_TOPK(KP) hipLaunchKernelGGL(k_router_topk<KP>, grid, block, 0, s, logits, T, E, d.top_k, \
                                        rr, has_sg, out_idx, out_w, out_sg)
    if (E <= 64) BRX_TOPK(1);
    else if (E <= 128) BRX_TOPK(2);
    else if (E <= 256) BRX_TOPK(4);
    else BRX_TOPK(8);
#undef BRX_TOPK
    return hipGetLastError();
}

}  // namespace

size_t router_workspace_bytes(const brx_layer_desc& d, int T) {
    return sizeof(float) * (size_t)T * (d.n_experts + 1);
}

hipError_t launch_router_logits(const brx_layer_desc& d, const void* x, const void* w_router,
                                const float* bias, const void* sgw, int T, float* logits,
                                hipStream_t s) {
    // sigmoid rules keep the logits raw: their bias enters the selection only
    if (d.route_mode >= BRX_ROUTE_SIGMOID_TOPK) bias = nullptr;
    return d.router_dtype == BRX_DT_F32 ? logits_launch<true>(d, x, w_router, bias, sgw, T, logits, s)
                                        : logits_launch<false>(d, x, w_router, bias, sgw, T, logits, s);
}

hipError_t launch_router(const brx_layer_desc& d, const void* x, const void* w_router,
                         const float* bias, const void* sgw, int T, int32_t* out_idx,
                         float* out_w, float* out_sg, float* ws_logits, hipStream_t s) {
    if (T <= 0) return hipSuccess;
    const bool f32 = d.router_dtype == BRX_DT_F32;
    // the tiled kernel stages 16 token rows of x in LDS, 32 * H bytes: within a block's 160 KB up
    // to H = 5120. Wider layers route every token tile with the small-T kernel (the same per-lane
    // chains and butterfly, so the same bits).
    if (T <= kSmallT || (size_t)32 * d.hidden > kMaxBlockLds) {
        hipError_t e = launch_router_logits(d, x, w_router, bias, sgw, T, ws_logits, s);
        if (e != hipSuccess) return e;
        return topk_launch(d, T, sgw ? 1 : 0, ws_logits, bias, out_idx, out_w, out_sg, s);
    }
    // many tokens: logits by token tiles, then the same top-k kernel
    // rows per block: 32 (each weight row read once per 16-token tile, by one wave), fewer
    // when there are too few token tiles for one round of blocks over the 256 CUs (a wave then
    // takes fewer rows; every block stages its token tile, so a second round would stage it
    // again for no more work in flight). Blocks per CU: as many staged tiles as fit in a CU's
    // 160 KB (two at H 2048, one at H 2880)
    constexpr int TT = 16;
    const int rows = d.n_experts + (sgw ? 1 : 0);
    const int tiles = (T + TT - 1) / TT;
    const size_t lds = sizeof(uint16_t) * (size_t)TT * d.hidden;
    const int per_cu = (int)(kMaxBlockLds / lds) < 2 ? 1 : 2;
    int RPB = 32;
    while (RPB > 4 && tiles * ((rows + RPB - 1) / RPB) < 256 * per_cu) RPB /= 2;
    dim3 grid(tiles, (rows + RPB - 1) / RPB);
    const float* lbias = d.route_mode >= BRX_ROUTE_SIGMOID_TOPK ? nullptr : bias;
    if (f32)
        hipLaunchKernelGGL((k_router_tiled<true, TT>), grid, dim3(kRouterThreads), lds, s, (const uint16_t*)x,
                           w_router, lbias, (const uint16_t*)sgw, T, d.hidden, d.n_experts, RPB, ws_logits);
    else
        hipLaunchKernelGGL((k_router_tiled<false, TT>), grid, dim3(kRouterThreads), lds, s, (const uint16_t*)x,
                           w_router, lbias, (const uint16_t*)sgw, T, d.hidden, d.n_experts, RPB, ws_logits);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return topk_launch(d, T, sgw ? 1 : 0, ws_logits, bias, out_idx, out_w, out_sg, s);
}

}  // namespace brx
