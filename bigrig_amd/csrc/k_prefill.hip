// Prefill chunks: (token, expert) pairs bucketed per expert, then grouped GEMMs on MFMA.
//
// Replaces the reference's expert-sorted prefill: the stable argsort of pairs by expert
// (bigrig_engine/stream.py:1526-1530, 1244-1250), the sorted `mx.gather_qmm` per projection
// (stream.py:1320-1336, 1605-1631), the SwiGLU between them and the inverse permutation that
// restores (token, k) order (stream.py:1558-1561, _scatter_unsort 1829-1831), followed by the
// caller's router-weighted combine (stream.py:1523-1525).
//
//   k_bucket     one block per expert: histogram of all pairs, the expert's run offset and
//                M-tile offset, and the stable (pair-order) compaction of its pairs.
//   k_pf_gateup  tile = (M tile of one expert's pairs, 64 intermediate features): A rows are
//                the pairs' token activations gathered from x, B rows are the gate and up
//                weights of those features dequantized to bf16 in LDS, one 64-wide K step
//                (= one affine group) at a time; v_mfma_f32_16x16x32_bf16 accumulates fp32;
//                the epilogue applies act() and stores h (bf16) in bucketed order.
//   k_pf_down    tile = (M tile, 128 output columns): A = h rows, B = down weights; the
//                epilogue stores each pair's bf16 row at its (token, k) position.
//   k_combine    out[t] = sum_j w[t,j] * y[t,j] (+ shared_gate[t] * y_shared[t]), k-ordered.
// Every output element is one MFMA accumulation over K in a fixed K order, so a row's value
// does not depend on which other pairs share its tile.
#include "brx_internal.h"

namespace brx {
namespace {

constexpr int kBM = 128;          // pairs per M tile
constexpr int kBK = 64;           // K step
constexpr int kLdsRow = 72;       // bf16 per LDS row (64 + 8 pad)
constexpr int kThreads = 256;

// ------------------------------------------------------------------ bucketing
__global__ __launch_bounds__(1024) void k_bucket(const int32_t* __restrict__ pexp, int P, int E,
                                                  int E_ext, int T_sh, int BM,
                                                  int32_t* __restrict__ order,
                                                  int32_t* __restrict__ offsets,
                                                  int32_t* __restrict__ tile_start) {
    // E_ext = E + 1 when a shared expert exists (id E); T_sh shared pairs follow the P routed
    extern __shared__ int32_t hist[];     // [E_ext]
    __shared__ int32_t wsum[16];
    __shared__ int32_t base_s[2];
    const int P_ext = P + T_sh;
    const int emax = E_ext - 1;
    const int e = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, nw = blockDim.x >> 6;
    for (int i = tid; i < E_ext; i += blockDim.x) hist[i] = 0;
    __syncthreads();
    for (int p = tid; p < P_ext; p += blockDim.x) {
        int ex = p < P ? min(max(pexp[p], 0), emax) : E;
        atomicAdd(&hist[ex], 1);
    }
    __syncthreads();
    if (wv == 0) {
        // offsets of expert e: sum of the counts (and of the M tiles) of the experts before it
        int off = 0, toff = 0;
        for (int j = lane; j < e; j += 64) { off += hist[j]; toff += (hist[j] + BM - 1) / BM; }
        for (int s = 32; s >= 1; s >>= 1) { off += __shfl_xor(off, s, 64); toff += __shfl_xor(toff, s, 64); }
        if (lane == 0) {
            base_s[0] = off;
            offsets[e] = off;
            tile_start[e] = toff;
            if (e == E_ext - 1) {
                offsets[E_ext] = P_ext;
                tile_start[E_ext] = toff + (hist[e] + BM - 1) / BM;
            }
        }
    }
    __syncthreads();
    int run = base_s[0];
    for (int p0 = 0; p0 < P_ext; p0 += blockDim.x) {
        int p = p0 + tid;
        bool m = false;
        if (p < P_ext) {
            int ex = p < P ? min(max(pexp[p], 0), emax) : E;
            m = ex == e;
        }
        uint64_t b = __ballot(m);
        if (lane == 0) wsum[wv] = __popcll(b);
        __syncthreads();
        int before = 0, total = 0;
        for (int w = 0; w < nw; ++w) { if (w < wv) before += wsum[w]; total += wsum[w]; }
        if (m) order[run + before + __popcll(b & ((1ull << lane) - 1ull))] = p;
        run += total;
        __syncthreads();
    }
}

__device__ __forceinline__ const uint8_t* pf_expert_base(const FwdArgs& a, int e) {
    if (e >= a.E) return a.shared;
    int s = a.g2s[e];
    s = min(max(s, 0), a.capacity - 1);
    return a.slots + (int64_t)s * a.slot_stride;
}

// M tile -> (expert, first bucketed row, valid rows); false if past the last tile.
__device__ __forceinline__ bool find_tile(const int32_t* tile_start, const int32_t* offsets,
                                          int E_ext, int mt, int& e, int& m0, int& rows) {
    if (mt >= tile_start[E_ext]) return false;
    int lo = 0, hi = E_ext - 1;          // largest e with tile_start[e] <= mt
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (tile_start[mid] <= mt) lo = mid; else hi = mid - 1;
    }
    e = lo;
    m0 = offsets[e] + (mt - tile_start[e]) * kBM;
    rows = min(kBM, offsets[e + 1] - m0);
    return rows > 0;
}

// Dequantize 32 weights (one 16-byte chunk) of row `row`, K offset k, into 16 bf16x2 words.
template <int MODE>
__device__ __forceinline__ void dequant32(const uint8_t* base, const Proj& P, int row, int k,
                                          int scale_f16, uint32_t out[16]) {
    const int n_in = P.n_in;
    uint4 v = *reinterpret_cast<const uint4*>(base + P.w + (int64_t)row * (n_in / 2) + k / 2);
    uint32_t wd[4] = {v.x, v.y, v.z, v.w};
    if constexpr (MODE == BRX_QUANT_AFFINE) {
        const int G = n_in / 64;
        float s = load_scale(base + P.s, (int64_t)row * G + k / 64, scale_f16);
        float b = load_scale(base + P.b, (int64_t)row * G + k / 64, scale_f16);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float v0 = fmaf(s, (float)((wd[q] >> (8 * i)) & 0xFu), b);
                float v1 = fmaf(s, (float)((wd[q] >> (8 * i + 4)) & 0xFu), b);
                out[4 * q + i] = f2bf(v0) | (f2bf(v1) << 16);
            }
        }
    } else {
        const int G = n_in / 32;
        float s = e8m0_f32(base[P.s + (int64_t)row * G + k / 32]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float v0 = e2m1_f32((wd[q] >> (8 * i)) & 0xFu) * s;
                float v1 = e2m1_f32((wd[q] >> (8 * i + 4)) & 0xFu) * s;
                out[4 * q + i] = f2bf(v0) | (f2bf(v1) << 16);
            }
        }
    }
}

__device__ __forceinline__ int pair_token(const FwdArgs& a, int pair) {
    return pair < a.P ? pair_tok(a, pair) : pair - a.P;
}

// ------------------------------------------------------------------ gate/up
template <int MODE>
__global__ __launch_bounds__(kThreads) void k_pf_gateup(FwdArgs a, const int32_t* __restrict__ order,
                                                        const int32_t* __restrict__ offsets,
                                                        const int32_t* __restrict__ tile_start,
                                                        uint16_t* __restrict__ hbuf, int hstride) {
    __shared__ __attribute__((aligned(16))) uint16_t As[kBM * kLdsRow];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[128 * kLdsRow];
    __shared__ int32_t tok_s[kBM];
    const int E_ext = a.E + (a.shared ? 1 : 0);
    int e, m0, rows;
    if (!find_tile(tile_start, offsets, E_ext, blockIdx.x, e, m0, rows)) return;
    const bool sh = e >= a.E;
    const int inter = sh ? a.I_sh : a.I;
    const int f0 = blockIdx.y * 64;
    if (f0 >= inter) return;
    const Layout& L = sh ? a.lay_sh : a.lay;
    const uint8_t* base = pf_expert_base(a, e);
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wm = wv & 1, wn = wv >> 1;
    const int H = a.H;

    if (tid < kBM) tok_s[tid] = tid < rows ? pair_token(a, order[m0 + tid]) : -1;
    __syncthreads();

    f32x4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    const int lrow = tid >> 1, lhalf = tid & 1;
    for (int k0 = 0; k0 < H; k0 += kBK) {
        // A: 128 rows x 64 bf16 of gathered activations
        {
            int t = tok_s[lrow];
            uint4 v[4];
            if (t >= 0) {
                const uint4* src = reinterpret_cast<const uint4*>(a.x + (int64_t)t * H + k0 + lhalf * 32);
#pragma unroll
                for (int q = 0; q < 4; ++q) v[q] = src[q];
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) v[q] = make_uint4(0, 0, 0, 0);
            }
            uint4* dst = reinterpret_cast<uint4*>(As + lrow * kLdsRow + lhalf * 32);
#pragma unroll
            for (int q = 0; q < 4; ++q) dst[q] = v[q];
        }
        // B: rows 0-63 gate features f0.., rows 64-127 up features f0..
        {
            int mat = lrow >> 6;
            int row = f0 + (lrow & 63);
            uint32_t wq[16];
            dequant32<MODE>(base, L.p[mat], row, k0 + lhalf * 32, a.scale_f16, wq);
            uint4* dst = reinterpret_cast<uint4*>(Bs + lrow * kLdsRow + lhalf * 32);
#pragma unroll
            for (int q = 0; q < 4; ++q) dst[q] = make_uint4(wq[4 * q], wq[4 * q + 1], wq[4 * q + 2], wq[4 * q + 3]);
        }
        __syncthreads();
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
            const int ko = kc * 32 + (lane >> 4) * 8;
            bf16x8_t af[4], bfr[4];
#pragma unroll
            for (int mi = 0; mi < 4; ++mi)
                af[mi] = *reinterpret_cast<const bf16x8_t*>(As + (wm * 64 + mi * 16 + (lane & 15)) * kLdsRow + ko);
#pragma unroll
            for (int nj = 0; nj < 4; ++nj) {
                int brow = (nj >> 1) * 64 + wn * 32 + (nj & 1) * 16 + (lane & 15);
                bfr[nj] = *reinterpret_cast<const bf16x8_t*>(Bs + brow * kLdsRow + ko);
            }
#pragma unroll
            for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                for (int nj = 0; nj < 4; ++nj)
                    acc[mi][nj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mi], bfr[nj], acc[mi][nj], 0, 0, 0);
        }
        __syncthreads();
    }

    // epilogue: frags nj=0,1 are gate, nj=2,3 the up rows of the same features
#pragma unroll
    for (int nj = 0; nj < 2; ++nj) {
        const int f = f0 + wn * 32 + nj * 16 + (lane & 15);
        float bg = 0.f, bu = 0.f;
        if (L.p[0].bias >= 0) {
            bg = bf2f(reinterpret_cast<const uint16_t*>(base + L.p[0].bias)[f]);
            bu = bf2f(reinterpret_cast<const uint16_t*>(base + L.p[1].bias)[f]);
        }
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                int r = wm * 64 + mi * 16 + (lane >> 4) * 4 + i;
                if (r < rows) {
                    float h = act_apply(a.act, acc[mi][nj][i] + bg, acc[mi][nj + 2][i] + bu, a.alpha, a.limit);
                    hbuf[(int64_t)(m0 + r) * hstride + f] = (uint16_t)f2bf(h);
                }
            }
        }
    }
}

// ------------------------------------------------------------------ down
template <int MODE>
__global__ __launch_bounds__(kThreads) void k_pf_down(FwdArgs a, const int32_t* __restrict__ order,
                                                      const int32_t* __restrict__ offsets,
                                                      const int32_t* __restrict__ tile_start,
                                                      const uint16_t* __restrict__ hbuf, int hstride,
                                                      uint16_t* __restrict__ y_routed,
                                                      uint16_t* __restrict__ y_shared) {
    __shared__ __attribute__((aligned(16))) uint16_t As[kBM * kLdsRow];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[128 * kLdsRow];
    const int E_ext = a.E + (a.shared ? 1 : 0);
    int e, m0, rows;
    if (!find_tile(tile_start, offsets, E_ext, blockIdx.x, e, m0, rows)) return;
    const bool sh = e >= a.E;
    const int inter = sh ? a.I_sh : a.I;
    const Layout& L = sh ? a.lay_sh : a.lay;
    const uint8_t* base = pf_expert_base(a, e);
    const int n0 = blockIdx.y * 128;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int wm = wv & 1, wn = wv >> 1;
    const int P = a.P, H = a.H;

    f32x4_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    const int lrow = tid >> 1, lhalf = tid & 1;
    for (int k0 = 0; k0 < inter; k0 += kBK) {
        {
            uint4 v[4];
            if (lrow < rows) {
                const uint4* src = reinterpret_cast<const uint4*>(hbuf + (int64_t)(m0 + lrow) * hstride + k0 + lhalf * 32);
#pragma unroll
                for (int q = 0; q < 4; ++q) v[q] = src[q];
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) v[q] = make_uint4(0, 0, 0, 0);
            }
            uint4* dst = reinterpret_cast<uint4*>(As + lrow * kLdsRow + lhalf * 32);
#pragma unroll
            for (int q = 0; q < 4; ++q) dst[q] = v[q];
        }
        {
            uint32_t wq[16];
            if (n0 + lrow < H) {
                dequant32<MODE>(base, L.p[2], n0 + lrow, k0 + lhalf * 32, a.scale_f16, wq);
            } else {
#pragma unroll
                for (int q = 0; q < 16; ++q) wq[q] = 0u;
            }
            uint4* dst = reinterpret_cast<uint4*>(Bs + lrow * kLdsRow + lhalf * 32);
#pragma unroll
            for (int q = 0; q < 4; ++q) dst[q] = make_uint4(wq[4 * q], wq[4 * q + 1], wq[4 * q + 2], wq[4 * q + 3]);
        }
        __syncthreads();
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
            const int ko = kc * 32 + (lane >> 4) * 8;
            bf16x8_t af[4], bfr[4];
#pragma unroll
            for (int mi = 0; mi < 4; ++mi)
                af[mi] = *reinterpret_cast<const bf16x8_t*>(As + (wm * 64 + mi * 16 + (lane & 15)) * kLdsRow + ko);
#pragma unroll
            for (int nj = 0; nj < 4; ++nj)
                bfr[nj] = *reinterpret_cast<const bf16x8_t*>(Bs + (wn * 64 + nj * 16 + (lane & 15)) * kLdsRow + ko);
#pragma unroll
            for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                for (int nj = 0; nj < 4; ++nj)
                    acc[mi][nj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mi], bfr[nj], acc[mi][nj], 0, 0, 0);
        }
        __syncthreads();
    }

#pragma unroll
    for (int nj = 0; nj < 4; ++nj) {
        const int n = n0 + wn * 64 + nj * 16 + (lane & 15);
        if (n >= H) continue;
        float bd = 0.f;
        if (L.p[2].bias >= 0) bd = bf2f(reinterpret_cast<const uint16_t*>(base + L.p[2].bias)[n]);
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                int r = wm * 64 + mi * 16 + (lane >> 4) * 4 + i;
                if (r < rows) {
                    int pair = order[m0 + r];
                    uint16_t yb = (uint16_t)f2bf(acc[mi][nj][i] + bd);
                    if (pair < P) y_routed[(int64_t)pair_row(a, pair) * H + n] = yb;
                    else y_shared[(int64_t)(pair - P) * H + n] = yb;
                }
            }
        }
    }
}

// ------------------------------------------------------------------ combine
__global__ __launch_bounds__(kThreads) void k_combine(const uint16_t* __restrict__ y_routed,
                                                      const uint16_t* __restrict__ y_shared,
                                                      const float* __restrict__ w,
                                                      const float* __restrict__ sg, int T, int k,
                                                      int H, uint16_t* __restrict__ out) {
    const int t = blockIdx.y;
    const int n = (blockIdx.x * kThreads + threadIdx.x) * 2;
    if (n >= H) return;
    float a0 = 0.f, a1 = 0.f;
    for (int j = 0; j < k; ++j) {
        float wj = w[t * k + j];
        uint32_t yv = *reinterpret_cast<const uint32_t*>(y_routed + ((int64_t)t * k + j) * H + n);
        a0 = fmaf(wj, bf2f(yv & 0xFFFFu), a0);
        a1 = fmaf(wj, bf2f(yv >> 16), a1);
    }
    if (y_shared && sg) {
        uint32_t yv = *reinterpret_cast<const uint32_t*>(y_shared + (int64_t)t * H + n);
        a0 = fmaf(sg[t], bf2f(yv & 0xFFFFu), a0);
        a1 = fmaf(sg[t], bf2f(yv >> 16), a1);
    }
    *reinterpret_cast<uint32_t*>(out + (int64_t)t * H + n) = f2bf(a0) | (f2bf(a1) << 16);
}

struct PfWs {
    int32_t* order;
    int32_t* offsets;
    int32_t* tile_start;
    uint16_t* hbuf;
    uint16_t* y_routed;
    uint16_t* y_shared;
    size_t bytes;
};

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

PfWs carve(const FwdArgs& a, void* ws) {
    const int P = a.P;
    const int T_sh = a.auto_shared ? a.T : 0;
    const int P_ext = P + T_sh;
    const int E_ext = a.E + (a.shared ? 1 : 0);
    const int Imax = a.I > a.I_sh ? a.I : a.I_sh;
    PfWs w{};
    size_t off = 0;
    char* b = reinterpret_cast<char*>(ws);
    w.order = reinterpret_cast<int32_t*>(b + off); off = align256(off + sizeof(int32_t) * P_ext);
    w.offsets = reinterpret_cast<int32_t*>(b + off); off = align256(off + sizeof(int32_t) * (E_ext + 1));
    w.tile_start = reinterpret_cast<int32_t*>(b + off); off = align256(off + sizeof(int32_t) * (E_ext + 1));
    w.hbuf = reinterpret_cast<uint16_t*>(b + off); off = align256(off + 2ull * P_ext * Imax);
    w.y_routed = reinterpret_cast<uint16_t*>(b + off); off = align256(off + 2ull * P * a.H);
    w.y_shared = reinterpret_cast<uint16_t*>(b + off); off = align256(off + 2ull * T_sh * a.H);
    w.bytes = off;
    return w;
}

}  // namespace

size_t prefill_workspace_bytes(const FwdArgs& a) { return carve(a, nullptr).bytes; }

hipError_t launch_sort_pairs(const int32_t* pexp, int P, int E, int E_ext, int T_sh, int BM,
                             int32_t* order, int32_t* offsets, int32_t* tile_start, hipStream_t s) {
    hipLaunchKernelGGL(k_bucket, dim3(E_ext), dim3(1024), sizeof(int32_t) * E_ext, s, pexp, P, E,
                       E_ext, T_sh, BM, order, offsets, tile_start);
    return hipGetLastError();
}

hipError_t launch_combine(const uint16_t* y_routed, const uint16_t* y_shared, const float* w,
                          const float* sg, int T, int k, int H, uint16_t* out, hipStream_t s) {
    hipLaunchKernelGGL(k_combine, dim3((H / 2 + kThreads - 1) / kThreads, T), dim3(kThreads), 0, s,
                       y_routed, y_shared, w, sg, T, k, H, out);
    return hipGetLastError();
}

hipError_t launch_prefill(const FwdArgs& a, void* ws, size_t ws_bytes, int phases, hipStream_t s) {
    PfWs w = carve(a, ws);
    if (w.bytes > ws_bytes) return hipErrorInvalidValue;
    const int P = a.P;
    const int T_sh = a.auto_shared ? a.T : 0;
    const int P_ext = P + T_sh;
    const int E_ext = a.E + (a.shared ? 1 : 0);
    const int Imax = a.I > a.I_sh ? a.I : a.I_sh;
    const int mt_max = (P_ext + kBM - 1) / kBM + E_ext;
    uint16_t* y_routed = a.yun ? a.yun : w.y_routed;
    hipError_t err = hipSuccess;
    if (phases & 1) {
        err = launch_sort_pairs(a.pexp, P, a.E, E_ext, T_sh, kBM, w.order, w.offsets, w.tile_start, s);
        if (err != hipSuccess) return err;
        if (a.quant_mode == BRX_QUANT_AFFINE)
            hipLaunchKernelGGL(k_pf_gateup<BRX_QUANT_AFFINE>, dim3(mt_max, Imax / 64), dim3(kThreads), 0, s,
                               a, w.order, w.offsets, w.tile_start, w.hbuf, Imax);
        else
            hipLaunchKernelGGL(k_pf_gateup<BRX_QUANT_MXFP4>, dim3(mt_max, Imax / 64), dim3(kThreads), 0, s,
                               a, w.order, w.offsets, w.tile_start, w.hbuf, Imax);
        err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    if (phases & 2) {
        if (a.quant_mode == BRX_QUANT_AFFINE)
            hipLaunchKernelGGL(k_pf_down<BRX_QUANT_AFFINE>, dim3(mt_max, (a.H + 127) / 128), dim3(kThreads), 0, s,
                               a, w.order, w.offsets, w.tile_start, w.hbuf, Imax, y_routed, w.y_shared);
        else
            hipLaunchKernelGGL(k_pf_down<BRX_QUANT_MXFP4>, dim3(mt_max, (a.H + 127) / 128), dim3(kThreads), 0, s,
                               a, w.order, w.offsets, w.tile_start, w.hbuf, Imax, y_routed, w.y_shared);
        err = hipGetLastError();
        if (err != hipSuccess) return err;
        if (a.out)
            err = launch_combine(y_routed, a.auto_shared ? w.y_shared : nullptr, a.w, a.sgate, a.T, a.k,
                                 a.H, a.out, s);
    }
    return err;
}

}  // namespace brx
