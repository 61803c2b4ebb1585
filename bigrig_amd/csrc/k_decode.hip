// Decode (1-8 tokens): fused gather-GEMV over the routed experts' packed 4-bit weights.
//
// Replaces the per-row `mx.gather_qmm(x, w, scales, biases, rhs_indices=slots,
// transpose=True)` of StreamingSwitchGLU._proj (bigrig_engine/stream.py:1605-1631) for the
// three projections, the SwiGLU between them (stream.py:1164-1166) and the caller's
// router-weighted combine (stream.py:1523-1525).
//
// Two kernels per layer:
//   k_dec_gateup  grid (row block, unique expert): gate and up rows of one expert for every
//                 token routed to it, act() in the epilogue, h -> bf16 workspace.
//   k_dec_down    grid (row block of H): down rows of every routed expert, the row's bf16
//                 result, and the k-ordered combine out[t] = sum_j w[t,j] * y[t,j].
// Weights stream from HBM once per step as 16-byte loads: each thread owns CPS consecutive
// 16-byte chunks (32 nibbles each) of one row, so a wave covers whole rows contiguously.
// Dequant is folded into the dot product: for a 32-element chunk with scale s and bias b,
//   sum_i (s q_i + b) x_i = s * sum_i (128 + q_i) x_i + (b - 128 s) * sum_i x_i,
// where (128 + q_i) is formed as an exact bf16 by bit operations and the products are
// accumulated in fp32 by v_dot2_f32_bf16. Row partials are combined in a fixed order, so a
// row's result does not depend on which other rows or tokens share the launch.
#include "brx_internal.h"

namespace brx {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxTok = 8;
constexpr int kMaxU = 65;     // 64 routed pairs + the shared expert

struct Plan {
    int n;                    // number of unique experts (shared last)
    int e[kMaxU];
    int ntok[kMaxU];
    int pair[kMaxU][kMaxTok]; // pair index: t*k + j, or P + t for the shared expert
    int tok[kMaxU][kMaxTok];
};

// Experts of the step in order of first appearance over the pairs, then the shared expert.
// Run by wave 0.
__device__ void build_plan(const FwdArgs& a, Plan& pl) {
    const int lane = threadIdx.x & 63;
    const int P = a.P;
    const int emax = a.shared ? a.E : a.E - 1;   // id E names the shared expert
    int e = -1;
    if (lane < P) e = min(max(a.pexp[lane], 0), emax);
    // An entry is a run of up to kMaxTok pairs of one expert: a pair leads an entry when the
    // number of earlier pairs routed to the same expert is a multiple of kMaxTok.
    int occ = 0;
    for (int q = 0; q < P; ++q) {
        int eq = __shfl(e, q, kWave);
        if (q < lane && eq == e) ++occ;
    }
    const bool lead = lane < P && (occ % kMaxTok) == 0;
    uint64_t mask = __ballot(lead);
    int rank = __popcll(mask & ((1ull << lane) - 1ull));
    int cnt = 0;
    for (int q = 0; q < P; ++q) {        // uniform loop: every lane takes part in the shuffle
        int eq = __shfl(e, q, kWave);
        if (lead && q >= lane && eq == e && cnt < kMaxTok) {
            pl.pair[rank][cnt] = q;
            pl.tok[rank][cnt] = pair_tok(a, q);
            ++cnt;
        }
    }
    if (lead) {
        pl.e[rank] = e;
        pl.ntok[rank] = cnt;
    }
    int nr = __popcll(mask);
    if (lane == 0) {
        if (a.auto_shared) {
            pl.e[nr] = a.E;
            pl.ntok[nr] = a.T;
            for (int t = 0; t < a.T; ++t) { pl.pair[nr][t] = P + t; pl.tok[nr][t] = t; }
            pl.n = nr + 1;
        } else {
            pl.n = nr;
        }
    }
}

__device__ __forceinline__ const uint8_t* expert_base(const FwdArgs& a, int e) {
    if (e >= a.E) return a.shared;
    int s = a.g2s[e];
    s = min(max(s, 0), a.capacity - 1);
    return a.slots + (int64_t)s * a.slot_stride;
}

// Partial of one row segment: CPS chunks of 32 elements against `nt` activation vectors.
// xp(i, c) -> pointer to 16 words (pair-permuted) of vector i at chunk c; xs(i, c) -> chunk sum.
template <int MODE, int CPS, typename XP, typename XS>
__device__ __forceinline__ void seg_partials(const uint8_t* wrow, const uint8_t* srow,
                                             const uint8_t* brow, int c0, int gs, int scale_f16,
                                             int nt, XP xp, XS xs, float* out) {
    uint4 wv[CPS];
#pragma unroll
    for (int j = 0; j < CPS; ++j) wv[j] = reinterpret_cast<const uint4*>(wrow)[c0 + j];
    float sc[CPS], bi[CPS];
#pragma unroll
    for (int j = 0; j < CPS; ++j) {
        int g = ((c0 + j) * 32) / gs;
        if constexpr (MODE == BRX_QUANT_AFFINE) {
            sc[j] = load_scale(srow, g, scale_f16);
            bi[j] = load_scale(brow, g, scale_f16) - 128.0f * sc[j];
        } else {
            sc[j] = e8m0_f32(srow[g]);
            bi[j] = 0.0f;
        }
    }
    for (int i = 0; i < nt; ++i) {
        float p = 0.0f;
#pragma unroll
        for (int j = 0; j < CPS; ++j) {
            const uint32_t* x16 = xp(i, c0 + j);
            uint32_t wd[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
            float acc = 0.0f;
            if constexpr (MODE == BRX_QUANT_AFFINE) {
#pragma unroll
                for (int q = 0; q < 4; ++q) acc = dot8_q4(wd[q], x16 + 4 * q, acc);
                p = fmaf(sc[j], acc, fmaf(bi[j], xs(i, c0 + j), p));
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        uint32_t xw = x16[4 * q + b];
                        acc = fmaf(e2m1_f32((wd[q] >> (4 * b)) & 0xFu), bf2f(xw & 0xFFFFu), acc);
                        acc = fmaf(e2m1_f32((wd[q] >> (4 * b + 16)) & 0xFu), bf2f(xw >> 16), acc);
                    }
                }
                p = fmaf(sc[j], acc, p);
            }
        }
        out[i] = p;
    }
}

// ------------------------------------------------------------------ gate/up
template <int MODE, int CPS>
__global__ __launch_bounds__(kThreads) void k_dec_gateup(FwdArgs a, uint16_t* __restrict__ hbuf,
                                                         int RB, int hstride) {
    __shared__ Plan pl;
    extern __shared__ uint32_t dsm[];
    const int tid = threadIdx.x;
    if (tid < kWave) build_plan(a, pl);
    __syncthreads();
    const int u = blockIdx.y;
    if (u >= pl.n) return;
    const int e = pl.e[u];
    const bool sh = e >= a.E;
    const int inter = sh ? a.I_sh : a.I;
    const int r0 = blockIdx.x * RB;
    if (r0 >= inter) return;
    const Layout& L = sh ? a.lay_sh : a.lay;
    const uint8_t* base = expert_base(a, e);
    const int nt = pl.ntok[u];
    const int H = a.H, CPR = H / 32, S = CPR / CPS;

    uint32_t* xperm = dsm;                                   // [nt][H/2] words
    float* xsum = reinterpret_cast<float*>(xperm + nt * (H / 2));  // [nt][CPR]
    float* part = xsum + nt * CPR;                           // [nt][2][RB][S]

    // stage the tokens' activations, pair-permuted, with chunk sums
    for (int it = tid; it < nt * CPR; it += kThreads) {
        int i = it / CPR, c = it - i * CPR;
        const uint4* src = reinterpret_cast<const uint4*>(a.x + (int64_t)pl.tok[u][i] * H + c * 32);
        uint32_t* dst = xperm + i * (H / 2) + c * 16;
        float s = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint4 v = src[q];
            uint32_t in[4] = {v.x, v.y, v.z, v.w}, o[4];
            perm8(in, o);
#pragma unroll
            for (int z = 0; z < 4; ++z) {
                dst[4 * q + z] = o[z];
                s += bf2f(in[z] & 0xFFFFu) + bf2f(in[z] >> 16);
            }
        }
        xsum[i * CPR + c] = s;
    }
    __syncthreads();

    auto xp = [&](int i, int c) { return xperm + i * (H / 2) + c * 16; };
    auto xs = [&](int i, int c) { return xsum[i * CPR + c]; };
    const int W = 2 * RB * S;
    for (int wi = tid; wi < W; wi += kThreads) {
        int mat = wi / (RB * S);
        int rem = wi - mat * RB * S;
        int rr = rem / S, seg = rem - rr * S;
        int row = r0 + rr;
        const Proj& P = L.p[mat];
        const uint8_t* wrow = base + P.w + (int64_t)row * (H / 2);
        int gcount = (MODE == BRX_QUANT_AFFINE) ? H / 64 : H / 32;
        int gs = (MODE == BRX_QUANT_AFFINE) ? 64 : 32;
        const uint8_t* srow = base + P.s + (int64_t)row * gcount * (MODE == BRX_QUANT_AFFINE ? 2 : 1);
        const uint8_t* brow = (MODE == BRX_QUANT_AFFINE) ? base + P.b + (int64_t)row * gcount * 2 : nullptr;
        float pr[kMaxTok];
        seg_partials<MODE, CPS>(wrow, srow, brow, seg * CPS, gs, a.scale_f16, nt, xp, xs, pr);
        for (int i = 0; i < nt; ++i) part[((i * 2 + mat) * RB + rr) * S + seg] = pr[i];
    }
    __syncthreads();

    // reduce segments in order, activation, h -> bf16 (pair-permuted in blocks of 8)
    uint16_t* hs = reinterpret_cast<uint16_t*>(part + nt * 2 * RB * S);  // [nt][RB]
    for (int it = tid; it < nt * RB; it += kThreads) {
        int i = it / RB, rr = it - i * RB;
        const float* pg = part + ((i * 2 + 0) * RB + rr) * S;
        const float* pu = part + ((i * 2 + 1) * RB + rr) * S;
        float g = 0.0f, v = 0.0f;
        for (int s2 = 0; s2 < S; ++s2) { g += pg[s2]; v += pu[s2]; }
        int row = r0 + rr;
        if (L.p[0].bias >= 0) {
            g += bf2f(reinterpret_cast<const uint16_t*>(base + L.p[0].bias)[row]);
            v += bf2f(reinterpret_cast<const uint16_t*>(base + L.p[1].bias)[row]);
        }
        hs[i * RB + rr] = (uint16_t)f2bf(act_apply(a.act, g, v, a.alpha, a.limit));
    }
    __syncthreads();
    for (int it = tid; it < nt * (RB / 8); it += kThreads) {
        int i = it / (RB / 8), m = it - i * (RB / 8);
        const uint16_t* hr = hs + i * RB + 8 * m;
        uint32_t in[4], o[4];
#pragma unroll
        for (int z = 0; z < 4; ++z) in[z] = (uint32_t)hr[2 * z] | ((uint32_t)hr[2 * z + 1] << 16);
        perm8(in, o);
        uint4* dst = reinterpret_cast<uint4*>(hbuf + (int64_t)pl.pair[u][i] * hstride + r0 + 8 * m);
        *dst = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

// ------------------------------------------------------------------ down + combine
template <int MODE, int CPS>
__global__ __launch_bounds__(kThreads) void k_dec_down(FwdArgs a, const uint16_t* __restrict__ hbuf,
                                                       int RBD, int hstride) {
    __shared__ Plan pl;
    extern __shared__ float fsm[];
    const int tid = threadIdx.x;
    if (tid < kWave) build_plan(a, pl);
    __syncthreads();
    const int P = a.P;
    const int PT = P + (a.auto_shared ? a.T : 0);
    const int I = a.I, CPR = I / 32, S = CPR / CPS;
    const int n0 = blockIdx.x * RBD;
    const int H = a.H;

    float* hsum = fsm;                          // [PT][CPR]
    float* part = hsum + PT * CPR;              // [PT][RBD][S]
    float* ys = part + PT * RBD * S;            // [PT][RBD]

    // chunk sums of every pair's h (pair-permuted order does not change a chunk's sum)
    for (int it = tid; it < PT * CPR; it += kThreads) {
        int p = it / CPR, c = it - p * CPR;
        const uint4* src = reinterpret_cast<const uint4*>(hbuf + (int64_t)p * hstride + c * 32);
        float s = 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint4 v = src[q];
            uint32_t in[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int z = 0; z < 4; ++z) s += bf2f(in[z] & 0xFFFFu) + bf2f(in[z] >> 16);
        }
        hsum[it] = s;
    }
    __syncthreads();

    const int gs = (MODE == BRX_QUANT_AFFINE) ? 64 : 32;
    const int gcount = I / gs;
    const int W = pl.n * RBD * S;
    for (int wi = tid; wi < W; wi += kThreads) {
        int u = wi / (RBD * S);
        int rem = wi - u * RBD * S;
        int rr = rem / S, seg = rem - rr * S;
        int n = n0 + rr;
        int e = pl.e[u];
        const Layout& L = e >= a.E ? a.lay_sh : a.lay;
        const uint8_t* base = expert_base(a, e);
        const Proj& Pd = L.p[2];
        const uint8_t* wrow = base + Pd.w + (int64_t)n * (I / 2);
        const uint8_t* srow = base + Pd.s + (int64_t)n * gcount * (MODE == BRX_QUANT_AFFINE ? 2 : 1);
        const uint8_t* brow = (MODE == BRX_QUANT_AFFINE) ? base + Pd.b + (int64_t)n * gcount * 2 : nullptr;
        const int nt = pl.ntok[u];
        auto xp = [&](int i, int c) {
            return reinterpret_cast<const uint32_t*>(hbuf + (int64_t)pl.pair[u][i] * hstride + c * 32);
        };
        auto xs = [&](int i, int c) { return hsum[pl.pair[u][i] * CPR + c]; };
        float pr[kMaxTok];
        seg_partials<MODE, CPS>(wrow, srow, brow, seg * CPS, gs, a.scale_f16, nt, xp, xs, pr);
        for (int i = 0; i < nt; ++i) part[(pl.pair[u][i] * RBD + rr) * S + seg] = pr[i];
    }
    __syncthreads();

    // each pair's row result, rounded to bf16 as the projection's output
    for (int it = tid; it < PT * RBD; it += kThreads) {
        int p = it / RBD, rr = it - p * RBD;
        const float* pp = part + (p * RBD + rr) * S;
        float y = 0.0f;
        for (int s2 = 0; s2 < S; ++s2) y += pp[s2];
        int n = n0 + rr;
        int e = p < P ? min(max(a.pexp[p], 0), a.shared ? a.E : a.E - 1) : a.E;
        const Layout& L = e >= a.E ? a.lay_sh : a.lay;
        if (L.p[2].bias >= 0)
            y += bf2f(reinterpret_cast<const uint16_t*>(expert_base(a, e) + L.p[2].bias)[n]);
        uint32_t yb = f2bf(y);
        ys[it] = bf2f(yb);
        if (a.yun && p < P) a.yun[(int64_t)pair_row(a, p) * H + n] = (uint16_t)yb;
    }
    __syncthreads();

    if (a.out) {
        for (int it = tid; it < a.T * RBD; it += kThreads) {
            int t = it / RBD, rr = it - t * RBD;
            float acc = 0.0f;
            for (int j = 0; j < a.k; ++j)
                acc = fmaf(a.w[t * a.k + j], ys[(t * a.k + j) * RBD + rr], acc);
            if (a.auto_shared && a.sgate) acc = fmaf(a.sgate[t], ys[(P + t) * RBD + rr], acc);
            a.out[(int64_t)t * H + n0 + rr] = (uint16_t)f2bf(acc);
        }
    }
}

int pick_cps(int cpr) {
    for (int c : {4, 3, 2}) if (cpr % c == 0) return c;
    return 1;
}

template <int MODE>
hipError_t launch_mode(const FwdArgs& a, uint16_t* hbuf, int phases, hipStream_t s) {
    const int P = a.P;
    const int PT = P + (a.auto_shared ? a.T : 0);
    const int nu = P + (a.auto_shared ? 1 : 0);
    const int Imax = a.I > a.I_sh ? a.I : a.I_sh;
    const int hstride = Imax;
    // gate/up
    if (phases & 1) {
        const int CPR = a.H / 32;
        const int cps = pick_cps(CPR);
        const int S = CPR / cps;
        const int nt = a.auto_shared ? a.T : (a.T < P ? a.T : P);  // worst case tokens per expert
        int RB = 16;
        auto lds = [&](int rb) {
            return (size_t)nt * (a.H / 2) * 4 + (size_t)nt * CPR * 4 + (size_t)nt * 2 * rb * S * 4 +
                   (size_t)nt * rb * 2;
        };
        while (RB > 8 && (lds(RB) > 56 * 1024 || Imax % RB)) RB /= 2;
        if (lds(RB) > 56 * 1024 || Imax % RB || a.I % RB || (a.shared && a.I_sh % RB))
            return hipErrorInvalidValue;
        dim3 grid((Imax + RB - 1) / RB, nu);
        size_t L = lds(RB);
        switch (cps) {
            case 4: hipLaunchKernelGGL((k_dec_gateup<MODE, 4>), grid, dim3(kThreads), L, s, a, hbuf, RB, hstride); break;
            case 3: hipLaunchKernelGGL((k_dec_gateup<MODE, 3>), grid, dim3(kThreads), L, s, a, hbuf, RB, hstride); break;
            case 2: hipLaunchKernelGGL((k_dec_gateup<MODE, 2>), grid, dim3(kThreads), L, s, a, hbuf, RB, hstride); break;
            default: hipLaunchKernelGGL((k_dec_gateup<MODE, 1>), grid, dim3(kThreads), L, s, a, hbuf, RB, hstride); break;
        }
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    // down + combine
    if (phases & 2) {
        const int CPR = a.I / 32;
        const int cps = pick_cps(CPR);
        const int S = CPR / cps;
        int RBD = 8;
        while (RBD > 1 && nu * RBD * S > kThreads) RBD /= 2;
        if (a.H % RBD) return hipErrorInvalidValue;
        size_t L = (size_t)PT * CPR * 4 + (size_t)PT * RBD * S * 4 + (size_t)PT * RBD * 4;
        dim3 grid(a.H / RBD);
        switch (cps) {
            case 4: hipLaunchKernelGGL((k_dec_down<MODE, 4>), grid, dim3(kThreads), L, s, a, hbuf, RBD, hstride); break;
            case 3: hipLaunchKernelGGL((k_dec_down<MODE, 3>), grid, dim3(kThreads), L, s, a, hbuf, RBD, hstride); break;
            case 2: hipLaunchKernelGGL((k_dec_down<MODE, 2>), grid, dim3(kThreads), L, s, a, hbuf, RBD, hstride); break;
            default: hipLaunchKernelGGL((k_dec_down<MODE, 1>), grid, dim3(kThreads), L, s, a, hbuf, RBD, hstride); break;
        }
        return hipGetLastError();
    }
    return hipSuccess;
}

}  // namespace

size_t decode_workspace_bytes(const FwdArgs& a) {
    const int PT = a.P + (a.auto_shared ? a.T : 0);
    const int Imax = a.I > a.I_sh ? a.I : a.I_sh;
    return (size_t)PT * Imax * 2;
}

hipError_t launch_decode(const FwdArgs& a, uint16_t* hbuf, int phases, hipStream_t s) {
    return a.quant_mode == BRX_QUANT_AFFINE ? launch_mode<BRX_QUANT_AFFINE>(a, hbuf, phases, s)
                                            : launch_mode<BRX_QUANT_MXFP4>(a, hbuf, phases, s);
}

}  // namespace brx
