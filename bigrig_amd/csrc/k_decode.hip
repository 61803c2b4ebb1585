// Decode (1-8 tokens): fused gather-GEMV over the routed experts' packed 4-bit weights.
//
// Replaces the per-row `mx.gather_qmm(x, w, scales, biases, rhs_indices=slots,
// transpose=True)` of StreamingSwitchGLU._proj (bigrig_engine/stream.py:1605-1631) for the
// three projections, the SwiGLU between them (stream.py:1164-1166) and the caller's
// router-weighted combine (stream.py:1523-1525).
//
// Two kernels per layer:
//   k_dec_gateup  grid (row block, expert entry): gate and up rows of one expert for every
//                 token routed to it, act() in the epilogue, h -> bf16 workspace; its blocks of
//                 row block 0 also record the entry table the down kernel reads.
//   k_dec_down    grid (row block of H): down rows of every entry, each pair's bf16 row result,
//                 and the k-ordered combine out[t] = sum_j w[t,j] * y[t,j].
// An entry is a run of at most 8 pairs routed to one expert (so an expert is read once for all
// the step's tokens that chose it), in order of first appearance; the shared expert, when the
// layer has one, is the last entry and takes every token.
//
// A row of K inputs is CPR = K/32 chunks of 16 bytes (32 nibbles); SP consecutive lanes own one
// row, lane `seg` the 4 chunks seg + SP j (so each load instruction reads SP adjacent chunks of
// the row). Each wave derives its entry
// itself (ballots and lane reads, no LDS and no barrier), then issues every weight, scale and
// activation load before it waits on any of them, and the SP lane partials of a row are summed
// by an in-wave xor butterfly: a launch costs the routing read, one slot-table read and one
// round trip for the weights. Dequant is folded into the dot product: for a chunk with scale s
// and bias b,
//   sum_i (s q_i + b) x_i = s * sum_i (128 + q_i) x_i + (b - 128 s) * sum_i x_i,
// where (128 + q_i) is formed as an exact bf16 by bit operations and the products accumulate
// in fp32 through v_dot2_f32_bf16. For MXFP4 the hardware converts two e2m1 codes to a bf16
// pair and the e8m0 scale multiplies the chunk sum. A row's value does not depend on which
// other rows or tokens share the launch.
#include "brx_internal.h"

namespace brx {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxTok = 8;
constexpr int kMaxU = 65;     // 64 routed pairs + the shared expert
constexpr int kCPS = 4;       // chunks per lane segment

struct DecEntry {
    int32_t slot;             // pool slot, or -1 for the shared expert
    int32_t nt;
    int32_t pair[kMaxTok];    // pair index: p, or P + t for the shared expert
};

struct DecTable {
    int32_t n;
    int32_t pad[3];
    DecEntry ent[kMaxU];
};

// One entry as a wave sees it: its expert, slot, token count and the pairs it covers (a lane
// mask over the pairs; the shared entry covers pairs P + t for every token t instead).
struct Entry {
    int e, slot, nt;
    bool shared;
    uint64_t mm;
};

__device__ __forceinline__ int rl(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }

// The slot table as the calling wave holds it: lane l has g2s[l + 64 j] in v[j]. Passed by
// value and only indexed with constants, so it stays in registers.
constexpr int kG = 8;                            // E <= 512
struct G2S {
    int v[kG];
};
__device__ __forceinline__ G2S load_g2s(const FwdArgs& a) {
    const int lane = threadIdx.x & 63;
    G2S g;
#pragma unroll
    for (int j = 0; j < kG; ++j) {
        const int ge = lane + kWave * j;
        g.v[j] = ge < a.E ? a.g2s[ge] : 0;
    }
    return g;
}

// Entry u of the step, computed by the calling wave (all results wave-uniform) from the
// lane's pair expert `e_raw` (lanes < P) and the slot table. Returns false when u is past the
// last entry.
__device__ __forceinline__ bool plan_entry(const FwdArgs& a, int u, int e_raw, const G2S gt,
                                           Entry& en, int& n_out) {
    const int lane = threadIdx.x & 63;
    const int P = a.P;
    const int emax = a.shared ? a.E : a.E - 1;   // id E names the shared expert
    const int e = lane < P ? min(max(e_raw, 0), emax) : -1;
    int occ = 0;
    for (int q = 0; q < P; ++q) occ += (q < lane && rl(e, q) == e) ? 1 : 0;
    const bool lead = lane < P && (occ % kMaxTok) == 0;
    const uint64_t mask = __ballot(lead);
    const int nr = __popcll(mask);
    const int n = nr + (a.auto_shared ? 1 : 0);
    n_out = n;
    if (u >= n) return false;
    if (u < nr) {
        uint64_t m = mask;
        for (int i = 0; i < u; ++i) m &= m - 1;
        const int pu = __builtin_ctzll(m);
        const int eu = rl(e, pu), occ0 = rl(occ, pu);
        const bool member = lane < P && e == eu && occ >= occ0 && occ < occ0 + kMaxTok;
        en.mm = __ballot(member);
        en.e = eu;
        en.nt = __popcll(en.mm);
        en.shared = false;
        int s = -1;
        if (eu < a.E) {
            const int gj = eu >> 6;
            int gv = gt.v[0];
#pragma unroll
            for (int j = 1; j < kG; ++j) gv = j == gj ? gt.v[j] : gv;
            s = min(max(rl(gv, eu & 63), 0), a.capacity - 1);
        }
        en.slot = s;
    } else {
        en.e = a.E;
        en.nt = a.T;
        en.slot = -1;
        en.shared = true;
        en.mm = 0;
    }
    return true;
}

// Routing inside the launch (a whole MoE block in decode): every block ranks the logits of
// every token itself (wave w takes tokens w, w + 4, ...) into s_e[t * k + r]; the block that
// `publish`es also writes idx, the routing weights and the shared-expert gate for the down
// kernel and the caller.
template <int kPer>
__device__ __forceinline__ void route_tokens(const FwdArgs& a, int32_t* s_e, bool publish) {
    const int lane = threadIdx.x & 63;
    const int E = a.E, k = a.k;
    for (int t = threadIdx.x >> 6; t < a.T; t += kThreads / kWave) {
        const float* l = a.logits + (int64_t)t * (E + 1);
        float v[kPer];
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int e = lane + kWave * i;
            v[i] = e < E ? l[e] : 0.0f;
        }
        int sel_e;
        float sel_v;
        wave_topk<kPer>(v, E, k, sel_e, sel_v);
        if (lane < k) s_e[t * k + lane] = sel_e;
        if (publish) {
            const float w = wave_route_weight<kPer>(v, E, k, a.route_mode, sel_v);
            if (lane < k) {
                a.route_idx[t * k + lane] = sel_e;
                a.route_w[t * k + lane] = w;
            }
            if (lane == 0 && a.route_sg) a.route_sg[t] = 1.0f / (1.0f + expf(-l[E]));
        }
    }
}

// Walks an entry's pairs in order: next() returns the pair index, tok the token it reads.
struct PairIter {
    uint64_t rem;
    int i;
    __device__ __forceinline__ int next(const FwdArgs& a, const Entry& en, int& tok) {
        int q;
        if (en.shared) {
            q = a.P + i;
            tok = i;
        } else {
            q = __builtin_ctzll(rem);
            rem &= rem - 1;
            tok = pair_tok(a, q);
        }
        ++i;
        return q;
    }
};

__device__ __forceinline__ const uint8_t* slot_base(const FwdArgs& a, int slot) {
    return slot >= 0 ? a.slots + (int64_t)slot * a.slot_stride : a.shared;
}

struct Seg {
    uint4 w[kCPS];
    float s[kCPS];   // scale per chunk
    float b[kCPS];   // affine: bias - 128 * scale per chunk; mxfp4: unused
};

// Issue the loads of one row segment (no waiting): chunks seg + SP * j, j < kCPS, so that the
// SP lanes of a row read SP consecutive 16-byte chunks per load instruction. Chunks past the
// row are clamped to its last chunk (loaded and then ignored), so no load sits behind a branch.
template <int MODE, int SP>
__device__ __forceinline__ void seg_load(const uint8_t* base, const Proj& P, int row, int seg,
                                         int scale_f16, Seg& sg) {
    const int n_in = P.n_in;
    const int cpr = n_in / 32;
    const uint4* wrow = reinterpret_cast<const uint4*>(base + P.w + (int64_t)row * (n_in / 2));
#pragma unroll
    for (int j = 0; j < kCPS; ++j) sg.w[j] = wrow[min(seg + SP * j, cpr - 1)];
    if constexpr (MODE == BRX_QUANT_AFFINE) {
        const int G = n_in / 64;
        const uint16_t* sp = reinterpret_cast<const uint16_t*>(base + P.s) + (int64_t)row * G;
        const uint16_t* bp = reinterpret_cast<const uint16_t*>(base + P.b) + (int64_t)row * G;
        uint32_t sv[kCPS], bv[kCPS];
#pragma unroll
        for (int j = 0; j < kCPS; ++j) {
            const int g = min(seg + SP * j, cpr - 1) >> 1;
            sv[j] = sp[g];
            bv[j] = bp[g];
        }
#pragma unroll
        for (int j = 0; j < kCPS; ++j) {
            float s = scale_f16 ? h2f(sv[j]) : bf2f(sv[j]);
            float b = scale_f16 ? h2f(bv[j]) : bf2f(bv[j]);
            sg.s[j] = s;
            sg.b[j] = b - 128.0f * s;
        }
    } else {
        const uint8_t* sp = base + P.s + (int64_t)row * cpr;
#pragma unroll
        for (int j = 0; j < kCPS; ++j) {
            sg.s[j] = e8m0_f32(sp[min(seg + SP * j, cpr - 1)]);
            sg.b[j] = 0.0f;
        }
    }
}

// One chunk of activations as the dot needs it.
struct XChunk {
    uint32_t w[16];   // affine: pair-permuted (x_i, x_{i+4}) per 8; mxfp4: natural (x_2i, x_2i+1)
    float sum;        // affine: sum of the 32 values
};

// From natural-order memory (x): permute for the affine dot, sum the chunk.
template <int MODE>
__device__ __forceinline__ void x_prepare(const uint4 raw[4], XChunk& xc) {
    if constexpr (MODE == BRX_QUANT_AFFINE) {
        float s = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            uint32_t in[4] = {raw[q].x, raw[q].y, raw[q].z, raw[q].w}, o[4];
            perm8(in, o);
#pragma unroll
            for (int z = 0; z < 4; ++z) {
                xc.w[4 * q + z] = o[z];
                s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, in[z]),
                                                    __builtin_bit_cast(bf16x2_t, 0x3F803F80u), s,
                                                    false);
            }
        }
        xc.sum = s;
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            xc.w[4 * q + 0] = raw[q].x;
            xc.w[4 * q + 1] = raw[q].y;
            xc.w[4 * q + 2] = raw[q].z;
            xc.w[4 * q + 3] = raw[q].w;
        }
        xc.sum = 0.f;
    }
}

// From the h buffer, which is stored in the order the dot needs (see h_pos).
template <int MODE>
__device__ __forceinline__ void h_prepare(const uint4 raw[4], XChunk& xc) {
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        uint32_t in[4] = {raw[q].x, raw[q].y, raw[q].z, raw[q].w};
#pragma unroll
        for (int z = 0; z < 4; ++z) {
            xc.w[4 * q + z] = in[z];
            if constexpr (MODE == BRX_QUANT_AFFINE)
                s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, in[z]),
                                                    __builtin_bit_cast(bf16x2_t, 0x3F803F80u), s,
                                                    false);
        }
    }
    xc.sum = s;
}

// Dot of chunk j of a loaded segment with a prepared activation chunk.
template <int MODE>
__device__ __forceinline__ float chunk_dot(const Seg& sg, int j, const XChunk& xc) {
    uint32_t wd[4] = {sg.w[j].x, sg.w[j].y, sg.w[j].z, sg.w[j].w};
    float acc = 0.0f;
    if constexpr (MODE == BRX_QUANT_AFFINE) {
#pragma unroll
        for (int q = 0; q < 4; ++q) acc = dot8_q4(wd[q], xc.w + 4 * q, acc);
        return fmaf(sg.s[j], acc, sg.b[j] * xc.sum);
    } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t v = wd[q];
            acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, 1.0f, 0),
                                                  __builtin_bit_cast(bf16x2_t, xc.w[4 * q + 0]), acc, false);
            acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, 1.0f, 1),
                                                  __builtin_bit_cast(bf16x2_t, xc.w[4 * q + 1]), acc, false);
            acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, 1.0f, 2),
                                                  __builtin_bit_cast(bf16x2_t, xc.w[4 * q + 2]), acc, false);
            acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(v, 1.0f, 3),
                                                  __builtin_bit_cast(bf16x2_t, xc.w[4 * q + 3]), acc, false);
        }
        return sg.s[j] * acc;
    }
}

template <int SP>
__device__ __forceinline__ float seg_reduce(float v) {
#pragma unroll
    for (int off = SP / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Position of element r of a row in the stored h layout: pair-permuted within 8 for the
// affine down projection, natural for MXFP4.
template <int MODE>
__device__ __forceinline__ int h_pos(int r) {
    if constexpr (MODE == BRX_QUANT_AFFINE) {
        const int m = r & ~7, i = r & 7;
        return m + (i < 4 ? 2 * i : 2 * (i - 4) + 1);
    } else {
        return r;
    }
}

// ------------------------------------------------------------------ gate/up
// Thread t owns row (t / SP) of the block's RB = 256 / SP rows and segment (t % SP), for both
// the gate and the up projection.
template <int MODE, int SP, int KP>
__global__ __launch_bounds__(kThreads) void k_dec_gateup(FwdArgs a, uint16_t* __restrict__ hbuf,
                                                         int hstride, DecTable* __restrict__ table) {
    constexpr int RB = kThreads / SP;
    const int lane = threadIdx.x & 63;
    const G2S gt = load_g2s(a);
    int e_raw;
    if constexpr (KP > 0) {   // routed here: KP logits per lane (E <= 64 KP)
        __shared__ int32_t s_e[kWave];   // P <= 64 pairs
        route_tokens<KP>(a, s_e, blockIdx.x == 0 && blockIdx.y == 0);
        __syncthreads();
        e_raw = lane < a.P ? s_e[lane] : 0;
    } else {
        e_raw = lane < a.P ? a.pexp[lane] : 0;
    }
    Entry en;
    int n;
    if (!plan_entry(a, blockIdx.y, e_raw, gt, en, n)) return;
    const int tid = threadIdx.x;
    if (blockIdx.x == 0 && tid == 0) {        // the entry table for the down kernel
        DecEntry& d = table->ent[blockIdx.y];
        d.slot = en.slot;
        d.nt = en.nt;
        PairIter it{en.mm, 0};
        for (int i = 0; i < en.nt; ++i) {
            int tok;
            d.pair[i] = it.next(a, en, tok);
        }
        if (blockIdx.y == 0) table->n = n;
    }
    const bool sh = en.e >= a.E;
    const int inter = sh ? a.I_sh : a.I;
    const int r0 = blockIdx.x * RB;
    if (r0 >= inter) return;
    const Layout& L = sh ? a.lay_sh : a.lay;
    const uint8_t* base = slot_base(a, en.slot);
    const int H = a.H, CPR = H / 32;
    const int rr = tid / SP, seg = tid % SP;
    const int row = min(r0 + rr, inter - 1);

    Seg g, v;
    seg_load<MODE, SP>(base, L.p[0], row, seg, a.scale_f16, g);
    seg_load<MODE, SP>(base, L.p[1], row, seg, a.scale_f16, v);
    float bg = 0.f, bu = 0.f;
    if (L.p[0].bias >= 0) {
        bg = bf2f(reinterpret_cast<const uint16_t*>(base + L.p[0].bias)[row]);
        bu = bf2f(reinterpret_cast<const uint16_t*>(base + L.p[1].bias)[row]);
    }
    PairIter pit{en.mm, 0};
    for (int i = 0; i < en.nt; ++i) {
        int tok;
        const int pair = pit.next(a, en, tok);
        const uint4* xp = reinterpret_cast<const uint4*>(a.x + (int64_t)tok * H);
        uint4 xr[kCPS][4];
#pragma unroll
        for (int j = 0; j < kCPS; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) xr[j][q] = xp[min(seg + SP * j, CPR - 1) * 4 + q];
        float pg = 0.f, pu = 0.f;
#pragma unroll
        for (int j = 0; j < kCPS; ++j) {
            if (seg + SP * j < CPR) {
                XChunk xc;
                x_prepare<MODE>(xr[j], xc);
                pg += chunk_dot<MODE>(g, j, xc);
                pu += chunk_dot<MODE>(v, j, xc);
            }
        }
        pg = seg_reduce<SP>(pg);
        pu = seg_reduce<SP>(pu);
        if (seg == 0 && r0 + rr < inter) {
            float h = act_apply(a.act, pg + bg, pu + bu, a.alpha, a.limit);
            hbuf[(int64_t)pair * hstride + h_pos<MODE>(r0 + rr)] = (uint16_t)f2bf(h);
        }
    }
}

// ------------------------------------------------------------------ down + combine
// Items (entry u, row rr, seg) in that order; SP consecutive lanes own one (entry, row).
template <int MODE, int SP>
__global__ __launch_bounds__(kThreads) void k_dec_down(FwdArgs a, const uint16_t* __restrict__ hbuf,
                                                       int RBD, int hstride,
                                                       const DecTable* __restrict__ table) {
    extern __shared__ float ys[];         // [PT][RBD]
    const int tid = threadIdx.x;
    const int P = a.P;
    const int PT = P + (a.auto_shared ? a.T : 0);
    const int I = a.I, CPR = I / 32;
    const int n0 = blockIdx.x * RBD;
    const int H = a.H;
    const int n = table->n;
    const int W = n * RBD * SP;
    for (int b0 = 0; b0 < W; b0 += kThreads) {
        const int it = b0 + tid;
        const bool valid = it < W;
        const int u = valid ? it / (RBD * SP) : 0;
        const int rem = it - u * RBD * SP;
        const int rr = valid ? rem / SP : 0;
        const int seg = valid ? rem - rr * SP : SP;
        const DecEntry& d = table->ent[u];
        const int slot = d.slot;
        const int nt = valid ? d.nt : 0;
        const uint8_t* base = slot_base(a, slot);
        const Layout& L = slot < 0 ? a.lay_sh : a.lay;
        const int sg0 = min(seg, SP - 1);
        Seg sg;
        seg_load<MODE, SP>(base, L.p[2], n0 + rr, sg0, a.scale_f16, sg);
        // the SP lanes of one (entry, row) share nt; lanes past W have nt = 0 and only take
        // part in the shuffles
        int ntg = nt;
#pragma unroll
        for (int off = SP / 2; off >= 1; off >>= 1) ntg = max(ntg, __shfl_xor(ntg, off, kWave));
        for (int i = 0; i < ntg; ++i) {
            const int pi = d.pair[i < kMaxTok ? i : 0];
            const uint4* hp = reinterpret_cast<const uint4*>(hbuf + (int64_t)pi * hstride);
            uint4 hr[kCPS][4];
#pragma unroll
            for (int j = 0; j < kCPS; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) hr[j][q] = hp[min(sg0 + SP * j, CPR - 1) * 4 + q];
            float p = 0.0f;
#pragma unroll
            for (int j = 0; j < kCPS; ++j) {
                if (valid && sg0 + SP * j < CPR && i < nt) {
                    XChunk xc;
                    h_prepare<MODE>(hr[j], xc);
                    p += chunk_dot<MODE>(sg, j, xc);
                }
            }
            p = seg_reduce<SP>(p);
            if (valid && seg == 0 && i < nt) ys[pi * RBD + rr] = p;
        }
    }
    __syncthreads();

    // each pair's row result, rounded to bf16 as the projection's output
    for (int it = tid; it < PT * RBD; it += kThreads) {
        int p = it / RBD, rr = it - p * RBD;
        float y = ys[it];
        int nn = n0 + rr;
        if (a.has_bias) {
            int e = p < P ? min(max(a.pexp[p], 0), a.shared ? a.E : a.E - 1) : a.E;
            int s = -1;
            if (e < a.E) s = min(max(a.g2s[e], 0), a.capacity - 1);
            const Layout& L = s < 0 ? a.lay_sh : a.lay;
            y += bf2f(reinterpret_cast<const uint16_t*>(slot_base(a, s) + L.p[2].bias)[nn]);
        }
        uint32_t yb = f2bf(y);
        ys[it] = bf2f(yb);
        if (a.yun && p < P) a.yun[(int64_t)pair_row(a, p) * H + nn] = (uint16_t)yb;
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

int pow2ceil(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}

template <int MODE, int SP>
hipError_t launch_gateup(const FwdArgs& a, uint16_t* hbuf, DecTable* table, int nu, int Imax,
                         hipStream_t s) {
    constexpr int RB = kThreads / SP;
    dim3 grid((Imax + RB - 1) / RB, nu), block(kThreads);
#define BRX_GU(KP) hipLaunchKernelGGL((k_dec_gateup<MODE, SP, KP>), grid, block, 0, s, a, hbuf, Imax, table)
    if (!a.logits) BRX_GU(0);
    else if (a.E <= 64) BRX_GU(1);
    else if (a.E <= 128) BRX_GU(2);
    else if (a.E <= 256) BRX_GU(4);
    else BRX_GU(8);
#undef BRX_GU
    return hipGetLastError();
}

template <int MODE, int SP>
hipError_t launch_down(const FwdArgs& a, uint16_t* hbuf, DecTable* table, int nu, int PT, int Imax,
                       hipStream_t s) {
    int RBD = 1;
    while (RBD < 16 && nu * (RBD * 2) * SP <= kThreads && a.H % (RBD * 2) == 0) RBD *= 2;
    size_t lds = (size_t)PT * RBD * 4;
    hipLaunchKernelGGL((k_dec_down<MODE, SP>), dim3(a.H / RBD), dim3(kThreads), lds, s, a, hbuf, RBD,
                       Imax, table);
    return hipGetLastError();
}

#define BRX_SEG_CASES(FN, ...)                                                   \
    do {                                                                         \
        if (sp_ == 1) return FN<MODE, 1>(__VA_ARGS__);                           \
        if (sp_ == 2) return FN<MODE, 2>(__VA_ARGS__);                           \
        if (sp_ == 4) return FN<MODE, 4>(__VA_ARGS__);                           \
        if (sp_ == 8) return FN<MODE, 8>(__VA_ARGS__);                           \
        if (sp_ == 16) return FN<MODE, 16>(__VA_ARGS__);                         \
        if (sp_ == 32) return FN<MODE, 32>(__VA_ARGS__);                         \
        return hipErrorInvalidValue;                                             \
    } while (0)

template <int MODE>
hipError_t dispatch_gateup(const FwdArgs& a, uint16_t* hbuf, DecTable* table, int nu, int Imax,
                           hipStream_t s) {
    const int sp_ = pow2ceil((a.H / 32 + kCPS - 1) / kCPS);
    BRX_SEG_CASES(launch_gateup, a, hbuf, table, nu, Imax, s);
}

template <int MODE>
hipError_t dispatch_down(const FwdArgs& a, uint16_t* hbuf, DecTable* table, int nu, int PT, int Imax,
                         hipStream_t s) {
    const int sp_ = pow2ceil((a.I / 32 + kCPS - 1) / kCPS);
    BRX_SEG_CASES(launch_down, a, hbuf, table, nu, PT, Imax, s);
}

template <int MODE>
hipError_t launch_mode(const FwdArgs& a, uint16_t* hbuf, DecTable* table, int phases, hipStream_t s) {
    const int P = a.P;
    const int PT = P + (a.auto_shared ? a.T : 0);
    const int nu = P + (a.auto_shared ? 1 : 0);
    const int Imax = a.I > a.I_sh ? a.I : a.I_sh;
    if (phases & 1) {
        hipError_t err = dispatch_gateup<MODE>(a, hbuf, table, nu, Imax, s);
        if (err != hipSuccess) return err;
    }
    if (phases & 2) {
        hipError_t err = dispatch_down<MODE>(a, hbuf, table, nu, PT, Imax, s);
        if (err != hipSuccess) return err;
    }
    return hipSuccess;
}

inline size_t table_bytes() { return (sizeof(DecTable) + 255) & ~(size_t)255; }

}  // namespace

size_t decode_workspace_bytes(const FwdArgs& a) {
    const int PT = a.P + (a.auto_shared ? a.T : 0);
    const int Imax = a.I > a.I_sh ? a.I : a.I_sh;
    return table_bytes() + (size_t)PT * Imax * 2;
}

hipError_t launch_decode(const FwdArgs& a, void* ws, int phases, hipStream_t s) {
    DecTable* table = reinterpret_cast<DecTable*>(ws);
    uint16_t* hbuf = reinterpret_cast<uint16_t*>(reinterpret_cast<char*>(ws) + table_bytes());
    return a.quant_mode == BRX_QUANT_AFFINE ? launch_mode<BRX_QUANT_AFFINE>(a, hbuf, table, phases, s)
                                            : launch_mode<BRX_QUANT_MXFP4>(a, hbuf, table, phases, s);
}

}  // namespace brx
