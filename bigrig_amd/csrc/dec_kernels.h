// Decode (1-8 tokens): fused gather-GEMV over the routed experts' packed weights. The kernels
// and their launchers, templated on the weight mode; k_decode.hip and k_decode_wide.hip each
// instantiate some of the modes (every translation unit launches only its own kernels).
//
// Replaces the per-row `mx.gather_qmm(x, w, scales, biases, rhs_indices=slots,
// transpose=True)` of StreamingSwitchGLU._proj (bigrig_engine/stream.py:1605-1631) for the
// three projections, the SwiGLU between them (stream.py:1164-1166) and the caller's
// router-weighted combine (stream.py:1523-1525).
//
// Gate/up, then down:
//   k_dec_gateup1  one token: one (entry, row) item per row group; every block ranks the
//                  token's top-k itself and block 0 records the entry table.
//   k_dec_gateup   several tokens with at most 32 possible entries (or one token the above
//                  does not take): grid (row block, entry row y < 16), gate and up rows of one
//                  expert for every token routed to it (entries y, y + 16, ...), act() in the
//                  epilogue, h -> bf16 workspace; its blocks of row block 0 record the entry
//                  table. With the layer's router logits given, every block ranks the top-k.
//   k_dec_plan + k_dec_gateupT  several tokens with more possible entries: one block ranks and
//                  plans the step once, then one block per (entry, row block).
//   k_dec_down_fit / k_dec_down  grid (row block of H): down rows of every entry, each pair's
//                  bf16 row result, and the k-ordered combine out[t] = sum_j w[t,j] * y[t,j].
//   k_dec_downT + k_combine  after the plan, when every block cannot stage every pair's h row:
//                  one block per (entry, row block), then the combine.
// An entry is a run of pairs routed to one expert (at most 8; at most 4 from the plan), so an
// expert is read once for all the step's tokens that chose it, numbered in order of first
// appearance; the shared expert, when the layer has one, is the last entry and takes every
// token. A row's value depends only on the row split (SP, UPL), which the launch fixes from the
// layer's widths and whether the step has one token or several.
//
// A weight row of K inputs is U = K/64 units of 64 codes: 8 * bits bytes for a b-bit affine
// row (one scale group of 64 codes, or half of one of 128), 32 bytes for MXFP4 (two groups whose
// two e8m0 scales are one 16-bit load). SP consecutive lanes own a row, lane s the UPL units
// s + SP j, so each load instruction of a row group reads SP adjacent units. The activations a
// block multiplies (x for gate/up, h for down) are staged once in LDS in the order the dot
// product wants them, with each unit's sum beside it; the lanes then read them from LDS
// instead of re-fetching them per row. Dequantization is folded into the dot product: for a
// unit with scale s and bias b,
//   sum_i (s q_i + b) x_i = s * sum_i (128 + q_i) x_i + (b - 128 s) * sum_i x_i,
// where (128 + q_i) is formed as an exact bf16 by bit operations (8-bit codes: q_i itself,
// converted through fp32, and no offset) and the products accumulate in fp32 through
// v_dot2_f32_bf16; for MXFP4 the hardware converts two e2m1 codes to a bf16 pair and each
// group's e8m0 scale multiplies its sum. A row's value does not depend on which other rows or
// tokens share the launch.
#pragma once

#include "brx_internal.h"

namespace brx {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxTok = 8;
constexpr int kMaxU = 65;     // 64 routed pairs + the shared expert
constexpr int kXU = 144;      // LDS bytes per staged activation unit: 64 bf16 + 16 pad
constexpr int kDownLds = 96 * 1024;   // staged h budget of the down kernel
constexpr int kEntryRows = 16;        // block rows of the one-launch several-token gate/up kernel

struct DecEntry {
    int32_t slot;             // pool slot, or -1 for the shared expert
    int32_t nt;               // pairs of the entry; 0 marks a grid row past the last entry
    int32_t pad[2];
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

// Entry u of the step, computed by the calling wave (all results wave-uniform) from the
// lane's pair expert `e_raw` (lanes < P) and the slot table (staged in LDS). Returns false when
// u is past the last entry.
__device__ __forceinline__ bool plan_entry(const FwdArgs& a, int u, int e_raw, const int32_t* s_g2s,
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
        if (eu < a.E) s = slot_code(a, eu, s_g2s[eu]);
        if (s == kAbsentCode && lane == 0) note_absent(a, eu);
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
// every token itself (wave w takes tokens w and w + 4) into s_e[t * k + r]; the block that
// `publish`es also writes idx, the routing weights and the shared-expert gate for the down
// kernel and the caller. Split into the loads (issued early) and the ranking.
template <int kPer>
struct RouteRegs {
    float v[2][kPer];
};

template <int kPer>
__device__ __forceinline__ void route_load(const FwdArgs& a, RouteRegs<kPer>& rg) {
    const int lane = threadIdx.x & 63;
    const int E = a.E;
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int t = (threadIdx.x >> 6) + kWaves * tt;
        const float* l = a.logits + (int64_t)min(t, a.T - 1) * (E + 1);
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int e = lane + kWave * i;
            // clamped and used as loaded (a select here would wait for the load): lanes past E
            // hold a copy of the last logit, which every ranking and weight step masks out
            rg.v[tt][i] = l[min(e, E - 1)];
        }
    }
}

template <int kPer>
__device__ __forceinline__ void route_rank(const FwdArgs& a, const RouteRegs<kPer>& rg, int32_t* s_e,
                                           bool publish) {
    const int lane = threadIdx.x & 63;
    const int E = a.E, k = a.k;
    const RouteRule rr{a.route_bias, a.route_mode, a.n_group, a.topk_group, a.route_scale};
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int t = (threadIdx.x >> 6) + kWaves * tt;
        if (t >= a.T) break;   // wave-uniform
        int sel_e;
        float sel_v;
        wave_select<kPer>(rg.v[tt], rr, E, k, sel_e, sel_v);
        if (lane < k) s_e[t * k + lane] = sel_e;
        if (publish) {
            const float w = wave_weight<kPer>(rg.v[tt], rr, E, k, sel_e, sel_v);
            if (lane < k) {
                a.route_idx[t * k + lane] = sel_e;
                a.route_w[t * k + lane] = w;
            }
            if (lane == 0 && a.route_sg)
                a.route_sg[t] = 1.0f / (1.0f + expf(-a.logits[(int64_t)t * (E + 1) + E]));
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



// ------------------------------------------------------------------ weight units
// One unit is 64 codes of a row: 8 * bits bytes (32 for MXFP4, two 32-code groups; 128 for
// unquantized bf16 weights).
template <int MODE, int UPL>
struct Units {
    uint32_t w[UPL][2 * kBits<MODE>];
    uint32_t s[UPL];   // affine: scale bits; mxfp4: the two e8m0 bytes
    uint32_t b[UPL];   // affine: bias bits
};

// Issue the loads of one row's units (no waiting). Units past the row are clamped to its last
// unit (loaded and then ignored), so no load sits behind a branch. Affine scale groups hold
// 64 << gs codes (a group of 128 is shared by two units).
template <int MODE, int UPL>
__device__ __forceinline__ void units_load(const uint8_t* base, const Proj& P, int row, int s, int SP, int gs,
                                           Units<MODE, UPL>& u) {
    constexpr int B = kBits<MODE>;
    const int U = P.n_in / 64;
    // rows and units are 8 * B bytes aligned: 3-bit units are three 8-byte loads, the others
    // B / 2 16-byte loads
    const uint8_t* wrow = base + P.w + (int64_t)row * (P.n_in * B / 8);
#pragma unroll
    for (int j = 0; j < UPL; ++j) {
        const int un = min(s + SP * j, U - 1);
        const uint8_t* up = wrow + un * (8 * B);
        if constexpr (B == 3) {
#pragma unroll
            for (int v = 0; v < 3; ++v) {
                const uint2 q = reinterpret_cast<const uint2*>(up)[v];
                u.w[j][2 * v] = q.x;
                u.w[j][2 * v + 1] = q.y;
            }
        } else {
#pragma unroll
            for (int v = 0; v < B / 2; ++v) {
                const uint4 q = reinterpret_cast<const uint4*>(up)[v];
                u.w[j][4 * v] = q.x;
                u.w[j][4 * v + 1] = q.y;
                u.w[j][4 * v + 2] = q.z;
                u.w[j][4 * v + 3] = q.w;
            }
        }
    }
    if constexpr (kAffine<MODE>) {
        const int G = U >> gs;
        const uint16_t* sp = reinterpret_cast<const uint16_t*>(base + P.s) + (int64_t)row * G;
        const uint16_t* bp = reinterpret_cast<const uint16_t*>(base + P.b) + (int64_t)row * G;
#pragma unroll
        for (int j = 0; j < UPL; ++j) {
            const int un = min(s + SP * j, U - 1);
            u.s[j] = sp[un >> gs];
            u.b[j] = bp[un >> gs];
        }
    } else if constexpr (kScaled<MODE>) {
        const uint16_t* sp = reinterpret_cast<const uint16_t*>(base + P.s + (int64_t)row * (2 * U));
#pragma unroll
        for (int j = 0; j < UPL; ++j) {
            u.s[j] = sp[min(s + SP * j, U - 1)];
            u.b[j] = 0u;
        }
    } else {
#pragma unroll
        for (int j = 0; j < UPL; ++j) u.s[j] = u.b[j] = 0u;
    }
}

// Piece m of unit j (8 weights) as the 4 bf16 pairs the dot product takes: affine c = 128 + q
// below 8 bits, c = q at 8 (see kCodeOffset); MXFP4 the hardware's conversion of two e2m1
// codes; bf16 the weights as stored.
template <int MODE, int UPL>
__device__ __forceinline__ void piece_ops(const Units<MODE, UPL>& u, int j, int m, uint32_t (&q)[4]) {
    const uint32_t* wd = u.w[j];
    if constexpr (kAffine<MODE>) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (kBits<MODE> == 8) {
                const float c0 = (float)((wd[2 * m] >> (8 * i)) & 0xFFu);
                const float c1 = (float)((wd[2 * m + 1] >> (8 * i)) & 0xFFu);
                q[i] = (__float_as_uint(c0) >> 16) | (__float_as_uint(c1) & 0xFFFF0000u);
            } else {
                q[i] = piece_pair<kBits<MODE>>(wd, m, i) | 0x43004300u;
            }
        }
    } else if constexpr (MODE == kModeBf16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = wd[4 * m + i];
    } else {
        q[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd[m], 1.0f, 0));
        q[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd[m], 1.0f, 1));
        q[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd[m], 1.0f, 2));
        q[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(wd[m], 1.0f, 3));
    }
}

// acc + the 4 pairs of a piece against 16 bytes of staged activations, in order.
__device__ __forceinline__ float piece_dot(const uint32_t (&q)[4], uint4 xv, float acc) {
    auto d2 = [](uint32_t w, uint32_t x, float c) __attribute__((always_inline)) {
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w), __builtin_bit_cast(bf16x2_t, x), c,
                                               false);
    };
    acc = d2(q[0], xv.x, acc);
    acc = d2(q[1], xv.y, acc);
    acc = d2(q[2], xv.z, acc);
    return d2(q[3], xv.w, acc);
}

// MXFP4 units sum their two 32-code groups apart (pieces 0-3 and 4-7).
template <int MODE>
constexpr bool kTwoGroups = !kAffine<MODE> && MODE != kModeBf16;

// A unit's value from its piece sums (`hi` over pieces 4-7 for MXFP4, `lo` the rest): affine
// s lo + (b - c0 s) xsum with c0 the code offset; MXFP4 each group's sum times its e8m0 scale;
// bf16 the sum as it is.
template <int MODE, int UPL>
__device__ __forceinline__ float unit_value(const Units<MODE, UPL>& u, int j, float lo, float hi, float xsum,
                                            int scale_f16) {
    if constexpr (kAffine<MODE>) {
        const float sc = scale_f16 ? h2f(u.s[j]) : bf2f(u.s[j]);
        const float bi = scale_f16 ? h2f(u.b[j]) : bf2f(u.b[j]);
        return fmaf(sc, lo, (bi - kCodeOffset<kBits<MODE>> * sc) * xsum);
    } else if constexpr (MODE == kModeBf16) {
        return lo;
    } else {
        return e8m0_f32(u.s[j] & 0xFFu) * lo + e8m0_f32(u.s[j] >> 8) * hi;
    }
}

// Dot of unit j with a staged activation unit `xu` (8 pieces of 16 bytes in LDS) whose sum is
// `xsum` (affine only).
template <int MODE, int UPL>
__device__ __forceinline__ float unit_dot(const Units<MODE, UPL>& u, int j, const uint4* xu, float xsum,
                                          int scale_f16) {
    float lo = 0.0f, hi = 0.0f;
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        uint32_t q[4];
        piece_ops<MODE, UPL>(u, j, m, q);
        if (kTwoGroups<MODE> && m >= 4) hi = piece_dot(q, xu[m], hi);
        else lo = piece_dot(q, xu[m], lo);
    }
    return unit_value<MODE, UPL>(u, j, lo, hi, xsum, scale_f16);
}

// Sums over aligned groups of 2, 4, 8 and 16 lanes through DPP (quad_perm [1,0,3,2] and
// [2,3,0,1], row_half_mirror, row_mirror); every lane of the group receives the sum.
__device__ __forceinline__ float sum8_dpp(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    return v;
}

// Sum over the SP consecutive lanes of a row group (SP a power of two, <= 64).
__device__ __forceinline__ float group_sum(float v, int SP) {
    if (SP >= 2) v += dpp_f<0xB1>(v);
    if (SP >= 4) v += dpp_f<0x4E>(v);
    if (SP >= 8) v += dpp_f<0x141>(v);
    if (SP >= 16) v += dpp_f<0x140>(v);
    if (SP >= 32) v += lane_xor16_f(v);
    if (SP >= 64) v += lane_xor32_f(v);
    return v;
}

// Max of a non-negative integer over the SP consecutive lanes of a row group, the same steps as
// group_sum.
__device__ __forceinline__ int group_max(int v, int SP) {
    uint32_t u = (uint32_t)v;
    if (SP >= 2) u = max(u, dpp_u<0xB1>(u));
    if (SP >= 4) u = max(u, dpp_u<0x4E>(u));
    if (SP >= 8) u = max(u, dpp_u<0x141>(u));
    if (SP >= 16) u = max(u, dpp_u<0x140>(u));
    if (SP >= 32) u = max(u, lane_xor16(u));
    if (SP >= 64) u = max(u, lane_xor32(u));
    return (int)u;
}

// ------------------------------------------------------------------ activation staging
// Stage `nrows` activation rows of K bf16 (row i at src + row_of(i) * K) into LDS as units of
// 8 pieces (kXU bytes a unit), each piece in the order the dot product wants (affine: pairs
// (x_i, x_{i+4}); MXFP4: natural), and each unit's sum (affine) in `sums` [nrows][U]. A thread
// fetches up to kStageB pieces before it waits on any of them. The 8 pieces of a unit are 8
// consecutive threads, so the unit sum is a fixed 3-step butterfly.
constexpr int kStageB = 4;
struct StageRegs {
    uint4 v[kStageB];
};

// Issue the loads of slots [base, base + kStageB): branch-free, every address clamped into the
// rows, so they can be scheduled together with any other loads issued next to them.
template <typename RowOf>
__device__ __forceinline__ void stage_issue(const uint16_t* __restrict__ src, int K, int nrows, RowOf row_of,
                                            int base, StageRegs& st) {
    const int pcs = (K / 64) * 8;
    const int per_row = (pcs + kThreads - 1) / kThreads;
    const int nslots = nrows * per_row;
#pragma unroll
    for (int b = 0; b < kStageB; ++b) {
        const int sl = min(base + b, nslots - 1);       // uniform
        const int r = sl / per_row;
        const int pi = min((sl - r * per_row) * kThreads + (int)threadIdx.x, pcs - 1);
        st.v[b] = *reinterpret_cast<const uint4*>(src + (int64_t)row_of(r) * K + (pi >> 3) * 64 + (pi & 7) * 8);
    }
}

// Write the slots [base, base + kStageB) loaded by stage_issue to LDS.
template <int MODE>
__device__ __forceinline__ void stage_store(int K, int nrows, int base, const StageRegs& st, uint8_t* xs,
                                            float* sums) {
    const int U = K / 64;
    const int pcs = U * 8;
    const int per_row = (pcs + kThreads - 1) / kThreads;
    const int nslots = nrows * per_row;
#pragma unroll
    for (int b = 0; b < kStageB; ++b) {
        const int sl = base + b;
        if (sl >= nslots) break;                        // uniform
        const int r = sl / per_row, pi = (sl - r * per_row) * kThreads + threadIdx.x;
        const bool ok = pi < pcs;
        const int un = pi >> 3, q = pi & 7;
        uint32_t in[4] = {st.v[b].x, st.v[b].y, st.v[b].z, st.v[b].w}, o[4];
        float part = 0.0f;
        if constexpr (kAffine<MODE>) {
            perm8(in, o);
#pragma unroll
            for (int z = 0; z < 4; ++z)
                part = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, in[z]),
                                                       __builtin_bit_cast(bf16x2_t, 0x3F803F80u), part, false);
        } else {
#pragma unroll
            for (int z = 0; z < 4; ++z) o[z] = in[z];
        }
        if (ok)
            *reinterpret_cast<uint4*>(xs + ((int64_t)r * U + un) * kXU + q * 16) = make_uint4(o[0], o[1], o[2], o[3]);
        if constexpr (kAffine<MODE>) {
            part = sum8_dpp(part);
            if (ok && q == 0) sums[r * U + un] = part;
        }
    }
}

// One pass of stage_dense, split so a caller can issue other loads between the two halves:
// dense_issue requests the pieces [base, base + NB * kThreads) into registers, dense_store
// writes them (and the unit sums) to LDS.
template <int NB>
struct DenseRegs {
    uint4 v[NB];
    int gi[NB];
};
template <int NB, typename RowOf>
__device__ __forceinline__ void dense_issue(const uint16_t* __restrict__ src, int K, int nrows, RowOf row_of,
                                            int base, DenseRegs<NB>& d) {
    const int pcs = (K / 64) * 8;
    const int total = nrows * pcs;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int g = min(base + b * kThreads + (int)threadIdx.x, total - 1);
        d.gi[b] = g;
        const int r = g / pcs, pi = g - r * pcs;
        const int off = row_of(r) * K + (pi >> 3) * 64 + (pi & 7) * 8;
        d.v[b] = *reinterpret_cast<const uint4*>(src + off);
    }
}
template <int MODE, int NB>
__device__ __forceinline__ void dense_store(int K, int nrows, int base, const DenseRegs<NB>& d, uint8_t* xs,
                                            float* sums) {
    const int U = K / 64;
    const int pcs = U * 8;
    const int total = nrows * pcs;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        if (base + b * kThreads >= total) break;   // uniform
        const bool ok = base + b * kThreads + (int)threadIdx.x < total;
        const int g = d.gi[b];
        const int r = g / pcs, pi = g - r * pcs;
        const int un = pi >> 3, q = pi & 7;
        uint32_t in[4] = {d.v[b].x, d.v[b].y, d.v[b].z, d.v[b].w}, o[4];
        float part = 0.0f;
        if constexpr (kAffine<MODE>) {
            perm8(in, o);
#pragma unroll
            for (int z = 0; z < 4; ++z)
                part = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, in[z]),
                                                       __builtin_bit_cast(bf16x2_t, 0x3F803F80u), part, false);
        } else {
#pragma unroll
            for (int z = 0; z < 4; ++z) o[z] = in[z];
        }
        if (ok)
            *reinterpret_cast<uint4*>(xs + ((int64_t)r * U + un) * kXU + q * 16) = make_uint4(o[0], o[1], o[2], o[3]);
        if constexpr (kAffine<MODE>) {
            part = sum8_dpp(part);
            if (ok && q == 0) sums[r * U + un] = part;
        }
    }
}

// The same staging with the pieces of all rows numbered densely (piece g of the block is row
// g / (8U), unit (g / 8) % U, piece g % 8) and handed to the threads kStageB at a time, so rows
// shorter than the block (h rows of 8-16 units) still take one round trip per kStageB * kThreads
// pieces. The 8 pieces of a unit stay on 8 consecutive lanes. `first` > 0 skips the pieces a
// caller already staged.
template <int MODE, int NB = kStageB, typename RowOf>
__device__ __forceinline__ void stage_dense(const uint16_t* __restrict__ src, int K, int nrows, RowOf row_of,
                                            uint8_t* xs, float* sums, int first = 0) {
    const int total = nrows * (K / 64) * 8;
    for (int base = first; base < total; base += NB * kThreads) {
        DenseRegs<NB> d;
        dense_issue<NB>(src, K, nrows, row_of, base, d);
        dense_store<MODE, NB>(K, nrows, base, d, xs, sums);
    }
}

// Stage `nrows` activation rows of K bf16 (row i at src + row_of(i) * K) into LDS as units of
// 8 pieces (kXU bytes a unit), each piece in the order the dot product wants (affine: pairs
// (x_i, x_{i+4}); MXFP4: natural), and each unit's sum (affine) in `sums` [nrows][U]. A thread
// fetches kStageB pieces before it waits on any of them; the 8 pieces of a unit are 8
// consecutive lanes, so the unit sum is a fixed 3-step DPP butterfly. `first` > 0 skips the
// slots a caller already staged.
template <int MODE, typename RowOf>
__device__ __forceinline__ void stage_rows(const uint16_t* __restrict__ src, int K, int nrows,
                                           RowOf row_of, uint8_t* xs, float* sums, int first = 0) {
    const int pcs = (K / 64) * 8;
    const int nslots = nrows * ((pcs + kThreads - 1) / kThreads);
    for (int base = first; base < nslots; base += kStageB) {
        StageRegs st;
        stage_issue(src, K, nrows, row_of, base, st);
        stage_store<MODE>(K, nrows, base, st, xs, sums);
    }
}

// ------------------------------------------------------------------ gate/up
// Wave w of the block owns rows w * RW + g (g = lane / SP, RW = 64 / SP) of the block's
// RB = 4 RW rows, for both the gate and the up projection.
template <int MODE, int UPL, int KP, bool MULTI>
__global__ __launch_bounds__(kThreads) void k_dec_gateup(FwdArgs a, uint16_t* __restrict__ hbuf,
                                                         int hstride, DecTable* __restrict__ table,
                                                         int lsp, int nu, int nby) {
    prefetch_args(a);
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ int32_t s_e[kWave];   // P <= 64 pairs
    const int SP = 1 << lsp;
    const int lane = threadIdx.x & 63;
    const int tid = threadIdx.x;
    const int H = a.H, U = H / 64;
    uint8_t* xs = lds;
    float* xsum = reinterpret_cast<float*>(lds + (size_t)a.T * U * kXU);
    // one round trip for the routing, the slot table and every token's activations: all their
    // loads are issued branch-free before the first wait; x is staged while the routing is
    // ranked
    __shared__ int32_t s_g2s[512];   // E <= 512
    const int gi0 = min(tid, a.E - 1), gi1 = min(tid + kThreads, a.E - 1);
    const int g2s0 = a.g2s[gi0], g2s1 = a.g2s[gi1];
    int pe = 0;
    if constexpr (KP == 0) pe = a.pexp[min(lane, a.P - 1)];
    RouteRegs<(KP > 0 ? KP : 1)> rg;
    if constexpr (KP > 0) route_load<KP>(a, rg);
    // MULTI (several tokens): most of the P + 1 possible entries are empty, so a block takes
    // entries y, y + 16, ... and stages x only once it has one, after the routing; otherwise
    // (one token) every block has its entry and x rides in the routing round trip
    constexpr bool late_x = MULTI;
    StageRegs st;
    auto tok_row = [](int i) { return i; };
    if (!late_x) stage_issue(a.x, H, a.T, tok_row, 0, st);
    if (tid < a.E) s_g2s[tid] = g2s0;
    if (tid + kThreads < a.E) s_g2s[tid + kThreads] = g2s1;
    if constexpr (KP == 0)
        if (tid < a.P) s_e[tid] = pe;
    if (!late_x) {
        stage_store<MODE>(H, a.T, 0, st, xs, xsum);
        stage_rows<MODE>(a.x, H, a.T, tok_row, xs, xsum, kStageB);
    }
    if constexpr (KP > 0) route_rank<KP>(a, rg, s_e, blockIdx.x == 0 && blockIdx.y == 0);
    __syncthreads();
    if constexpr (!MULTI) {
        const int e_raw = lane < a.P ? s_e[lane] : 0;
        Entry en;
        int n;
        if (!plan_entry(a, blockIdx.y, e_raw, s_g2s, en, n)) {
            if (blockIdx.x == 0 && tid == 0) {    // no entry here: an empty table row
                table->ent[blockIdx.y].slot = 0;
                table->ent[blockIdx.y].nt = 0;
            }
            return;
        }
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
        const int RW = kWave >> lsp;
        const int r0 = blockIdx.x * kWaves * RW;
        if (r0 >= inter) return;
        const Layout& L = sh ? a.lay_sh : a.lay;
        const uint8_t* base = code_base(a, en.slot);
        const int g = lane >> lsp, sl = lane & (SP - 1);
        const int rr = (tid >> 6) * RW + g;
        const int row = min(r0 + rr, inter - 1);

        // a two-layer expert (fc1 / fc2) has no up projection: only fc1's rows are read
        const bool gated = a.act != BRX_ACT_SILU_MLP;
        Units<MODE, UPL> ug, uu;
        units_load<MODE, UPL>(base, L.p[0], row, sl, SP, a.gshift, ug);
        if (gated) units_load<MODE, UPL>(base, L.p[1], row, sl, SP, a.gshift, uu);
        float bg = 0.f, bu = 0.f;
        if (L.p[0].bias >= 0) {
            bg = bf2f(reinterpret_cast<const uint16_t*>(base + L.p[0].bias)[row]);
            if (gated) bu = bf2f(reinterpret_cast<const uint16_t*>(base + L.p[1].bias)[row]);
        }
        PairIter pit{en.mm, 0};
        for (int i = 0; i < en.nt; ++i) {
            int tok;
            const int pair = pit.next(a, en, tok);
            float pg = 0.f, pu = 0.f;
    #pragma unroll
            for (int j = 0; j < UPL; ++j) {
                const int un = sl + SP * j;
                if (un < U) {
                    const uint4* xu = reinterpret_cast<const uint4*>(xs + ((int64_t)tok * U + un) * kXU);
                    const float sx = kAffine<MODE> ? xsum[tok * U + un] : 0.0f;
                    pg += unit_dot<MODE, UPL>(ug, j, xu, sx, a.scale_f16);
                    if (gated) pu += unit_dot<MODE, UPL>(uu, j, xu, sx, a.scale_f16);
                }
            }
            pg = group_sum(pg, SP);
            if (gated) pu = group_sum(pu, SP);
            if (sl == 0 && r0 + rr < inter) {
                const float h = en.slot == kAbsentCode ? absent_nan() : act_apply(a.act, pg + bg, pu + bu, a.alpha, a.limit);
                hbuf[(int64_t)pair * hstride + r0 + rr] = (uint16_t)f2bf(h);
            }
        }
    } else {
        const int e_raw = lane < a.P ? s_e[lane] : 0;
        // entries by, by + NB, ... (NB = the grid's rows, passed in so the kernel reads no
        // hidden argument and its argument block stays under 512 bytes); x is staged once,
        // with the first entry
        const int NB = nby;
        bool staged = false;
        for (int u = blockIdx.y; u < nu; u += NB) {
            Entry en;
            int n;
            if (!plan_entry(a, u, e_raw, s_g2s, en, n)) {
                if (blockIdx.x == 0 && tid == 0)      // entry rows past the last: empty table rows
                    for (int v = u; v < nu; v += NB) {
                        table->ent[v].slot = 0;
                        table->ent[v].nt = 0;
                    }
                return;
            }
            if (blockIdx.x == 0 && tid == 0) {        // the entry table for the down kernel
                DecEntry& d = table->ent[u];
                d.slot = en.slot;
                d.nt = en.nt;
                PairIter it{en.mm, 0};
                for (int i = 0; i < en.nt; ++i) {
                    int tok;
                    d.pair[i] = it.next(a, en, tok);
                }
                if (u == 0) table->n = n;
            }
            const bool sh = en.e >= a.E;
            const int inter = sh ? a.I_sh : a.I;
            const int RW = kWave >> lsp;
            const int r0 = blockIdx.x * kWaves * RW;
            if (r0 >= inter) continue;   // uniform
            const Layout& L = sh ? a.lay_sh : a.lay;
            const uint8_t* base = code_base(a, en.slot);
            const int g = lane >> lsp, sl = lane & (SP - 1);
            const int rr = (tid >> 6) * RW + g;
            const int row = min(r0 + rr, inter - 1);

            const bool gated = a.act != BRX_ACT_SILU_MLP;
            Units<MODE, UPL> ug, uu;
            units_load<MODE, UPL>(base, L.p[0], row, sl, SP, a.gshift, ug);
            if (gated) units_load<MODE, UPL>(base, L.p[1], row, sl, SP, a.gshift, uu);
            float bg = 0.f, bu = 0.f;
            if (L.p[0].bias >= 0) {
                bg = bf2f(reinterpret_cast<const uint16_t*>(base + L.p[0].bias)[row]);
                if (gated) bu = bf2f(reinterpret_cast<const uint16_t*>(base + L.p[1].bias)[row]);
            }
            if (!staged) {   // the weights are in flight
                stage_dense<MODE>(a.x, H, a.T, tok_row, xs, xsum);
                __syncthreads();
                staged = true;
            }
            PairIter pit{en.mm, 0};
            for (int i = 0; i < en.nt; ++i) {
                int tok;
                const int pair = pit.next(a, en, tok);
                float pg = 0.f, pu = 0.f;
    #pragma unroll
                for (int j = 0; j < UPL; ++j) {
                    const int un = sl + SP * j;
                    if (un < U) {
                        const uint4* xu = reinterpret_cast<const uint4*>(xs + ((int64_t)tok * U + un) * kXU);
                        const float sx = kAffine<MODE> ? xsum[tok * U + un] : 0.0f;
                        pg += unit_dot<MODE, UPL>(ug, j, xu, sx, a.scale_f16);
                        if (gated) pu += unit_dot<MODE, UPL>(uu, j, xu, sx, a.scale_f16);
                    }
                }
                pg = group_sum(pg, SP);
                if (gated) pu = group_sum(pu, SP);
                if (sl == 0 && r0 + rr < inter) {
                    const float h = en.slot == kAbsentCode ? absent_nan()
                                                           : act_apply(a.act, pg + bg, pu + bu, a.alpha, a.limit);
                    hbuf[(int64_t)pair * hstride + r0 + rr] = (uint16_t)f2bf(h);
                }
            }
        }
    }
}

// ------------------------------------------------------------------ gate/up, one token
// One token's gate/up: entry u is pair u (the shared expert last) and the (entry, row) items
// are dealt out one per row group, RG row groups a block, in order. Wave 0 ranks the routing,
// holds the slot table in registers and resolves every entry's slot before the block's one
// barrier -- no per-block entry planning, which for several tokens merges repeated experts --
// and block 0 records the entry table for the down kernel.
template <int MODE, int UPL, int KP>
__global__ __launch_bounds__(kThreads) void k_dec_gateup1(FwdArgs a, uint16_t* __restrict__ hbuf, int hstride,
                                                          DecTable* __restrict__ table, int lsp, int nu) {
    prefetch_args(a);
    __builtin_amdgcn_s_setprio(2);
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ int32_t s_slot[kMaxU];
    constexpr int kG = 8;                         // slot-table registers per lane (E <= 512)
    const int SP = 1 << lsp;
    const int lane = threadIdx.x & 63, tid = threadIdx.x, wv = tid >> 6;
    const int H = a.H, U = H / 64, E = a.E, P = a.P;
    const int Imax = hstride;
    uint8_t* xs = lds;
    float* xsum = reinterpret_cast<float*>(lds + (size_t)U * kXU);
    // one round trip: the routing (logits or the given pairs), the slot table (wave 0) and x
    // (every wave issues these loads, only wave 0 uses them: no branch around a load, so none is
    // waited for before x is requested; the table registers past E repeat its last entry and
    // are never selected)
    constexpr int kGn = KP > 0 ? KP : kG;   // KP * 64 >= E
    int g2s[kGn];
#pragma unroll
    for (int i = 0; i < kGn; ++i) g2s[i] = a.g2s[min(lane + kWave * i, E - 1)];
    int pe = 0;
    if constexpr (KP == 0) pe = a.pexp[min(lane, P - 1)];
    RouteRegs<(KP > 0 ? KP : 1)> rg;
    float lsg = 0.0f;   // the shared-expert gate's logit (block 0 publishes its sigmoid)
    if constexpr (KP > 0) {
        route_load<KP>(a, rg);
        lsg = a.logits[E];
    }
    StageRegs st;
    auto tok_row = [](int i) { return i; };
    stage_issue(a.x, H, 1, tok_row, 0, st);
    stage_store<MODE>(H, 1, 0, st, xs, xsum);
    stage_rows<MODE>(a.x, H, 1, tok_row, xs, xsum, kStageB);
    // the entries this block's items fall in: only their ranks are needed here (block 0 ranks
    // all k, to publish the routing and the table), so blocks of the first entries start their
    // weight loads after fewer rounds
    const int RGn = kWaves * (kWave >> lsp);          // row groups per block
    const int u_first = blockIdx.x * RGn / Imax;
    const int u_last = min(blockIdx.x * RGn + RGn - 1, nu * Imax - 1) / Imax;
    const int kr = blockIdx.x == 0 ? a.k : (u_first >= P ? 0 : min(u_last, P - 1) + 1);
    // block 0 publishes the routing and the entry table after the barrier (stores issued before
    // it would be waited for there: they count in the same in-order counter as the loads)
    int e = pe, eslot = -1;   // wave 0: rank lane's expert and its slot
    float w = 0.0f, sg = 0.0f;
    if (wv == 0) {
        // the ranking is every wave's wait: it issues ahead of the other blocks' work on the CU
        __builtin_amdgcn_s_setprio(3);
        if constexpr (KP > 0) {
            const RouteRule rr{a.route_bias, a.route_mode, a.n_group, a.topk_group, a.route_scale};
            float sel_v;
            wave_select<KP>(rg.v[0], rr, E, a.k, e, sel_v, kr);
            if (blockIdx.x == 0) {
                w = wave_weight<KP>(rg.v[0], rr, E, a.k, e, sel_v);
                if (a.route_sg) sg = 1.0f / (1.0f + expf(-lsg));
            }
        }
        // entry lane < P: expert e's slot, fetched from the lane holding its table entry
        const int ec = min(max(e, 0), E - 1);
        int v = -1;
#pragma unroll
        for (int i = 0; i < kGn; ++i) {
            const int t = __shfl(g2s[i], ec & (kWave - 1), kWave);
            if (i == (ec >> 6)) v = t;
        }
        if (lane < P) {
            if (KP > 0 && lane >= kr) {
                eslot = 0;   // an entry this block does not compute
            } else {
                eslot = slot_code(a, ec, v);
                if (eslot == kAbsentCode) note_absent(a, ec);
            }
        }
        if (lane < nu) s_slot[lane] = eslot;
        __builtin_amdgcn_s_setprio(2);
    }
    __syncthreads();
    if (wv == 0 && blockIdx.x == 0) {
        if constexpr (KP > 0) {
            if (lane < a.k) {
                a.route_idx[lane] = e;
                a.route_w[lane] = w;
            }
            if (lane == 0 && a.route_sg) a.route_sg[0] = sg;
        }
        if (lane < nu) {
            DecEntry& d = table->ent[lane];
            d.slot = eslot;
            d.nt = 1;
            d.pair[0] = lane;
        }
        if (lane == 0) table->n = nu;
    }

    const int g = lane >> lsp, sl = lane & (SP - 1);
    const int q = blockIdx.x * RGn + wv * (kWave >> lsp) + g;
    const int u = min(q / Imax, nu - 1), r = q - (q / Imax) * Imax;
    const int slot = s_slot[u];
    const bool sh = slot == -1;
    const int inter = sh ? a.I_sh : a.I;
    const bool ok = q < nu * Imax && r < inter;
    const Layout& L = sh ? a.lay_sh : a.lay;
    const uint8_t* base = code_base(a, clamp_code(a, slot));
    const int row = min(r, inter - 1);
    const bool gated = a.act != BRX_ACT_SILU_MLP;
    if (!ok) return;   // rows past a narrower entry (no barrier follows)
    Units<MODE, UPL> ug, uu;
    units_load<MODE, UPL>(base, L.p[0], row, sl, SP, a.gshift, ug);
    if (gated) units_load<MODE, UPL>(base, L.p[1], row, sl, SP, a.gshift, uu);
    float bg = 0.f, bu = 0.f;
    if (L.p[0].bias >= 0) {
        bg = bf2f(reinterpret_cast<const uint16_t*>(base + L.p[0].bias)[row]);
        if (gated) bu = bf2f(reinterpret_cast<const uint16_t*>(base + L.p[1].bias)[row]);
    }
    __builtin_amdgcn_s_setprio(0);
    float pg = 0.f, pu = 0.f;
#pragma unroll
    for (int j = 0; j < UPL; ++j) {
        const int un = sl + SP * j;
        if (un < U) {
            const uint4* xu = reinterpret_cast<const uint4*>(xs + (int64_t)un * kXU);
            const float sx = kAffine<MODE> ? xsum[un] : 0.0f;
            pg += unit_dot<MODE, UPL>(ug, j, xu, sx, a.scale_f16);
            if (gated) pu += unit_dot<MODE, UPL>(uu, j, xu, sx, a.scale_f16);
        }
    }
    pg = group_sum(pg, SP);
    if (gated) pu = group_sum(pu, SP);
    if (sl == 0) {
        const float h = slot == kAbsentCode ? absent_nan() : act_apply(a.act, pg + bg, pu + bu, a.alpha, a.limit);
        hbuf[(int64_t)u * hstride + r] = (uint16_t)f2bf(h);
    }
}

// ------------------------------------------------------------------ several tokens
// k_dec_plan: one block ranks every token's top-k once (wave t takes token t; with the pairs
// given, they are read instead) and plans the step: the pairs routed to one expert are merged,
// in pair order, into entries of at most kPlanTok pairs, numbered in order of their first pair
// (so an expert is read by one entry per kPlanTok of the step's tokens that chose it); the
// shared expert, when the layer has one, is the last entry and takes every token. It writes the
// entry table and the routing (indices, weights, shared-expert gate) that the gate/up and down
// kernels read.
constexpr int kPlanThreads = kWave * kMaxTok;
// pairs per entry the plan forms: an expert chosen by more tokens is read by more entries, so
// the blocks of a popular expert do no more than 4 tokens' dot products each
constexpr int kPlanTok = 4;

template <int KP>
__global__ __launch_bounds__(kPlanThreads) void k_dec_plan(FwdArgs a, DecTable* __restrict__ table) {
    __shared__ __attribute__((aligned(16))) int32_t s_e[kWave], s_occ[kWave];
    __shared__ int32_t s_tot[kWave], s_lq[kWave];
    __shared__ int32_t s_part[kMaxTok][2][kWave];
    __shared__ int32_t s_g2s[kPlanThreads];   // E <= 512
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int P = a.P, E = a.E, k = a.k;
    // the routing and the slot table in one round trip (the table is stored to LDS only after
    // the ranking, so no wait for it comes first)
    float v[KP > 0 ? KP : 1];
    const float* l = a.logits + (int64_t)min(wv, a.T - 1) * (E + 1);
    if constexpr (KP > 0) {
#pragma unroll
        for (int i = 0; i < KP; ++i) {
            const int e = lane + kWave * i;
            v[i] = l[min(e, E - 1)];   // clamped, used as loaded (lanes past E are masked later)
        }
    }
    float lsg = 0.0f;   // the shared-expert gate's logit
    if constexpr (KP > 0) lsg = l[E];
    const int g0 = a.g2s[min(tid, E - 1)];
    int sel_e = -1;
    float w = 0.0f;
    if constexpr (KP > 0) {
        if (wv < a.T) {   // wave t ranks token t
            const RouteRule rr{a.route_bias, a.route_mode, a.n_group, a.topk_group, a.route_scale};
            float sel_v;
            wave_select<KP>(v, rr, E, k, sel_e, sel_v);
            w = wave_weight<KP>(v, rr, E, k, sel_e, sel_v);
            if (lane < k) s_e[wv * k + lane] = sel_e;
        }
    } else {
        if (tid < P) s_e[tid] = a.pexp[tid];
    }
    if (tid < E) s_g2s[tid] = g0;
    const float sg = 1.0f / (1.0f + expf(-lsg));
    // every load has landed here, on every path (vmcnt 0), so no wait below covers the stores
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __syncthreads();
    // the routing is published after the barrier: global stores count in the same in-order
    // counter as the loads, so stores issued before the wait for g0 would be waited for too
    if constexpr (KP > 0) {
        if (wv < a.T) {
            if (lane < k) {
                a.route_idx[wv * k + lane] = sel_e;
                a.route_w[wv * k + lane] = w;
            }
            if (lane == 0 && a.route_sg) a.route_sg[wv] = sg;
        }
    }
    // pair p = lane (p < P) against the pairs q of chunk c = wave: q = 8 c .. 8 c + 7. Experts
    // are clamped (id E names the shared expert); idle pairs match nothing.
    const int emax = a.shared ? E : E - 1;
    // (the reads are unconditional -- entries past P hold no pair and are masked after the
    // read -- so each chunk's eight come in two 16-byte reads rather than eight waits)
    auto expert_of = [&](int q, int v) { return q < P ? min(max(v, 0), emax) : -1 - q; };
    auto chunk = [&](const int32_t* arr, int out[kMaxTok]) {
        const int4 lo = *reinterpret_cast<const int4*>(arr + wv * kMaxTok);
        const int4 hi = *reinterpret_cast<const int4*>(arr + wv * kMaxTok + 4);
        out[0] = lo.x; out[1] = lo.y; out[2] = lo.z; out[3] = lo.w;
        out[4] = hi.x; out[5] = hi.y; out[6] = hi.z; out[7] = hi.w;
    };
    static_assert(kMaxTok == 8, "two 16-byte reads a chunk");
    const int e = expert_of(lane, s_e[lane]);
    int ce[kMaxTok];
    chunk(s_e, ce);
#pragma unroll
    for (int i = 0; i < kMaxTok; ++i) ce[i] = expert_of(wv * kMaxTok + i, ce[i]);
    {
        int occ = 0, tot = 0;
#pragma unroll
        for (int i = 0; i < kMaxTok; ++i) {
            const int q = wv * kMaxTok + i;
            const bool m = ce[i] == e;
            occ += (m && q < lane) ? 1 : 0;
            tot += m ? 1 : 0;
        }
        s_part[wv][0][lane] = occ;
        s_part[wv][1][lane] = tot;
    }
    __syncthreads();
    if (wv == 0) {
        int occ = 0, tot = 0;
#pragma unroll
        for (int c = 0; c < kMaxTok; ++c) {
            occ += s_part[c][0][lane];
            tot += s_part[c][1][lane];
        }
        s_occ[lane] = occ;   // pairs of the same expert before this one
        s_tot[lane] = tot;   // all pairs of that expert
    }
    __syncthreads();
    // the lane of the pair that leads this pair's entry: the (occ & ~(kPlanTok - 1))-th pair of
    // its expert
    {
        const int occ0 = s_occ[lane] & ~(kPlanTok - 1);
        int co[kMaxTok];
        chunk(s_occ, co);
#pragma unroll
        for (int i = 0; i < kMaxTok; ++i) {
            const int q = wv * kMaxTok + i;
            if (ce[i] == e && co[i] == occ0) s_lq[lane] = q;
        }
    }
    __syncthreads();
    if (wv != 0) return;
    const int occ = s_occ[lane], occ0 = occ & ~(kPlanTok - 1), lq = s_lq[lane];
    const uint64_t leads = __ballot(lane < P && occ == occ0);
    const int nr = __popcll(leads);
    if (lane < P) {
        const int u = __popcll(leads & ((1ull << lq) - 1ull));
        DecEntry& d = table->ent[u];
        d.pair[occ - occ0] = lane;
        if (occ == occ0) {
            int sc = -1;
            if (e < E) sc = slot_code(a, e, s_g2s[e]);
            if (sc == kAbsentCode) note_absent(a, e);
            d.slot = sc;
            d.nt = min(kPlanTok, s_tot[lane] - occ0);
        }
    }
    if (a.auto_shared) {
        DecEntry& d = table->ent[nr];
        if (lane < a.T) d.pair[lane] = P + lane;
        if (lane == 0) {
            d.slot = -1;
            d.nt = a.T;
        }
    }
    // rows past the planned entries are empty: the down kernel reads every row it may be given
    const int n = nr + (a.auto_shared ? 1 : 0);
    for (int v = n + lane; v < kMaxU; v += kWave) {
        table->ent[v].slot = 0;
        table->ent[v].nt = 0;
    }
    if (lane == 0) table->n = n;
}

// The (entry, token group, row block) of per-entry block b: blocks u * nrb + rb with u < n take
// entry u's first kPlanTok pairs; past the n entries, the next groups of the last entry (the
// shared expert, which takes every token). Returns the row block, or -1 for a block with no
// work; u, t0 (its first pair's index in the entry), nt (its pair count), slot (entry u's slot
// code) and, for threads below kPlanTok, pair (the entry's pair t0 + thread) are set otherwise.
// Row b / nrb's entry is read together with n -- that is the block's entry for every block but
// the shared expert's later token groups, which read entry n - 1 once n is known -- and before
// any weight load, so the pairs (and the token rows staged from them) do not wait behind the
// weights: loads complete in issue order.
__device__ __forceinline__ int entry_group(const DecTable* table, int b, int nrb, int& u, int& t0, int& nt,
                                           int& slot, int& pair) {
    const int tid = threadIdx.x;
    const int n = table->n;
    u = b / nrb;
    const int rb = b - u * nrb;
    const int u0 = min(u, kMaxU - 1);
    const int2 h0 = *reinterpret_cast<const int2*>(&table->ent[u0]);   // (slot, nt)
    pair = tid < kPlanTok ? table->ent[u0].pair[tid] : 0;
    int c = 0, nt_all = h0.y;
    slot = h0.x;
    if (u >= n) {
        c = u - n + 1;
        u = n - 1;
        if (u >= 0 && u < kMaxU) {
            slot = table->ent[u].slot;
            nt_all = table->ent[u].nt;
            pair = tid < kPlanTok ? table->ent[u].pair[min(c * kPlanTok + tid, kMaxTok - 1)] : 0;
        }
    }
    if (u < 0 || u >= kMaxU) return -1;
    const int nall = min(max(nt_all, 0), kMaxTok);
    t0 = c * kPlanTok;
    nt = min(kPlanTok, nall - t0);
    return nt > 0 ? rb : -1;
}

// k_dec_gateupT: block b takes entry b / nrb of the plan and its rows (b % nrb) RB ..
// (b % nrb) RB + RB - 1, for every pair of the entry; blocks past the last entry return. One
// round trip reads the entry; the weight loads are then issued before the entry's token rows
// of x are staged, so the two overlap.
template <int MODE, int UPL>
__global__ __launch_bounds__(kThreads) void k_dec_gateupT(FwdArgs a, uint16_t* __restrict__ hbuf, int hstride,
                                                          const DecTable* __restrict__ table, int lsp, int nrb) {
    prefetch_args(a);
    __builtin_amdgcn_s_setprio(2);
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ int32_t s_tok[kMaxTok];
    const int SP = 1 << lsp;
    const int lane = threadIdx.x & 63, tid = threadIdx.x;
    const int H = a.H, U = H / 64;
    __shared__ int32_t s_pair[kPlanTok];
    int u, t0, nt;
    int eslot, epair;
    const int rb = entry_group(table, blockIdx.x, nrb, u, t0, nt, eslot, epair);
    if (rb < 0) return;   // uniform
    const int slot = clamp_code(a, eslot);
    const int PT = a.P + (a.auto_shared ? a.T : 0);
    const bool sh = slot == -1;
    const int inter = sh ? a.I_sh : a.I;
    const int RW = kWave >> lsp;
    const int r0 = rb * kWaves * RW;
    if (r0 >= inter) return;   // uniform
    const Layout& L = sh ? a.lay_sh : a.lay;
    const uint8_t* base = code_base(a, slot);
    const int g = lane >> lsp, sl = lane & (SP - 1);
    const int rr = (tid >> 6) * RW + g;
    const int row = min(r0 + rr, inter - 1);
    const bool gated = a.act != BRX_ACT_SILU_MLP;
    Units<MODE, UPL> ug, uu;
    units_load<MODE, UPL>(base, L.p[0], row, sl, SP, a.gshift, ug);
    if (gated) units_load<MODE, UPL>(base, L.p[1], row, sl, SP, a.gshift, uu);
    float bg = 0.f, bu = 0.f;
    if (L.p[0].bias >= 0) {
        bg = bf2f(reinterpret_cast<const uint16_t*>(base + L.p[0].bias)[row]);
        if (gated) bu = bf2f(reinterpret_cast<const uint16_t*>(base + L.p[1].bias)[row]);
    }
    // the entry's token rows, staged while the weights are in flight
    if (tid < nt) {
        const int pair = min(max(epair, 0), PT - 1);
        s_pair[tid] = pair;
        s_tok[tid] = pair < a.P ? pair_tok(a, pair) : pair - a.P;
    }
    __syncthreads();
    uint8_t* xs = lds;
    float* xsum = reinterpret_cast<float*>(lds + (size_t)kPlanTok * U * kXU);
    stage_dense<MODE>(a.x, H, nt, [&](int i) { return s_tok[i]; }, xs, xsum);
    __syncthreads();
    __builtin_amdgcn_s_setprio(0);
    for (int i = 0; i < nt; ++i) {
        const int pair = s_pair[i];
        float pg = 0.f, pu = 0.f;
#pragma unroll
        for (int j = 0; j < UPL; ++j) {
            const int un = sl + SP * j;
            if (un < U) {
                const uint4* xu = reinterpret_cast<const uint4*>(xs + ((int64_t)i * U + un) * kXU);
                const float sx = kAffine<MODE> ? xsum[i * U + un] : 0.0f;
                pg += unit_dot<MODE, UPL>(ug, j, xu, sx, a.scale_f16);
                if (gated) pu += unit_dot<MODE, UPL>(uu, j, xu, sx, a.scale_f16);
            }
        }
        pg = group_sum(pg, SP);
        if (gated) pu = group_sum(pu, SP);
        if (sl == 0 && r0 + rr < inter) {
            const float h = slot == kAbsentCode ? absent_nan() : act_apply(a.act, pg + bg, pu + bu, a.alpha, a.limit);
            hbuf[(int64_t)pair * hstride + r0 + rr] = (uint16_t)f2bf(h);
        }
    }
}

// k_dec_downT: block b takes entry b / nrb and down rows (b % nrb) RB .. of it: each pair's row
// result plus the projection's bias, rounded to bf16, into y_routed at the pair's row (the
// shared expert's into y_shared at its token); the k-ordered combine follows in its own launch.
// One round trip reads the entry, then the weights and the entry's h rows are requested together.
template <int MODE, int UPL>
__global__ __launch_bounds__(kThreads) void k_dec_downT(FwdArgs a, const uint16_t* __restrict__ hbuf, int hstride,
                                                        const DecTable* __restrict__ table, int lsp, int nrb,
                                                        uint16_t* __restrict__ y_routed,
                                                        uint16_t* __restrict__ y_shared) {
    prefetch_args(a);
    __builtin_amdgcn_s_setprio(2);
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ int32_t s_pair[kMaxTok];
    const int SP = 1 << lsp;
    const int lane = threadIdx.x & 63, tid = threadIdx.x;
    const int H = a.H;
    int u, t0, nt;
    int eslot, epair;
    const int rb = entry_group(table, blockIdx.x, nrb, u, t0, nt, eslot, epair);
    if (rb < 0) return;   // uniform
    const int slot = clamp_code(a, eslot);
    const int PT = a.P + (a.auto_shared ? a.T : 0);
    const Layout& L = slot == -1 ? a.lay_sh : a.lay;
    const int K = L.p[2].n_in, U = K / 64;
    const int RW = kWave >> lsp;
    const int r0 = rb * kWaves * RW;
    if (r0 >= H) return;   // uniform
    const uint8_t* base = code_base(a, slot);
    const int g = lane >> lsp, sl = lane & (SP - 1);
    const int rr = (tid >> 6) * RW + g;
    const int row = min(r0 + rr, H - 1);
    Units<MODE, UPL> ud;
    units_load<MODE, UPL>(base, L.p[2], row, sl, SP, a.gshift, ud);
    const float bd = L.p[2].bias >= 0 ? bf2f(reinterpret_cast<const uint16_t*>(base + L.p[2].bias)[row]) : 0.f;
    if (tid < nt) s_pair[tid] = min(max(epair, 0), PT - 1);
    __syncthreads();
    // h rows are staged at their full width (hstride / 64 units); the entry reads its U
    const int Us = hstride / 64;
    uint8_t* hs = lds;
    float* hsum = reinterpret_cast<float*>(lds + (size_t)kPlanTok * Us * kXU);
    stage_dense<MODE>(hbuf, hstride, nt, [&](int i) { return s_pair[i]; }, hs, hsum);
    __syncthreads();
    __builtin_amdgcn_s_setprio(0);
    for (int i = 0; i < nt; ++i) {
        const int pair = s_pair[i];
        float p = 0.f;
#pragma unroll
        for (int j = 0; j < UPL; ++j) {
            const int un = sl + SP * j;
            if (un < U) {
                const uint4* hu = reinterpret_cast<const uint4*>(hs + ((int64_t)i * Us + un) * kXU);
                const float sx = kAffine<MODE> ? hsum[i * Us + un] : 0.0f;
                p += unit_dot<MODE, UPL>(ud, j, hu, sx, a.scale_f16);
            }
        }
        p = group_sum(p, SP);
        if (sl == 0 && r0 + rr < H) {
            const uint16_t y = (uint16_t)f2bf(p + bd);
            if (pair < a.P) y_routed[(int64_t)pair_row(a, pair) * H + r0 + rr] = y;
            else if (y_shared) y_shared[(int64_t)(pair - a.P) * H + r0 + rr] = y;
        }
    }
}

// ------------------------------------------------------------------ down + combine
// Each pair's row result rounded to bf16 (the projection's output, with its bias), the
// unreduced rows when asked for, and the k-ordered combine out[t] = sum_j w[t,j] * y[t,j]
// (+ the gated shared expert): the rows [n0, n0 + RBD) of every pair, ys [PT][RBD] in LDS.
__device__ __forceinline__ void dec_down_epilogue(const FwdArgs& a, float* ys, int RBD, int lrbd, int n0) {
    const int tid = threadIdx.x;
    const int P = a.P;
    const int PT = P + (a.auto_shared ? a.T : 0);
    const int H = a.H;
    for (int it = tid; it < PT * RBD; it += kThreads) {
        int p = it >> lrbd, rr = it & (RBD - 1);
        int nn = n0 + rr;
        if (nn >= H) continue;
        float y = ys[it];
        if (a.has_bias) {
            int e = p < P ? min(max(a.pexp[p], 0), a.shared ? a.E : a.E - 1) : a.E;
            int s = -1;
            if (e < a.E) s = slot_code(a, e, a.g2s[e]);
            const Layout& L = s == -1 ? a.lay_sh : a.lay;
            y += bf2f(reinterpret_cast<const uint16_t*>(code_base(a, s) + L.p[2].bias)[nn]);
        }
        uint32_t yb = f2bf(y);
        ys[it] = bf2f(yb);
        if (a.yun && p < P) a.yun[(int64_t)pair_row(a, p) * H + nn] = (uint16_t)yb;
    }
    __syncthreads();

    if (a.out) {
        for (int it = tid; it < a.T * RBD; it += kThreads) {
            int t = it >> lrbd, rr = it & (RBD - 1);
            if (n0 + rr >= H) continue;
            float acc = 0.0f;
            for (int j = 0; j < a.k; ++j)
                acc = fmaf(a.w[t * a.k + j], ys[(t * a.k + j) * RBD + rr], acc);
            if (a.auto_shared && a.sgate) acc = fmaf(a.sgate[t], ys[(P + t) * RBD + rr], acc);
            a.out[(int64_t)t * H + n0 + rr] = (uint16_t)f2bf(acc);
        }
    }
}


// Items (entry u, row r) of the block's RBD rows: wave w, row group g takes item
// (pass * 4 + w) * RW + g. The h rows of a batch of entries are staged in LDS first.
template <int MODE, int UPL>
__global__ __launch_bounds__(kThreads) void k_dec_down(FwdArgs a, const uint16_t* __restrict__ hbuf,
                                                       int RBD, int hstride,
                                                       const DecTable* __restrict__ table, int lsp,
                                                       int lrbd, int hs_bytes) {
    prefetch_args(a);
    const int SP = 1 << lsp;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int P = a.P;
    const int PT = P + (a.auto_shared ? a.T : 0);
    const int Imax = a.I > a.I_sh ? a.I : a.I_sh;
    const int n0 = blockIdx.x * RBD;
    const int H = a.H;
    const int n = table->n;
    __shared__ int32_t s_pair[kMaxU + kMaxTok];
    __shared__ int32_t s_first[kMaxU + 1], s_nt[kMaxU + 1], s_slot[kMaxU + 1];
    float* ys = reinterpret_cast<float*>(lds);                         // [PT][RBD]
    uint8_t* hs = lds + (((size_t)PT * RBD * 4 + 15) & ~(size_t)15);  // staged h
    const int RW = kWave >> lsp;
    const int g = lane >> lsp, sl = lane & (SP - 1);
    const int Umax = Imax / 64;

    // the table in one parallel read: wave 0 takes the entries' pair counts and slots and scans
    // the counts (s_first[u] = staged row of entry u's first pair); every thread holds up to
    // three (entry, i) pair ids until the scan is known, then files them as s_pair[row]
    // Every read of the table is issued at once and masked by n afterwards (all indices are in
    // bounds of the table whatever n is), together with this row group's first item's slot and,
    // when every pair's h row fits in LDS, the h rows themselves (staged row = pair id): one
    // round trip. The first item's weights are then requested before the scan and the barriers.
    constexpr int kQ = (kMaxU * kMaxTok + kThreads - 1) / kThreads;
    int qp[kQ];
#pragma unroll
    for (int z = 0; z < kQ; ++z) {
        const int q = min(tid + kThreads * z, kMaxU * kMaxTok - 1);
        qp[z] = table->ent[q / kMaxTok].pair[q % kMaxTok];
    }
    int nt0 = 0, sl0 = 0, nt64 = 0, sl64 = 0;
    if (tid < kWave) {
        nt0 = table->ent[tid].nt;
        sl0 = table->ent[tid].slot;
        nt64 = table->ent[kWave].nt;
        sl64 = table->ent[kWave].slot;
    }
    const int it_first = (tid >> 6) * RW + g;
    const int slot_first = table->ent[min(it_first >> lrbd, kMaxU - 1)].slot;
    const bool all_fit = (size_t)PT * Umax * (kXU + 4) <= (size_t)hs_bytes;
    float* hsum_all = reinterpret_cast<float*>(hs + (size_t)PT * Umax * kXU);
    if (all_fit) stage_dense<MODE>(hbuf, hstride, PT, [](int i) { return i; }, hs, hsum_all);
    Units<MODE, UPL> ud;
    const bool have_first = all_fit;
    if (have_first) {
        // an item past the last entry reads a stale table slot: point it at slot 0 instead
        int sf = (it_first >> lrbd) < n ? slot_first : 0;
        sf = clamp_code(a, sf);
        const Layout& L = sf == -1 ? a.lay_sh : a.lay;
        units_load<MODE, UPL>(code_base(a, sf), L.p[2], min(n0 + (it_first & (RBD - 1)), H - 1), sl, SP, a.gshift, ud);
    }
    if (tid < kWave) {
        nt0 = tid < n ? nt0 : 0;
        sl0 = tid < n ? sl0 : 0;
        const bool has64 = n > kWave;
        nt64 = has64 ? nt64 : 0;
        sl64 = has64 ? sl64 : 0;
        const int inc = wave_incl_scan(nt0);
        const int tot0 = __builtin_amdgcn_readlane(inc, kWave - 1);
        s_first[tid] = inc - nt0;
        s_nt[tid] = nt0;
        s_slot[tid] = sl0;
        if (tid == 0) {   // entry 64 exists only with 64 routed pairs and the shared expert
            s_first[kWave] = tot0;
            s_nt[kWave] = nt64;
            s_slot[kWave] = sl64;
            s_first[kWave + 1] = tot0 + nt64;
        }
    }
    __syncthreads();
#pragma unroll
    for (int z = 0; z < kQ; ++z) {
        const int q = tid + kThreads * z;
        const int u = q / kMaxTok, i = q - u * kMaxTok;
        if (q < n * kMaxTok && i < s_nt[u]) s_pair[s_first[u] + i] = qp[z];
    }
    __syncthreads();

    int u0 = 0;
    while (u0 < n) {
        // the entries [u0, u1) whose pairs fit the staging budget (at least one entry)
        int u1 = all_fit ? n : u0 + 1;
        while (u1 < n && (size_t)(s_first[u1 + 1] - s_first[u0]) * Umax * (kXU + 4) <= (size_t)hs_bytes) ++u1;
        const int rows = s_first[u1] - s_first[u0];
        const int row0 = s_first[u0];
        const int items = (u1 - u0) * RBD;
        // this row group's item of the first pass: its weights are requested before the h rows
        // are staged, so the two fetches overlap (already in flight when every row fits)
        int it = (tid >> 6) * RW + g;
        bool valid = it < items;
        int iu = valid ? it >> lrbd : 0;
        int r = valid ? it & (RBD - 1) : 0;
        if (!have_first) {
            const int slot = s_slot[u0 + iu];
            const Layout& L = slot == -1 ? a.lay_sh : a.lay;
            units_load<MODE, UPL>(code_base(a, slot), L.p[2], min(n0 + r, H - 1), sl, SP, a.gshift, ud);
        }
        float* hsum = all_fit ? hsum_all : reinterpret_cast<float*>(hs + (size_t)rows * Umax * kXU);
        if (!all_fit) {
            stage_dense<MODE>(hbuf, hstride, rows, [&](int i) { return s_pair[row0 + i]; }, hs, hsum);
            __syncthreads();
        }
        for (int it0 = 0; it0 < items; it0 += kWaves * RW) {
            if (it0 > 0) {
                it = it0 + (tid >> 6) * RW + g;
                valid = it < items;
                iu = valid ? it >> lrbd : 0;
                r = valid ? it & (RBD - 1) : 0;
                const int slot = s_slot[u0 + iu];
                const Layout& L = slot == -1 ? a.lay_sh : a.lay;
                units_load<MODE, UPL>(code_base(a, slot), L.p[2], min(n0 + r, H - 1), sl, SP, a.gshift, ud);
            }
            const int u = u0 + iu;
            const int slot = s_slot[u];
            const int nt = valid ? s_nt[u] : 0;
            const int U = (slot == -1 ? a.lay_sh : a.lay).p[2].n_in / 64;
            const int srow = s_first[u] - row0;   // staged row of the item's first pair (batched)
            // the SP lanes of one item share nt; lanes past the items have nt = 0 and only take
            // part in the shuffles
            int ntg = nt;
            ntg = group_max(ntg, SP);
            for (int i = 0; i < ntg; ++i) {
                float p = 0.0f;
#pragma unroll
                for (int j = 0; j < UPL; ++j) {
                    const int un = sl + SP * j;
                    if (i < nt && un < U) {
                        const int hr = all_fit ? s_pair[s_first[u] + i] : srow + i;
                        const uint4* hu = reinterpret_cast<const uint4*>(hs + ((int64_t)hr * Umax + un) * kXU);
                        const float sx = kAffine<MODE> ? hsum[hr * Umax + un] : 0.0f;
                        p += unit_dot<MODE, UPL>(ud, j, hu, sx, a.scale_f16);
                    }
                }
                p = group_sum(p, SP);
                if (valid && sl == 0 && i < nt && n0 + r < H) ys[s_pair[s_first[u] + i] * RBD + r] = p;
            }
        }
        __syncthreads();
        u0 = u1;
    }

    dec_down_epilogue(a, ys, RBD, lrbd, n0);
}

// The down kernel when the h rows of every pair fit in LDS (every decode step of the shipped
// shapes): each row group reads its item's table row itself, the h rows are staged by pair id,
// and the item's weights are requested as soon as its slot is known -- two memory round trips
// in all, no scan and one barrier before the dot products.
template <int MODE, int UPL, int NT>
__global__ __launch_bounds__(kThreads) void k_dec_down_fit(FwdArgs a, const uint16_t* __restrict__ hbuf,
                                                           int RBD, int hstride,
                                                           const DecTable* __restrict__ table, int lsp,
                                                           int lrbd, int nu) {
    prefetch_args(a);
    __builtin_amdgcn_s_setprio(2);
    const int SP = 1 << lsp;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int P = a.P;
    const int PT = P + (a.auto_shared ? a.T : 0);
    const int Imax = a.I > a.I_sh ? a.I : a.I_sh;
    const int Umax = Imax / 64;
    const int n0 = blockIdx.x * RBD;
    const int H = a.H;
    float* ys = reinterpret_cast<float*>(lds);                         // [PT][RBD]
    uint8_t* hs = lds + (((size_t)PT * RBD * 4 + 15) & ~(size_t)15);  // [PT][Umax] units
    float* hsum = reinterpret_cast<float*>(hs + (size_t)PT * Umax * kXU);
    const int RW = kWave >> lsp;
    const int g = lane >> lsp, sl = lane & (SP - 1);
    const int items = nu * RBD;

    // every pair's h rows: the first pass requested with the first items' table rows, stored to
    // LDS once those items' weights are requested
    auto ident = [](int i) { return i; };
    DenseRegs<kStageB> hrows;
    dense_issue<kStageB>(hbuf, hstride, PT, ident, 0, hrows);
    // the pass body; the first pass runs outside the loop, as straight-line code after the h
    // loads, so nothing copies (and so waits for) the h registers before the weights are
    // requested
    auto pass = [&](int it0, bool first) __attribute__((always_inline)) {
        const int it = it0 + (tid >> 6) * RW + g;
        const bool in_range = it < items;
        const int u = min(it >> lrbd, nu - 1);
        const int r = it & (RBD - 1);
        // the item's table row: header and pair ids, three 16-byte loads
        const uint4* ep = reinterpret_cast<const uint4*>(&table->ent[u]);
        const uint4 hd = ep[0], p0 = ep[1], p1 = ep[2];
        const int nt = in_range ? (int)hd.y : 0;
        int slot = nt > 0 ? (int)hd.x : 0;
        slot = clamp_code(a, slot);
        const Layout& L = slot == -1 ? a.lay_sh : a.lay;
        const int U = L.p[2].n_in / 64;
        Units<MODE, UPL> ud;
        units_load<MODE, UPL>(code_base(a, slot), L.p[2], min(n0 + r, H - 1), sl, SP, a.gshift, ud);
        if (first) {
            // (an empty asm on the loaded registers keeps the store's arithmetic here, after the
            // weight requests, rather than hoisted next to the loads)
#pragma unroll
            for (int q = 0; q < kStageB; ++q)
                asm volatile("" : "+v"(hrows.v[q].x), "+v"(hrows.v[q].y), "+v"(hrows.v[q].z),
                             "+v"(hrows.v[q].w));
            dense_store<MODE, kStageB>(hstride, PT, 0, hrows, hs, hsum);
            stage_dense<MODE>(hbuf, hstride, PT, ident, hs, hsum, kStageB * kThreads);
            __syncthreads();
            __builtin_amdgcn_s_setprio(0);
        }
        const int pr[kMaxTok] = {(int)p0.x, (int)p0.y, (int)p0.z, (int)p0.w,
                                 (int)p1.x, (int)p1.y, (int)p1.z, (int)p1.w};
        // the SP lanes of one item share nt; lanes past the items have nt = 0 and only take
        // part in the sums
        int ntg = nt;
        ntg = group_max(ntg, SP);
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            if (i >= ntg) break;
            const int hr = min(max(pr[i], 0), PT - 1);
            float p = 0.0f;
#pragma unroll
            for (int j = 0; j < UPL; ++j) {
                const int un = sl + SP * j;
                if constexpr (NT == 1) {
                    // one pair: each piece's h read sits under the pair test, so the unit's
                    // reads are not all hoisted ahead of its dots (fewer registers, more waves)
                    if (un < U) {
                        const uint4* hu = reinterpret_cast<const uint4*>(hs + ((int64_t)hr * Umax + un) * kXU);
                        float lo = 0.0f, hi = 0.0f;
#pragma unroll
                        for (int m = 0; m < 8; ++m) {
                            uint32_t q[4];
                            piece_ops<MODE, UPL>(ud, j, m, q);
                            if (i < nt) {
                                if (kTwoGroups<MODE> && m >= 4) hi = piece_dot(q, hu[m], hi);
                                else lo = piece_dot(q, hu[m], lo);
                            }
                        }
                        if (i < nt) {
                            const float sx = kAffine<MODE> ? hsum[hr * Umax + un] : 0.0f;
                            p += unit_value<MODE, UPL>(ud, j, lo, hi, sx, a.scale_f16);
                        }
                    }
                } else if (i < nt && un < U) {
                    const uint4* hu = reinterpret_cast<const uint4*>(hs + ((int64_t)hr * Umax + un) * kXU);
                    const float sx = kAffine<MODE> ? hsum[hr * Umax + un] : 0.0f;
                    p += unit_dot<MODE, UPL>(ud, j, hu, sx, a.scale_f16);
                }
            }
            p = group_sum(p, SP);
            if (sl == 0 && i < nt && n0 + r < H) ys[hr * RBD + r] = p;
        }
    };
    pass(0, true);
    for (int it0 = kWaves * RW; it0 < items; it0 += kWaves * RW) {
        if (it0 >= table->n * RBD) break;   // passes past the step's entries: no work
        pass(it0, false);
    }
    __syncthreads();
    dec_down_epilogue(a, ys, RBD, lrbd, n0);
}

// (SP, UPL) for a row of U units: the fewest lane slots SP * UPL >= U, then the units per lane
// nearest `pref` (UPL <= max_upl, SP a power of two <= 64).
void pick_split(int U, int pref, int& SP, int& UPL, int max_upl = 4) {
    int best = 1 << 30, bestd = 1 << 30;
    SP = 64;
    UPL = 1;
    for (int sp = 1; sp <= 64; sp <<= 1)
        for (int upl = 1; upl <= max_upl; ++upl) {
            if (sp * upl < U) continue;
            const int cost = sp * upl, dist = upl > pref ? upl - pref : pref - upl;
            if (cost < best || (cost == best && dist < bestd)) { best = cost; bestd = dist; SP = sp; UPL = upl; }
        }
}

template <int MODE, int UPL>
hipError_t launch_gateup(const FwdArgs& a, uint16_t* hbuf, DecTable* table, int nu, int Imax, int SP,
                         hipStream_t s) {
    const int RB = kWaves * (kWave / SP);
    // entry rows: one per block row up to 16; past that (several tokens, where most of the
    // P + 1 possible entries are empty) a block takes entries y, y + 16, ...
    dim3 grid((Imax + RB - 1) / RB, a.T > 1 && nu > kEntryRows ? kEntryRows : nu), block(kThreads);
    // staged x of up to T tokens
    const size_t lds = (size_t)a.T * (a.H / 64) * (kXU + 4);
    const int lsp = __builtin_ctz(SP);
#define BRX_GU(KP)                                                                                     \
    do {                                                                                               \
        if (a.T > 1)                                                                                   \
            hipLaunchKernelGGL((k_dec_gateup<MODE, UPL, KP, true>), grid, block, lds, s, a, hbuf, Imax, table, lsp, nu, (int)grid.y); \
        else                                                                                           \
            hipLaunchKernelGGL((k_dec_gateup<MODE, UPL, KP, false>), grid, block, lds, s, a, hbuf, Imax, table, lsp, nu, (int)grid.y); \
    } while (0)
    if (!a.logits) BRX_GU(0);
    else if (a.E <= 64) BRX_GU(1);
    else if (a.E <= 128) BRX_GU(2);
    else if (a.E <= 256) BRX_GU(4);
    else BRX_GU(8);
#undef BRX_GU
    return hipGetLastError();
}

// One token (token mode): one (entry, row) item per row group.
template <int MODE, int UPL>
hipError_t launch_gateup1(const FwdArgs& a, uint16_t* hbuf, DecTable* table, int nu, int Imax, int SP,
                          hipStream_t s) {
    const int RGn = kWaves * (kWave / SP);
    const int nblk = (nu * Imax + RGn - 1) / RGn;
    const size_t lds = (size_t)(a.H / 64) * (kXU + 4);
    const int lsp = __builtin_ctz(SP);
#define BRX_G1(KP) hipLaunchKernelGGL((k_dec_gateup1<MODE, UPL, KP>), dim3(nblk), dim3(kThreads), lds, s, a, hbuf, \
                                      Imax, table, lsp, nu)
    if (!a.logits) BRX_G1(0);
    else if (a.E <= 64) BRX_G1(1);
    else if (a.E <= 128) BRX_G1(2);
    else BRX_G1(4);
#undef BRX_G1
    return hipGetLastError();
}

// Block rows of the per-entry kernels: every entry the step may have, plus the shared expert's
// token groups past its first.
inline int entry_groups(const FwdArgs& a, int nu) {
    return nu + (a.auto_shared ? (a.T - 1) / kPlanTok : 0);
}

// Several tokens: the plan (one block), then one block per (entry, RB rows) for every entry
// the step may have (P routed pairs + the shared expert); blocks past the planned entries return.
template <int MODE, int UPL>
hipError_t launch_gateupT(const FwdArgs& a, uint16_t* hbuf, DecTable* table, int nu, int Imax, int SP,
                          hipStream_t s) {
#define BRX_PLAN(KP) hipLaunchKernelGGL((k_dec_plan<KP>), dim3(1), dim3(kPlanThreads), 0, s, a, table)
    if (!a.logits) BRX_PLAN(0);
    else if (a.E <= 64) BRX_PLAN(1);
    else if (a.E <= 128) BRX_PLAN(2);
    else if (a.E <= 256) BRX_PLAN(4);
    else BRX_PLAN(8);
#undef BRX_PLAN
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    const int RB = kWaves * (kWave / SP);
    const int nrb = (Imax + RB - 1) / RB;
    const size_t lds = (size_t)kPlanTok * (a.H / 64) * (kXU + 4);
    hipLaunchKernelGGL((k_dec_gateupT<MODE, UPL>), dim3(entry_groups(a, nu) * nrb), dim3(kThreads), lds, s, a, hbuf, Imax, table,
                       (int)__builtin_ctz(SP), nrb);
    return hipGetLastError();
}

// Several tokens, down: one block per (entry, RB rows), then the k-ordered combine.
template <int MODE, int UPL>
hipError_t launch_downT(const FwdArgs& a, uint16_t* hbuf, DecTable* table, int nu, int Imax, int SP,
                        uint16_t* y_routed, uint16_t* y_shared, hipStream_t s) {
    const int RB = kWaves * (kWave / SP);
    const int nrb = (a.H + RB - 1) / RB;
    const size_t lds = (size_t)kPlanTok * (Imax / 64) * (kXU + 4);
    hipLaunchKernelGGL((k_dec_downT<MODE, UPL>), dim3(entry_groups(a, nu) * nrb), dim3(kThreads), lds, s, a, hbuf, Imax, table,
                       (int)__builtin_ctz(SP), nrb, y_routed, y_shared);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess || !a.out) return err;
    return launch_combine(y_routed, a.auto_shared ? y_shared : nullptr, a.w, a.sgate, a.T, a.k, a.H, a.out, s);
}

template <int MODE, int UPL>
hipError_t launch_down(const FwdArgs& a, uint16_t* hbuf, DecTable* table, int nu, int PT, int Imax, int SP,
                       bool one_pair, hipStream_t s) {
    // rows per block: enough (entry, row) items to give every row group of the 4 waves one
    const int per_pass = kWaves * (kWave / SP);
    int RBD = 1;
    while (RBD < 64 && nu * RBD * 2 <= per_pass && a.H % (RBD * 2) == 0) RBD *= 2;
    // every block stages the h rows of every pair: when they are many (several tokens), give
    // each block at least H / 256 output rows so the staging is shared by enough of them
    if ((size_t)PT * Imax * 2 > 32 * 1024)
        while (RBD < 64 && RBD * 256 < a.H && a.H % (RBD * 2) == 0) RBD *= 2;
    const int Umax = Imax / 64;
    const size_t need = (size_t)PT * Umax * (kXU + 4);
    const int hs_bytes = (int)(need < (size_t)kDownLds ? need : (size_t)kDownLds);
    const size_t ys_b = (((size_t)PT * RBD * 4) + 15) & ~(size_t)15;
    const size_t lds = ys_b + (size_t)hs_bytes + 16;
    if (need <= (size_t)kDownLds)
        // (at most NT pairs an entry: one after the one-token gate/up kernel, whose entries are
        // single pairs; the one-pair form holds fewer registers)
        if (one_pair)
            hipLaunchKernelGGL((k_dec_down_fit<MODE, UPL, 1>), dim3((a.H + RBD - 1) / RBD), dim3(kThreads), lds, s,
                               a, hbuf, RBD, Imax, table, __builtin_ctz(SP), __builtin_ctz(RBD), nu);
        else
            hipLaunchKernelGGL((k_dec_down_fit<MODE, UPL, kMaxTok>), dim3((a.H + RBD - 1) / RBD), dim3(kThreads),
                               lds, s, a, hbuf, RBD, Imax, table, __builtin_ctz(SP), __builtin_ctz(RBD), nu);
    else
        hipLaunchKernelGGL((k_dec_down<MODE, UPL>), dim3((a.H + RBD - 1) / RBD), dim3(kThreads), lds, s, a, hbuf,
                           RBD, Imax, table, __builtin_ctz(SP), __builtin_ctz(RBD), hs_bytes);
    return hipGetLastError();
}

// Units per lane a mode's kernels are built for: a bf16 unit is 128 bytes (32 registers), so
// unquantized rows take at most two units a lane (SP up to 64 covers widths up to 8192).
template <int MODE>
constexpr int kMaxUpl = MODE == kModeBf16 ? 2 : 4;

#define BRX_UPL_CASES(FN, ...)                                                   \
    do {                                                                         \
        if (upl_ == 1) return FN<MODE, 1>(__VA_ARGS__);                          \
        if constexpr (kMaxUpl<MODE> == 2) {                                      \
            return FN<MODE, 2>(__VA_ARGS__);                                     \
        } else {                                                                 \
            if (upl_ == 2) return FN<MODE, 2>(__VA_ARGS__);                      \
            if (upl_ == 3) return FN<MODE, 3>(__VA_ARGS__);                      \
            return FN<MODE, 4>(__VA_ARGS__);                                     \
        }                                                                        \
    } while (0)

template <int MODE>
hipError_t launch_mode(const FwdArgs& a, uint16_t* hbuf, DecTable* table, uint16_t* y_routed,
                       uint16_t* y_shared, int phases, hipStream_t s) {
    const int P = a.P;
    const int PT = P + (a.auto_shared ? a.T : 0);
    const int nu = P + (a.auto_shared ? 1 : 0);
    const int Imax = a.I > a.I_sh ? a.I : a.I_sh;
    // Several tokens with more possible entries than the one-launch kernel's 16 block rows take
    // in two passes: the plan launch, then one block per (entry, rows). With fewer, every
    // gate/up block ranks and plans the step itself.
    const bool per_entry = a.T > 1 && nu > 2 * kEntryRows;
    // one token: one unit per lane where the row allows it (twice the waves of two units per
    // lane, each with half the dequant-dot work and far fewer registers: 11.1 -> 10.2 us per
    // layer on H = 2048); several tokens: two units per lane, half the blocks, each staging
    // x once for twice the rows. The split fixes each row's summation order, so both
    // several-token kernels take the same one: a step's rows do not depend on how many
    // pairs share its launch (a pool's span calls against the whole step).
    int SPg, uplg;
    pick_split(a.H / 64, a.T > 1 && kMaxUpl<MODE> > 2 ? 2 : 1, SPg, uplg, kMaxUpl<MODE>);
    // the one-token gate/up kernel makes every pair its own entry (pairs given by the caller may
    // repeat an expert, which the other kernels merge into one entry)
    const bool one_token = a.T == 1 && !a.ptok && uplg <= 3 && a.E <= 256 && nu <= kWave;
    if (phases & 1) {
        const int SP = SPg, upl_ = uplg;
        hipError_t err;
        if (one_token) {
            if constexpr (kMaxUpl<MODE> == 2)
                err = upl_ == 1 ? launch_gateup1<MODE, 1>(a, hbuf, table, nu, Imax, SP, s)
                                : launch_gateup1<MODE, 2>(a, hbuf, table, nu, Imax, SP, s);
            else
                err = upl_ == 1   ? launch_gateup1<MODE, 1>(a, hbuf, table, nu, Imax, SP, s)
                      : upl_ == 2 ? launch_gateup1<MODE, 2>(a, hbuf, table, nu, Imax, SP, s)
                                  : launch_gateup1<MODE, 3>(a, hbuf, table, nu, Imax, SP, s);
        } else if (per_entry) {
            err = [&]() -> hipError_t { BRX_UPL_CASES(launch_gateupT, a, hbuf, table, nu, Imax, SP, s); }();
        } else {
            err = [&]() -> hipError_t { BRX_UPL_CASES(launch_gateup, a, hbuf, table, nu, Imax, SP, s); }();
        }
        if (err != hipSuccess) return err;
    }
    if (phases & 2) {
        int SP, upl_;
        hipError_t err;
        // (the same split for both down kernels, as for gate/up)
        pick_split(Imax / 64, kMaxUpl<MODE> > 2 ? 3 : 1, SP, upl_, kMaxUpl<MODE>);
        // several tokens whose h rows are too many for every block to stage them all: one block
        // per (entry, rows), then the combine; otherwise every block stages every pair's h rows
        // and combines in its epilogue
        if (per_entry && (size_t)PT * Imax * 2 > 32 * 1024) {
            uint16_t* yr = a.yun ? a.yun : y_routed;
            err = [&]() -> hipError_t { BRX_UPL_CASES(launch_downT, a, hbuf, table, nu, Imax, SP, yr, y_shared, s); }();
        } else {
            err = [&]() -> hipError_t { BRX_UPL_CASES(launch_down, a, hbuf, table, nu, PT, Imax, SP, one_token, s); }();
        }
        if (err != hipSuccess) return err;
    }
    return hipSuccess;
}

inline size_t table_bytes() { return (sizeof(DecTable) + 255) & ~(size_t)255; }

// [table][h rows: PT x Imax bf16] and, for several tokens, [y rows: P x H][shared y rows: T x H]
struct DecWs {
    DecTable* table;
    uint16_t* hbuf;
    uint16_t* y_routed;
    uint16_t* y_shared;
    size_t bytes;
};

inline DecWs dec_carve(const FwdArgs& a, void* ws) {
    const int PT = a.P + (a.auto_shared ? a.T : 0);
    const int Imax = a.I > a.I_sh ? a.I : a.I_sh;
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    char* b = reinterpret_cast<char*>(ws);
    DecWs w{};
    size_t off = 0;
    w.table = reinterpret_cast<DecTable*>(b + off); off += table_bytes();
    w.hbuf = reinterpret_cast<uint16_t*>(b + off); off = al(off + (size_t)PT * Imax * 2);
    if (a.T > 1) {
        w.y_routed = reinterpret_cast<uint16_t*>(b + off); off = al(off + (size_t)a.P * a.H * 2);
        w.y_shared = reinterpret_cast<uint16_t*>(b + off); off = al(off + (size_t)a.T * a.H * 2);
    }
    w.bytes = off;
    return w;
}

}  // namespace
}  // namespace brx
