// Internal declarations of libbrx: expert layout arithmetic, device helpers, kernel launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "brx.h"

namespace brx {

constexpr int kWave = 64;
constexpr int kMaxTableEdits = 32;   // table entries one brx_pool_publish_async launch sets
constexpr int kMaxWidth = 8192;      // largest hidden / intermediate width the kernels take

// Kernel weight modes: MXFP4, and one mode per affine code width (4-bit affine keeps the public
// BRX_QUANT_AFFINE value). Every affine width stores a row as one continuous stream of codes,
// least significant bits first (code k at bits [bits k, bits k + bits) of the row's bytes), so
// 64 codes -- a decode unit, a 64-K prefill stage -- are 8 * bits bytes, and a run of 8 codes
// (a "piece") is `bits` bytes. Scale groups hold 64 or 128 codes (gshift 0 or 1).
constexpr int kModeAffine4 = BRX_QUANT_AFFINE;
constexpr int kModeAffine3 = 2;
constexpr int kModeAffine2 = 3;
constexpr int kModeAffine6 = 4;
constexpr int kModeAffine8 = 5;
constexpr int kModeBf16 = 6;           // unquantized bf16 weights (BRX_QUANT_NONE)
template <int MODE>
constexpr bool kAffine = MODE != BRX_QUANT_MXFP4 && MODE != kModeBf16;   // scale + bias per group
template <int MODE>
constexpr bool kScaled = MODE != kModeBf16;                           // any per-group scales
template <int MODE>
constexpr int kBits = MODE == kModeAffine2 ? 2 : MODE == kModeAffine3 ? 3 : MODE == kModeAffine6 ? 6
                    : MODE == kModeAffine8 ? 8 : MODE == kModeBf16 ? 16 : 4;

// The kernel mode of a descriptor's quantization (-1: none takes it).
inline int kernel_mode(int quant_mode, int bits) {
    if (quant_mode == BRX_QUANT_MXFP4) return bits == 4 ? BRX_QUANT_MXFP4 : -1;
    if (quant_mode == BRX_QUANT_NONE) return bits == 16 ? kModeBf16 : -1;
    switch (bits) {
        case 2: return kModeAffine2;
        case 3: return kModeAffine3;
        case 4: return kModeAffine4;
        case 6: return kModeAffine6;
        case 8: return kModeAffine8;
        default: return -1;
    }
}

// Codes i and i + 4 of a 3-byte group in the low bits of the two 16-bit halves.
__device__ __forceinline__ uint32_t pair3(uint32_t g, int i) {
    const uint32_t t = g >> (3 * i);
    return (t & 0x7u) | ((t << 4) & 0x70000u);
}

// Codes 8m + i (low 16 bits) and 8m + i + 4 (high 16 bits) of piece m of a run of little-endian
// words `w` holding whole pieces of BITS-bit codes (i < 4; m and i compile-time after
// unrolling). Two codes a 32-bit value, so one AND/OR turns both into operands.
__device__ __forceinline__ uint32_t bits_at(const uint32_t* w, int b, int n) {
    // n <= 24 bits starting at bit b of `w` (in the low bits; the rest is garbage)
    const int wi = b >> 5, sh = b & 31;
    return sh + n <= 32 ? w[wi] >> sh : __builtin_amdgcn_alignbit(w[wi + 1], w[wi], sh);
}
template <int BITS>
__device__ __forceinline__ uint32_t piece_pair(const uint32_t* w, int m, int i) {
    if constexpr (BITS == 4) {
        return (w[m] >> (4 * i)) & 0x000F000Fu;
    } else if constexpr (BITS == 3) {
        return pair3(bits_at(w, 24 * m, 24), i);
    } else if constexpr (BITS == 2) {
        // the piece is 16 bits: its low byte holds codes 0..3, its high byte codes 4..7
        const uint32_t v = w[m >> 1] >> (16 * (m & 1));
        const uint32_t sp = (v & 0xFFu) | ((v & 0xFF00u) << 8);
        return (sp >> (2 * i)) & 0x00030003u;
    } else if constexpr (BITS == 8) {
        // byte i of each of the piece's two words
        return ((w[2 * m] >> (8 * i)) & 0xFFu) | (((w[2 * m + 1] >> (8 * i)) & 0xFFu) << 16);
    } else {
        static_assert(BITS == 6, "affine widths are 2, 3, 4, 6 and 8 bits");
        // codes 0..3 and 4..7 of the piece as two runs of 24 bits
        const uint32_t lo = bits_at(w, 48 * m, 24), hi = bits_at(w, 48 * m + 24, 24);
        return ((lo >> (6 * i)) & 0x3Fu) | (((hi >> (6 * i)) & 0x3Fu) << 16);
    }
}


// ------------------------------------------------------------------ layout (host + device)
struct Proj {
    int32_t w, s, b, bias;  // byte offsets inside the expert (-1 = absent); widths <= 8192 keep
                            // an expert under 2^31 bytes
    int32_t n_out, n_in;
};

struct Layout {
    Proj p[3];              // gate, up, down
    int64_t bytes;
};

// Offsets in the order stream.pack_experts writes components (weight, scales, biases, bias)
// for projections gate_proj, up_proj, down_proj (bigrig_engine/stream.py:152-164). A plain
// two-layer expert (BRX_ACT_SILU_MLP) packs fc1 then fc2: they take slots 0 and 2 and slot 1
// is absent.
inline Layout make_layout(const brx_layer_desc& d, int inter) {
    Layout L{};
    int64_t pos = 0;
    for (int p = 0; p < 3; ++p) {
        if (p == 1 && d.act == BRX_ACT_SILU_MLP) {
            L.p[1] = Proj{-1, -1, -1, -1, 0, 0};
            continue;
        }
        int n_out = p < 2 ? inter : d.hidden;
        int n_in = p < 2 ? d.hidden : inter;
        int64_t G = d.group_size > 0 ? n_in / d.group_size : 0;
        L.p[p].n_out = n_out;
        L.p[p].n_in = n_in;
        L.p[p].w = (int32_t)pos;
        pos += (int64_t)n_out * n_in * d.bits / 8;
        if (d.quant_mode == BRX_QUANT_NONE) {          // unquantized bf16: the weight alone
            L.p[p].s = L.p[p].b = -1;
        } else if (d.quant_mode == BRX_QUANT_AFFINE) {
            L.p[p].s = (int32_t)pos; pos += (int64_t)n_out * G * 2;
            L.p[p].b = (int32_t)pos; pos += (int64_t)n_out * G * 2;
        } else {
            L.p[p].s = (int32_t)pos; pos += (int64_t)n_out * G;
            L.p[p].b = -1;
        }
        if (d.has_bias) { L.p[p].bias = (int32_t)pos; pos += (int64_t)n_out * 2; }
        else L.p[p].bias = -1;
    }
    L.bytes = pos;
    return L;
}

// Everything a forward kernel needs, passed by value.
struct FwdArgs {
    // pointers first, then the 32-bit fields packed together: the struct is passed by value
    // and kernels whose argument block grows past 512 bytes measured ~0.4 us slower per launch
    const uint16_t* x;          // [T, H] bf16
    const int32_t* pexp;        // [P] expert of each pair (token mode: idx [T, k] flattened)
    const int32_t* ptok;        // [P] token row of each pair, or null: pair / k
    const int32_t* prow;        // [P] row of each pair in yun, or null: the pair index
    const float* w;             // [T, k]
    const float* sgate;         // [T] or null
    const uint8_t* slots;       // pool slot array base
    int64_t slot_stride;        // bytes between slots
    const int32_t* g2s;         // [E]
    const uint8_t* host;        // host backing: expert e at host + e * slot_stride, or null
    const uint8_t* shared;      // shared expert bytes or null (expert id E)
    uint16_t* out;              // [T, H] bf16 or null
    uint16_t* yun;              // [yrows, H] bf16 or null (token mode: [T, k, H])
    // routed in-kernel (decode of a whole MoE block): the gate/up kernel ranks `logits`
    // [T, E + 1] itself and its first block publishes the routing through these, which then
    // alias pexp / w / sgate for the down kernel
    const float* logits;        // or null: routing comes in through pexp / w
    int32_t* route_idx;         // [T, k]
    float* route_w;             // [T, k]
    float* route_sg;            // [T] or null
    int32_t* err;               // the pool's error word {flag, expert} (device), or null
    const float* route_bias;    // sigmoid routing: the selection (score-correction) bias [E] or null
    Layout lay;                 // routed expert layout
    Layout lay_sh;              // shared expert layout
    int32_t P;                  // routed (token, expert) pairs
    int32_t capacity;
    int32_t auto_shared;        // token mode: every token also runs the shared expert
    int32_t T, H, I, I_sh, E, k;
    int32_t quant_mode, scale_f16, has_bias, act;   // quant_mode: a kernel mode (kModeAffine*, MXFP4)
    float alpha, limit;
    int32_t yrows;              // rows of yun
    int8_t route_mode;
    int8_t gshift;              // affine scale groups of 64 << gshift codes (0 or 1)
    uint8_t n_group, topk_group;   // group-limited routing (1, 1: none); at most 64
    float route_scale;          // multiplies every routing weight
};
static_assert(sizeof(FwdArgs) <= 480, "kernel argument blocks must stay under 512 bytes");

// Token row of pair p, and the row its result is written to; explicit lists are clamped so a
// bad entry computes a wrong row rather than reading or writing out of bounds.
__device__ __forceinline__ int pair_tok(const FwdArgs& a, int p) {
    return a.ptok ? min(max(a.ptok[p], 0), a.T - 1) : p / a.k;
}
__device__ __forceinline__ int pair_row(const FwdArgs& a, int p) {
    return a.prow ? min(max(a.prow[p], 0), a.yrows - 1) : p;
}

// Where an expert's bytes are read from, as one int "slot code": 0 <= c < capacity pool slot
// c; c == -1 the shared expert; c <= -2 routed expert -2 - c read straight from the pool's host
// backing (pinned host memory the GPU reads over the bus), which a table entry < 0 selects when
// the pool has one; kAbsentCode an expert that is neither in a slot nor host-backed. An absent
// expert is never computed as if it were another: the pool's error word records it (the host
// reports it as BRX_ERANGE), its bytes are read from the last slot only so every address stays
// in bounds, and the activations of its rows are written as NaN, so every output it touches
// is NaN rather than a plausible wrong value.
constexpr int kAbsentCode = 0x40000000;
__device__ __forceinline__ void note_absent(const FwdArgs& a, int e) {
    if (a.err) {
        a.err[1] = e;
        a.err[0] = 1;
    }
}
__device__ __forceinline__ int slot_code(const FwdArgs& a, int e, int v) {
    if (v >= 0) return min(v, a.capacity - 1);
    return a.host ? -2 - e : kAbsentCode;
}
// A code read back from the library's own tables, clamped into what the arguments allow
// (kAbsentCode stays as it is: code_base keeps its reads in bounds).
__device__ __forceinline__ int clamp_code(const FwdArgs& a, int c) {
    if (c == -1) return a.shared ? -1 : 0;
    if (c < -1) return a.host ? max(c, -1 - a.E) : 0;
    return c == kAbsentCode ? c : min(c, a.capacity - 1);
}
__device__ __forceinline__ const uint8_t* code_base(const FwdArgs& a, int c) {
    if (c >= 0) return a.slots + (int64_t)min(c, a.capacity - 1) * a.slot_stride;
    if (c == -1) return a.shared;
    return a.host + (int64_t)(-2 - c) * a.slot_stride;
}
__device__ __forceinline__ float absent_nan() { return __uint_as_float(0x7fc00000u); }

// ------------------------------------------------------------------ device helpers
__device__ __forceinline__ float bf2f(uint32_t b16) { return __uint_as_float(b16 << 16); }

__device__ __forceinline__ uint32_t f2bf(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

__device__ __forceinline__ float h2f(uint32_t h16) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h16);
}

__device__ __forceinline__ float load_scale(const uint8_t* base, int64_t idx, int scale_f16) {
    uint16_t v = *reinterpret_cast<const uint16_t*>(base + 2 * idx);
    return scale_f16 ? h2f(v) : bf2f(v);
}

// e2m1 code -> fp32 (OCP FP4 E2M1).
__device__ __forceinline__ float e2m1_f32(uint32_t c) {
    uint32_t mag = c & 7u;
    uint32_t e = mag >> 1, m = mag & 1u;
    uint32_t bits = e ? (((126u + e) << 23) | (m << 22)) : (m ? 0x3F000000u : 0u);
    bits |= (c & 8u) << 28;
    return __uint_as_float(bits);
}

// e8m0 -> 2^(e-127) (NaN for 0xFF)
__device__ __forceinline__ float e8m0_f32(uint32_t e) {
    if (e == 255u) return __uint_as_float(0x7fc00000u);
    if (e == 0u) return __uint_as_float(0x00400000u);  // 2^-127, subnormal in fp32
    return __uint_as_float(e << 23);
}

// x * sigmoid(a x) = x / (1 + 2^(-a x log2(e))) with the hardware exp2 and reciprocal
// (v_exp_f32, v_rcp_f32, about 1 ulp each) instead of the library expf and an IEEE division,
// which cost ~40 instructions per element in the GEMM epilogues. For very negative a x the
// exp2 overflows to +inf and the result is x * 0 = -0, the limit.
__device__ __forceinline__ float x_sigmoid(float x, float a) {
    const float e = __builtin_amdgcn_exp2f(-a * x * 1.44269504088896341f);
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ float silu_mul(float g, float u) { return x_sigmoid(g, 1.0f) * u; }

__device__ __forceinline__ float act_apply(int act, float g, float u, float alpha, float limit) {
    if (act == BRX_ACT_SWIGLU) return silu_mul(g, u);
    if (act == BRX_ACT_SILU_MLP) return x_sigmoid(g, 1.0f);
    g = fminf(g, limit);
    u = fminf(fmaxf(u, -limit), limit);
    return x_sigmoid(g, alpha) * (u + 1.0f);
}

// The kernel arguments sit in memory the scalar cache fills on first touch, one 64-byte line
// at a time. Touching every line of a by-value argument struct at kernel entry brings them all
// in one round trip, instead of one round trip at each first use of a field deeper in the kernel.
template <typename T>
__device__ __forceinline__ void prefetch_args(const T& a) {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(&a);
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < (int)(sizeof(T) / 4); i += 16) acc ^= p[i];
    asm volatile("" ::"s"(acc));
}

// ------------------------------------------------------------------ wave reductions (DPP)
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                 0xF, 0xF, false));
}
__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// v combined with a row broadcast (DPP row_bcast:15 or row_bcast:31) into the rows `rows`;
// the other rows keep v.
template <int CTRL, int ROWS>
__device__ __forceinline__ float bcast_f(float v) {
    const int b = __builtin_bit_cast(int, v);
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(b, b, CTRL, ROWS, 0xF, false));
}

// Max over the 64 lanes of a wave, returned to every lane: quad_perm [1,0,3,2] and [2,3,0,1],
// row_half_mirror and row_mirror leave each row of 16 lanes holding its maximum; row_bcast:15
// into rows 1 and 3 and row_bcast:31 into rows 2 and 3 carry them to lane 63, read once (one
// lane read instead of four: the top-k ranking calls this k times in a dependent chain).
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    v = fmaxf(v, bcast_f<0x142, 0xA>(v));
    v = fmaxf(v, bcast_f<0x143, 0xC>(v));
    return readlane_f(v, 63);
}

// The value of lane i ^ 16 and of lane i ^ 32, through the gfx950 lane swaps (v_permlane16_swap,
// v_permlane32_swap: the half or row that holds the partner is picked per lane), not LDS.
__device__ __forceinline__ uint32_t lane_xor16(uint32_t v) {
    const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (threadIdx.x & 16) ? p[0] : p[1];
}
__device__ __forceinline__ uint32_t lane_xor32(uint32_t v) {
    const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (threadIdx.x & 32) ? p[0] : p[1];
}
__device__ __forceinline__ float lane_xor16_f(float v) {
    return __builtin_bit_cast(float, lane_xor16(__builtin_bit_cast(uint32_t, v)));
}
__device__ __forceinline__ float lane_xor32_f(float v) {
    return __builtin_bit_cast(float, lane_xor32(__builtin_bit_cast(uint32_t, v)));
}

// Inclusive prefix sum of an integer over the 64 lanes: row_shr 1, 2, 4, 8 within each row of 16
// (lanes shifted in from outside the row read 0), then row_bcast:15 adds row 0's total to row 1
// and row 2's to row 3, and row_bcast:31 adds rows 0-1's total to rows 2 and 3.
__device__ __forceinline__ int wave_incl_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);
    return v;
}

// Sum over the 64 lanes of a wave by an xor butterfly (offsets 32, 16, ..., 1; every lane adds
// its partner's value), the router logits' reduction order, returned to every lane. No step goes
// through LDS: offsets 32 and 16 are the lane swaps above, offset 8 is row_ror:8 (lane i + 8
// mod 16 is i ^ 8), and offset 4 is row_ror:4 -- lane i + 4 mod 16 is i ^ 4 or i ^ 4 ^ 8, and
// after the offset-8 step lanes i and i ^ 8 hold the same value; offsets 2 and 1 are quad
// permutes.
__device__ __forceinline__ float wave_sum_xor(float v) {
    v += lane_xor32_f(v);
    v += lane_xor16_f(v);
    v += dpp_f<0x128>(v);   // row_ror:8
    v += dpp_f<0x124>(v);   // row_ror:4
    v += dpp_f<0x4E>(v);    // quad_perm [2,3,0,1]
    v += dpp_f<0xB1>(v);    // quad_perm [1,0,3,2]
    return v;
}

// Sum over the 64 lanes of a wave by wave_max's DPP pattern, returned to every lane.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    v += dpp_f<0x140>(v);
    return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}

// Unsigned max over the 64 lanes of a wave, returned to every lane (wave_max's DPP pattern; 0 is
// the identity, so lanes a step leaves without a source read 0).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t bcast_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, ROWS, 0xF, false);
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, dpp_u<0xB1>(v));
    v = max(v, dpp_u<0x4E>(v));
    v = max(v, dpp_u<0x141>(v));
    v = max(v, dpp_u<0x140>(v));
    v = max(v, bcast_u<0x142, 0xA>(v));
    v = max(v, bcast_u<0x143, 0xC>(v));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// The ranking key of a value: unsigned order of keys is the order of the values, +0 and -0
// share a key (they compare equal), every NaN keys 1 (below every number) and 0 is left for
// entries taken or absent.
__device__ __forceinline__ uint32_t rank_key(float f) {
    const uint32_t b = __builtin_bit_cast(uint32_t, f + 0.0f);   // -0 + 0 = +0
    const uint32_t k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return f != f ? 1u : k;
}
__device__ __forceinline__ float rank_value(uint32_t k) {
    return __builtin_bit_cast(float, (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// Top-k of E <= 64 * kPer logits held by one wave (lane l holds expert l + 64 i in v[i]):
// descending by value, ties to the lower expert id -- the order the oracle's selection loop
// defines -- and NaN after every number (lowest id first; its value reads as -inf). Each round
// takes the wave max of the values' keys and the lowest id holding it; after the call lane
// r < k holds rank r's expert and value (fewer than k entries: the ranks past them hold -1 and
// 0). With kr < k only the first kr ranks are found (the others hold -1): a prefix of the same
// order, for a caller that needs only those.
template <int kPer>
__device__ __forceinline__ void wave_topk(const float v[kPer], int E, int k, int& sel_e, float& sel_v,
                                          int kr = -1) {
    const int lane = threadIdx.x & (kWave - 1);
    uint32_t key[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) key[i] = lane + kWave * i < E ? rank_key(v[i]) : 0u;
    sel_e = -1;
    sel_v = 0.0f;
    const int rounds = kr < 0 ? k : min(kr, k);
    for (int r = 0; r < rounds; ++r) {
        uint32_t lm = key[0];
#pragma unroll
        for (int i = 1; i < kPer; ++i) lm = max(lm, key[i]);
        const uint32_t mx = wave_max_u32(lm);
        int pick = -1;
        if (mx != 0u) {
#pragma unroll
            for (int i = kPer - 1; i >= 0; --i) {
                const uint64_t b = __ballot(key[i] == mx);
                if (b) pick = kWave * i + __builtin_ctzll(b);
            }
        }
#pragma unroll
        for (int i = 0; i < kPer; ++i)
            if (lane + kWave * i == pick) key[i] = 0u;
        if (lane == r) {
            sel_e = pick;
            sel_v = pick < 0 ? 0.0f : (mx == 1u ? -__builtin_inff() : rank_value(mx));
        }
    }
}

// The routing rule a ranking applies beyond plain top-k of the logits.
struct RouteRule {
    const float* bias;   // sigmoid modes: selection bias [E] or null
    int mode, n_group, topk_group;
    float scale;
};

__device__ __forceinline__ bool route_sigmoid(int mode) { return mode >= BRX_ROUTE_SIGMOID_TOPK; }

// e^x as x = n ln2 + r (|r| <= ln2 / 2; ln2 split into a 12-bit head and a tail, Cody-Waite),
// e^r by its Taylor polynomial of degree 7 in Horner form with fused multiply-adds, scaled by
// 2^n: every step is one correctly rounded operation, so the host restatement of the routing
// gives the same bits (within 2 ulp of e^x). The sigmoid routing scores use it because their
// order decides the experts.
__device__ __forceinline__ float exp_rt(float x) {
    if (x > 88.5f) return __builtin_inff();
    if (x < -104.0f) return 0.0f;
    const float n = __builtin_rintf(x * 1.44269502f);
    float r = __builtin_fmaf(-n, 0.693115234375f, x);
    r = __builtin_fmaf(-n, 3.19461833e-05f, r);
    float p = 1.98412701e-04f;
    p = __builtin_fmaf(p, r, 1.38888892e-03f);
    p = __builtin_fmaf(p, r, 8.33333377e-03f);
    p = __builtin_fmaf(p, r, 4.16666679e-02f);
    p = __builtin_fmaf(p, r, 1.66666672e-01f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_ldexpf(p, (int)n);
}
__device__ __forceinline__ float sigmoid_f(float v) { return 1.0f / (1.0f + exp_rt(-v)); }

// Selection values of the experts this lane holds (lane l: experts l + 64 i), from their logits:
// the logit itself (softmax modes) or sigmoid(logit) + bias (sigmoid modes); with groups
// (n_group > 1) the experts outside the topk_group best groups are then taken out (softmax:
// -inf; sigmoid: 0). A group's score is its largest logit (softmax) or the sum of its two
// largest selection values (sigmoid; the second largest is the largest of the others after one
// holder of the maximum, the lowest id, is set aside); groups rank by score, ties to the lower
// group, as the top-k does.
template <int kPer>
__device__ __forceinline__ void route_values(const float v[kPer], const RouteRule& rr, int E, float c[kPer]) {
    const int lane = threadIdx.x & (kWave - 1);
    const bool sig = route_sigmoid(rr.mode);
    // the selection bias: one branch around all kPer loads (uniform), so they are in flight
    // together rather than one round trip each
    float bv[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) bv[i] = 0.0f;
    if (sig && rr.bias) {
#pragma unroll
        for (int i = 0; i < kPer; ++i) bv[i] = rr.bias[min(lane + kWave * i, E - 1)];
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) c[i] = sig ? sigmoid_f(v[i]) + bv[i] : v[i];
    if (rr.n_group <= 1) return;
    const int G = E / rr.n_group;
    float gs = -__builtin_inff();          // lane g: group g's score
    for (int g = 0; g < rr.n_group; ++g) {
        float lm = -__builtin_inff();
        bool mem[kPer];
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int e = lane + kWave * i;
            mem[i] = e >= g * G && e < (g + 1) * G;
            if (mem[i]) lm = fmaxf(lm, c[i]);
        }
        const float m1 = wave_max(lm);
        float score = m1;
        if (sig) {
            int first = -1;
#pragma unroll
            for (int i = 0; i < kPer; ++i) {
                const uint64_t b = __ballot(mem[i] && c[i] == m1);
                if (first < 0 && b) first = kWave * i + __builtin_ctzll(b);
            }
            float l2 = -__builtin_inff();
#pragma unroll
            for (int i = 0; i < kPer; ++i)
                if (mem[i] && lane + kWave * i != first) l2 = fmaxf(l2, c[i]);
            score = m1 + wave_max(l2);
        }
        if (lane == g) gs = score;
    }
    uint64_t keep = 0;
    bool live = lane < rr.n_group;
    for (int r = 0; r < rr.topk_group; ++r) {
        const float m = wave_max(live ? gs : -__builtin_inff());
        uint64_t b = __ballot(live && gs == m);
        if (!b) b = __ballot(live);        // only NaN scores left: the lowest live group
        const int g = __builtin_ctzll(b);
        keep |= 1ull << g;
        if (lane == g) live = false;
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int grp = min((lane + kWave * i) / G, 63);
        if (!((keep >> grp) & 1ull)) c[i] = sig ? 0.0f : -__builtin_inff();
    }
}

// Routing weight of the rank this lane holds (lanes >= k return 0): softmax over all E logits
// then the selected entries (renormalised to sum 1 for BRX_ROUTE_SOFTMAX_TOPK_RENORM), or a
// softmax over the k selected logits (BRX_ROUTE_TOPK_SOFTMAX).
template <int kPer>
__device__ __forceinline__ float wave_route_weight(const float v[kPer], int E, int k, int mode,
                                                   float sel_v) {
    const int lane = threadIdx.x & (kWave - 1);
    const float m = readlane_f(sel_v, 0);
    const float ex = lane < k ? expf(sel_v - m) : 0.0f;
    if (mode == BRX_ROUTE_TOPK_SOFTMAX) return ex / wave_sum(ex);
    float part = 0.0f;
#pragma unroll
    for (int i = 0; i < kPer; ++i)
        if (lane + kWave * i < E) part += expf(v[i] - m);
    float w = ex / wave_sum(part);
    if (mode == BRX_ROUTE_SOFTMAX_TOPK_RENORM) w = w / wave_sum(w);
    return w;
}

// The rule's top-k for one token whose logits this wave holds: lane r < k ends holding rank
// r's expert in sel_e and its selection value in sel_v (softmax modes: the logit). Softmax
// modes without groups rank the logits directly.
template <int kPer>
__device__ __forceinline__ void wave_select(const float v[kPer], const RouteRule& rr, int E, int k,
                                            int& sel_e, float& sel_v, int kr = -1) {
    if (!route_sigmoid(rr.mode) && rr.n_group <= 1) {
        wave_topk<kPer>(v, E, k, sel_e, sel_v, kr);
        return;
    }
    float c[kPer];
    route_values<kPer>(v, rr, E, c);
    wave_topk<kPer>(c, E, k, sel_e, sel_v, kr);
}

// The routing weight of the rank this lane holds (lanes >= k: 0), after wave_select. Softmax
// modes weigh as wave_route_weight (an eligible expert's selection value is its logit);
// sigmoid modes weigh sigmoid(logit) of the chosen expert, whose logit is fetched from the
// lane holding it (lane sel_e % 64, register sel_e / 64), renormalised to sum 1 for
// BRX_ROUTE_SIGMOID_TOPK_RENORM. The weight is then multiplied by the rule's scale.
template <int kPer>
__device__ __forceinline__ float wave_weight(const float v[kPer], const RouteRule& rr, int E, int k, int sel_e,
                                             float sel_v) {
    const int lane = threadIdx.x & (kWave - 1);
    float w;
    if (!route_sigmoid(rr.mode)) {
        w = wave_route_weight<kPer>(v, E, k, rr.mode, sel_v);
    } else {
        const int src = sel_e >= 0 ? sel_e : 0;
        float lg = 0.0f;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const float t = __shfl(v[i], src & (kWave - 1), kWave);
            if ((src >> 6) == i) lg = t;
        }
        const float s = lane < k && sel_e >= 0 ? sigmoid_f(lg) : 0.0f;
        w = rr.mode == BRX_ROUTE_SIGMOID_TOPK_RENORM ? s / wave_sum(s) : s;
    }
    return w * rr.scale;
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// The affine dot product's code values: pair i of piece m of `w` (BITS-bit affine) is the bf16
// pair (c_i, c_{i+4}) against x packed as (x_i, x_{i+4}). Below 8 bits c = 128 + q: the code pair
// of piece_pair OR'd with 0x43004300 is (128 + q_i, 128 + q_{i+4}) exactly (q < 128 fills the 7
// mantissa bits of 128). 8-bit codes do not fit there and take c = q: each code is converted to
// fp32 (exact) and its upper half kept, exact in bf16 since q has at most 8 significant bits.
template <int BITS>
constexpr float kCodeOffset = BITS == 8 ? 0.0f : 128.0f;

// Permute 8 natural-order bf16 (4 words: (x0,x1),(x2,x3),(x4,x5),(x6,x7)) into the pair
// order the affine dot product takes: (x0,x4),(x1,x5),(x2,x6),(x3,x7).
__device__ __forceinline__ void perm8(const uint32_t in[4], uint32_t out[4]) {
    out[0] = (in[0] & 0xFFFFu) | (in[2] << 16);
    out[1] = (in[0] >> 16) | (in[2] & 0xFFFF0000u);
    out[2] = (in[1] & 0xFFFFu) | (in[3] << 16);
    out[3] = (in[1] >> 16) | (in[3] & 0xFFFF0000u);
}

// The descriptor's routing rule (route_scale 0 means 1).
inline RouteRule route_rule(const brx_layer_desc& d, const float* bias) {
    RouteRule r;
    r.bias = d.route_mode >= BRX_ROUTE_SIGMOID_TOPK ? bias : nullptr;
    r.mode = d.route_mode;
    r.n_group = d.n_group > 1 ? d.n_group : 1;
    r.topk_group = d.n_group > 1 ? d.topk_group : 1;
    r.scale = d.route_scale == 0.0f ? 1.0f : d.route_scale;
    return r;
}

// ------------------------------------------------------------------ launchers
hipError_t launch_router(const brx_layer_desc& d, const void* x, const void* w_router,
                         const float* bias, const void* sgw, int T, int32_t* out_idx,
                         float* out_w, float* out_sg, float* ws_logits, hipStream_t s);
size_t router_workspace_bytes(const brx_layer_desc& d, int T);
// logits [T, E + 1] only (the shared-gate logit in column E), for T <= 64
hipError_t launch_router_logits(const brx_layer_desc& d, const void* x, const void* w_router,
                                const float* bias, const void* sgw, int T, float* logits,
                                hipStream_t s);
// phases: bit 0 = first half (gate/up), bit 1 = second half (down + combine)
struct TableEdits {
    int32_t n;
    int32_t e[kMaxTableEdits];
    int32_t v[kMaxTableEdits];
};
hipError_t launch_table_set(int32_t* g2s, const TableEdits& ed, hipStream_t s);
hipError_t launch_decode(const FwdArgs& a, void* ws, int phases, hipStream_t s);
hipError_t launch_decode_wide(const FwdArgs& a, void* ws, int phases, hipStream_t s);   // 2, 6, 8 bits
hipError_t launch_prefill(const FwdArgs& a, void* ws, size_t ws_bytes, int phases, hipStream_t s);
size_t prefill_workspace_bytes(const FwdArgs& a);
size_t decode_workspace_bytes(const FwdArgs& a);
hipError_t launch_dequant(const brx_layer_desc& d, const Layout& L, const uint8_t* expert,
                          int proj, float* out, hipStream_t s);
hipError_t launch_sort_pairs(const int32_t* pexp, int P, int E, int E_ext, int T_shared, int BM,
                             int32_t* order, int32_t* offsets, int32_t* tile_start,
                             hipStream_t s);
hipError_t launch_combine(const uint16_t* y_routed, const uint16_t* y_shared, const float* w,
                          const float* sg, int T, int k, int H, uint16_t* out, hipStream_t s);

}  // namespace brx
