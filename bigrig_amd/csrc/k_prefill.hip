// Prefill chunks: (token, expert) pairs bucketed per expert, then grouped GEMMs on MFMA.
//
// Replaces the reference's expert-sorted prefill: the stable argsort of pairs by expert
// (bigrig_engine/stream.py:1526-1530, 1244-1250), the sorted `mx.gather_qmm` per projection
// (stream.py:1320-1336, 1605-1631), the SwiGLU between them and the inverse permutation that
// restores (token, k) order (stream.py:1558-1561, _scatter_unsort 1829-1831), followed by the
// caller's router-weighted combine (stream.py:1523-1525).
//
//   k_bucket   one block per expert: in one pass over the pairs, the histogram of all of them
//              and the stable (pair-order) compaction of the expert's pairs into LDS; then the
//              expert's run offset, the run copied out in order, and one tile descriptor {expert,
//              first bucketed row, rows, slot} per 128-row M tile, placed in a tile list that
//              holds every tile of more than 64 rows before the smaller ones, so the GEMM grids
//              dispatch the long tiles first and the short ones fill the end.
//   k_pf_gemm  grouped GEMM, tile = (M tile of one expert's pairs, 256 columns), one wave
//              per SIMD, v_mfma_f32_32x32x16_bf16.  KIND 0 (gate/up): A rows are the pairs'
//              token activations gathered from x, B rows the gate and up weights of 128
//              intermediate features; the epilogue applies act() and stores h (bf16) in
//              bucketed order.  KIND 1 (down):
//              A = h rows, B = down weights of 256 output columns; the epilogue stores each
//              pair's bf16 row at its (token, k) position.  A is staged through LDS, B is
//              dequantized from its packed codes (affine 2-8 bits, MXFP4; bf16 as loaded) into MFMA
//              operand registers; fp32 accumulators (details at the kernel). M tiles are 128
//              rows (64 for 6- and 8-bit codes and bf16 weights).
//   k_combine  out[t] = sum_j w[t,j] * y[t,j] (+ shared_gate[t] * y_shared[t]), k-ordered.
// Every output element is one MFMA accumulation over K in a fixed K order, so a row's value
// does not depend on which other pairs share its tile.
//
// Blocks are dispatched round-robin over the 8 XCDs (block b runs on XCD b % 8).  The GEMM
// grids are 1-D and map b to (M tile, N tile) so that an XCD sweeps every N tile of an M
// tile before the next one: the tile's A rows are read into that XCD's L2 once and reused by
// all its N tiles.
#include <type_traits>

#include "brx_internal.h"

namespace brx {
namespace {

constexpr int kBM = 128;          // pairs per M tile
constexpr int kBK = 64;           // K step
constexpr int kThreads = 256;
constexpr int kXcd = 8;

// ------------------------------------------------------------------ bucketing
// Pairs are read coalesced: in each pass of kBucketPass pairs, wave w takes the 1024 pairs
// [w * 1024, w * 1024 + 1024) and its lane l the pairs l + 64 i (i < 16), so a load
// instruction reads 64 consecutive pairs, and the histogram's LDS atomics of one instruction
// (8 tokens x top-8, distinct experts within a token) hit one address at most 8 times. The
// stable compaction of a pass is 16 ballots per wave and one scan of the 16 wave totals.
constexpr int kBucketThreads = 1024;
constexpr int kBucketPer = 16;                                 // pairs per lane per pass
constexpr int kBucketWaveRun = kWave * kBucketPer;            // pairs per wave per pass
constexpr int kBucketPass = kBucketThreads * kBucketPer;
constexpr int kBucketListMax = 8192;                          // pairs an LDS list may hold

// The experts of a lane's pairs pb + 64 i (i < kBucketPer; id E for the shared expert's pairs
// past the P routed ones). The loads are unconditional (index clamped into the routed pairs), so
// a lane's sixteen are in flight together rather than one round trip each.
__device__ __forceinline__ void bucket_experts(const int32_t* __restrict__ pexp, int pb, int P, int E, int emax,
                                               int ex[kBucketPer]) {
    if (P > 0) {   // uniform
#pragma unroll
        for (int i = 0; i < kBucketPer; ++i) ex[i] = pexp[min(pb + i * kWave, P - 1)];
    }
#pragma unroll
    for (int i = 0; i < kBucketPer; ++i) ex[i] = pb + i * kWave < P ? min(max(ex[i], 0), emax) : E;
}

__global__ __launch_bounds__(kBucketThreads) void k_bucket(const int32_t* __restrict__ pexp, int P, int E,
                                                           int E_ext, int T_sh, int BM,
                                                           const int32_t* __restrict__ g2s, int capacity,
                                                           int host, int32_t* __restrict__ err,
                                                           int32_t* __restrict__ order,
                                                           int32_t* __restrict__ offsets,
                                                           int32_t* __restrict__ tile_start,
                                                           int4* __restrict__ tinfo, int lcap) {
    // E_ext = E + 1 when a shared expert exists (id E); T_sh shared pairs follow the P routed.
    // LDS: the histogram [E_ext], then a list of up to lcap of this expert's pairs.
    extern __shared__ int32_t hist[];
    int32_t* list = hist + E_ext;
    constexpr int kNw = kBucketThreads / kWave;
    __shared__ int32_t wsum[kNw];
    __shared__ int32_t base_s[3];
    const int P_ext = P + T_sh;
    const int emax = E_ext - 1;
    const int e = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const uint64_t below = (1ull << lane) - 1ull;
    for (int i = tid; i < E_ext; i += kBucketThreads) hist[i] = 0;
    __syncthreads();
    // one pass over the pairs: the histogram of every pair's expert (each block needs all counts
    // below its own expert) and the stable (pair-order) compaction of this expert's pairs into
    // the LDS list, pair order = (pass, wave, i, lane)
    int run = 0;
    for (int p0 = 0; p0 < P_ext; p0 += kBucketPass) {
        const int pb = p0 + wv * kBucketWaveRun + lane;
        int ex[kBucketPer];
        bucket_experts(pexp, pb, P, E, emax, ex);
#pragma unroll
        for (int i = 0; i < kBucketPer; ++i)
            if (pb + i * kWave < P_ext) atomicAdd(&hist[ex[i]], 1);
        {
            uint64_t m[kBucketPer];
            int cnt = 0;
#pragma unroll
            for (int i = 0; i < kBucketPer; ++i) {
                m[i] = __ballot(pb + i * kWave < P_ext && ex[i] == e);
                cnt += __popcll(m[i]);
            }
            if (lane == 0) wsum[wv] = cnt;
            __syncthreads();
            int before = 0, total = 0;
#pragma unroll
            for (int w = 0; w < kNw; ++w) {
                const int v = wsum[w];
                before += w < wv ? v : 0;
                total += v;
            }
            int dst = run + before;
#pragma unroll
            for (int i = 0; i < kBucketPer; ++i) {
                const int q = dst + __popcll(m[i] & below);
                if (((m[i] >> lane) & 1ull) && q < lcap) list[q] = pb + i * kWave;
                dst += __popcll(m[i]);
            }
            run += total;
            __syncthreads();
        }
    }
    __syncthreads();
    if (wv == 0) {
        // expert e's run offset (counts of the experts before it) and its tiles' places in the
        // tile list, which holds the tiles of more than BM / 2 rows of every expert first, then
        // the smaller ones (at most one per expert, its last), each class in expert order, so
        // the GEMMs take the long tiles first
        int off = 0, big = 0, small = 0, big_all = 0, small_all = 0;
        for (int j = lane; j < E_ext; j += 64) {
            const int n = hist[j], r = n % BM;
            const int nb = n / BM + (r > BM / 2 ? 1 : 0), ns = (r > 0 && r <= BM / 2) ? 1 : 0;
            if (j < e) { off += n; big += nb; small += ns; }
            big_all += nb;
            small_all += ns;
        }
        for (int sft = 32; sft >= 1; sft >>= 1) {
            off += __shfl_xor(off, sft, 64);
            big += __shfl_xor(big, sft, 64);
            small += __shfl_xor(small, sft, 64);
            big_all += __shfl_xor(big_all, sft, 64);
            small_all += __shfl_xor(small_all, sft, 64);
        }
        if (lane == 0) {
            base_s[0] = off;
            base_s[1] = big;
            base_s[2] = big_all + small;
            offsets[e] = off;
            tile_start[e] = big;
            if (e == E_ext - 1) {
                offsets[E_ext] = P_ext;
                tile_start[E_ext] = big_all + small_all;   // tiles in all (what the GEMMs read)
            }
        }
    }
    __syncthreads();
    const int n = hist[e], off = base_s[0];
    if (tinfo) {
        const int big = base_s[1], small = base_s[2];
        int slot = 0;
        if (e < E && g2s) {   // the slot code: a slot, -2 - e for an expert read from host backing
            const int v = g2s[e];
            slot = v >= 0 ? min(v, capacity - 1) : (host ? -2 - e : kAbsentCode);
            if (slot == kAbsentCode && n > 0 && tid == 0 && err) {
                err[1] = e;
                err[0] = 1;
            }
        }
        for (int j = tid; j * BM < n; j += kBucketThreads) {
            const int rows = min(BM, n - j * BM);
            tinfo[rows > BM / 2 ? big + j : small] = make_int4(e, off + j * BM, rows, slot);
        }
    }
    if (n <= lcap) {
        // the run, copied out in order (coalesced)
        for (int i = tid; i < n; i += kBucketThreads) order[off + i] = list[i];
        return;
    }
    // the expert's pairs did not fit the LDS list: a second pass compacts straight into the run
    run = off;
    for (int p0 = 0; p0 < P_ext; p0 += kBucketPass) {
        const int pb = p0 + wv * kBucketWaveRun + lane;
        uint64_t m[kBucketPer];
        int cnt = 0;
        int ex[kBucketPer];
        bucket_experts(pexp, pb, P, E, emax, ex);
#pragma unroll
        for (int i = 0; i < kBucketPer; ++i) {
            const int p = pb + i * kWave;
            m[i] = __ballot(p < P_ext && ex[i] == e);
            cnt += __popcll(m[i]);
        }
        if (lane == 0) wsum[wv] = cnt;
        __syncthreads();
        int before = 0, total = 0;
#pragma unroll
        for (int w = 0; w < kNw; ++w) {
            const int v = wsum[w];
            before += w < wv ? v : 0;
            total += v;
        }
        int dst = run + before;
#pragma unroll
        for (int i = 0; i < kBucketPer; ++i) {
            if ((m[i] >> lane) & 1ull) order[dst + __popcll(m[i] & below)] = pb + i * kWave;
            dst += __popcll(m[i]);
        }
        run += total;
        __syncthreads();
    }
}

__device__ __forceinline__ int pair_token(const FwdArgs& a, int pair) {
    return pair < a.P ? pair_tok(a, pair) : pair - a.P;
}

__device__ __forceinline__ uint32_t pk_bf16(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, bf16x2_t{(__bf16)lo, (__bf16)hi});
}

// native vector (not HIP's uint4 struct, whose copies are memcpys that keep arrays of it in
// scratch memory)
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3_t __attribute__((ext_vector_type(3)));

// ------------------------------------------------------------------ grouped GEMM
// One block = 256 threads = 4 waves, one wave per SIMD; the tile is MF * 16 rows (one M tile
// of one expert, MF in {2, 4, 8} chosen by the tile's row count) by 256 columns, wave w owning
// columns [64 w, 64 w + 64) and every row, so each weight is dequantized by exactly one lane
// and each A fragment read from LDS feeds two MFMAs.  KIND 0 (gate/up): a wave's 64 columns
// are 32 gate features and the up rows of the same 32 features; KIND 1 (down): 64 output
// columns.  The MFMA is v_mfma_f32_32x32x16_bf16 (32 x 32 fragments, fp32 accumulators in
// VGPRs): on gfx950 it issues at close to the bf16 peak next to the dequantization's VALU
// work, where 16x16x32 loses a third.
//
// K order inside a 64-wide stage: MFMA kk (0..3) takes from lane l the 8 K of chunk
// 4 (l >> 5) + kk, so a lane's B operands for the stage are the four words of one 16-byte half
// of its weight row's 32-byte stage segment, and its A operand the matching 16-byte chunk of
// the activation row.  Each output is still the sum over all K.
//
// Per stage, the A tile (128 rows x 64 bf16) and the rows' scales are copied global -> LDS by
// the buffer unit (buffer_load ... lds, no registers): A's 16-byte chunks XOR-swizzled by row
// so the rows an MFMA operand read touches fall in distinct bank groups, each weight row's
// scale (and bias) in a 32-bit slot, two stages' values per slot when the scale rows are
// 4-byte aligned. The weights are not shared between waves, so each lane loads its own B
// words straight into registers (one 16-byte load per fragment and stage); keeping them out
// of LDS leaves room for a ring of NS = 4 stages, two of them in flight while the MFMAs consume
// one (under a full load HBM answers in ~4 us, so the bytes in flight per CU bound the rate).
// Per stage s:
//   wait until stage s + 1 has landed (s_waitcnt vmcnt(N), N = the later stages' loads);
//   barrier (so every wave's copies are visible and stage s - 1's slot is free);
//   issue the loads of stage s + NS - 1 (none past the last stage); read the scales of stage
//   s + 1 from LDS;
//   MFMA kk of stage s  | dequantize B(s) kk + 1 (kk = 3: B(s + 1) kk 0), read A(s) kk + 1
//   (kk = 3: A(s + 1) kk 0) from LDS
// The MFMA-interleaved VALU code is plain C++ so that the compiler's MFMA hazard checks cover
// it.
constexpr int kGemmWaves = 4;
constexpr int kGemmThreads = 64 * kGemmWaves;
constexpr int kNJ = 2;                       // 32-column fragments per wave
constexpr int kWaveN = 32 * kNJ;             // columns per wave
constexpr int kBlockN = kGemmWaves * kWaveN; // columns per block
constexpr int kNS = 4;                       // LDS ring stages (even: see pf_tile)
constexpr int kStA = kBM * kBK * 2;          // stage bytes: A tile
constexpr int kStS = kBlockN * 4 * 2;        // scale and bias per row, one 32-bit LDS slot each
constexpr int kStage = kStA + kStS;
static_assert(kNS % 2 == 0, "the paired scale copies follow stage parity through the unrolled ring");
// The block's LDS: the ring (A stages, per-stage scale slots or the scale table, then the output
// tile) takes all of a CU's 160 KB that two blocks can share, less the down kernel's row list.
constexpr int kRing = 80 * 1024 - kBM * 4;
constexpr int kBPairLds = 16 * 1024;   // paired-B staging of 32-row tiles, at the ring's end
constexpr int kBPairSets = 3;          // paired-B register sets (pairs in flight + the current)
static_assert(kNS * kStage <= kRing, "the per-stage ring must fit");
static_assert(kNS * (2 * 16 * kBK * 2 + kStS) + kBPairLds <= kRing, "a 32-row tile's ring and B staging must fit");
static_assert(8 * 16 * (kBlockN + 8) * 2 <= kRing, "the widest output tile must fit in the ring");

typedef __attribute__((address_space(3))) void* LDS_PTR;
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// swizzle key of A tile row m: 16-byte chunk c of the row sits in slot c ^ a_key(m); rows
// 2t and 2t + 1 share a 256-byte bank row, so keys (m >> 1) & 7 spread 16 consecutive rows
// over 16 distinct bank groups
__device__ __forceinline__ int a_key(int m) { return (m >> 1) & 7; }

// waits for this wave's LDS accesses, then for every wave
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// waits until at most N of this wave's memory loads (copies into LDS and loads into registers)
// are in flight, then for every wave. The wait is the builtin, so the compiler's own wait
// placement knows which loads it covers and adds none for the registers it has made ready;
// the barrier is inline asm with a memory clobber, so no LDS access moves across it.
template <int N>
__device__ __forceinline__ void dma_wait_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
    asm volatile("s_barrier" ::: "memory");
}

// Copies into LDS a wave has issued after stage s + 1's when it waits for stage s + 1 at
// iteration s (s of parity par): those of stages s + 2 .. s + ns - 2, nv0 for an even stage,
// nv1 for an odd one.
constexpr int loads_after(int ns, int nv0, int nv1, int par) {
    int n = 0;
    for (int i = 2; i <= ns - 2; ++i) n += ((par + i) & 1) ? nv1 : nv0;
    return n;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// Dequantize piece kk (8 weights, natural K order) of a lane's words `w` into a bf16x8 MFMA
// operand.
//   affine: w = s q + b with one fp32 rounding, then rounded to bf16 (v_cvt_pk_bf16_f32).
//     Each code q is read as the fp16 subnormal q 2^-24 (the code alone in a 16-bit half, exact
//     when widened to fp32: q < 1024) and v_fma_mix_f32 forms fma(q 2^-24, s 2^24, b): the
//     product is exactly s q, so the result is the same fl(s q + b) as fmaf(s, q, b). `s24` is
//     s 2^24 (exact for any scale below 2^104). piece_pair puts codes i and 4 + i in the two
//     halves of one register, so a 4-bit piece costs 7 extractions, 8 fma_mix and 4 packs.
//   MXFP4: the hardware converts two e2m1 codes with the e8m0 scale, exact in bf16.
//   Unquantized bf16 weights are the operand as loaded.
template <int MODE>
__device__ __forceinline__ bf16x8_t dq8(const uint32_t* w, int kk, float s24, float b, float sc) {
    uint32_t o[4];
    if constexpr (kAffine<MODE>) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // codes i (low half) and 4 + i (high half)
            const uint32_t t = piece_pair<kBits<MODE>>(w, kk, i);
            v[i] = __builtin_fmaf((float)__builtin_bit_cast(_Float16, (uint16_t)(t & 0xFFFFu)), s24, b);
            v[4 + i] = __builtin_fmaf((float)__builtin_bit_cast(_Float16, (uint16_t)(t >> 16)), s24, b);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = pk_bf16(v[2 * j], v[2 * j + 1]);
    } else if constexpr (MODE == kModeBf16) {
        // unquantized: the piece is 8 bf16 weights, 4 words in natural K order
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = w[4 * kk + j];
    } else {
        const uint32_t q = w[kk];
        o[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, sc, 0));
        o[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, sc, 1));
        o[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, sc, 2));
        o[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(q, sc, 3));
    }
    return __builtin_bit_cast(bf16x8_t, u32x4_t{o[0], o[1], o[2], o[3]});
}

// B words a lane holds per stage (half of a row's 64-code stage segment: 32 codes), and the
// loads that bring them in (16-byte loads, plus one 8-byte load for 6 bits; one 8- or 12-byte
// load for 2 and 3 bits; four 16-byte loads for bf16 weights).
template <int MODE>
constexpr int kBW = kBits<MODE>;
template <int MODE>
constexpr int kBLoads = kBits<MODE> == 16 ? 4 : kBits<MODE> >= 6 ? 2 : 1;
// M tile height: 128 rows, or 64 for 6- and 8-bit codes and bf16 weights, whose B words (48, 64
// and 128 registers over the ring) leave no room for the accumulators of a 128-row tile at two
// blocks per CU
template <int MODE>
constexpr int kTileRows = kBits<MODE> >= 6 ? 64 : 128;

// The activation of one output element with the rule fixed at compile time (act_apply's
// arithmetic for that rule, so the same bits).
template <int ACT>
__device__ __forceinline__ float act_fixed(float g, float u, float alpha, float limit) {
    if constexpr (ACT == BRX_ACT_SWIGLU) return silu_mul(g, u);
    else if constexpr (ACT == BRX_ACT_SILU_MLP) return x_sigmoid(g, 1.0f);
    else {
        g = fminf(g, limit);
        u = fminf(fmaxf(u, -limit), limit);
        return x_sigmoid(g, alpha) * (u + 1.0f);
    }
}

// The gate/up epilogue of one activation rule: act(gate + bias, up + bias) (or SiLU(fc1 + bias))
// of every accumulator into the LDS tile T (row stride TS elements), NaN for an absent expert.
// A gated tile's wave holds 32 features: fragment 0 their gate rows, fragment 1 their up rows;
// a two-layer expert's fragment nj holds 32 fc1 features of its own. Element i of a 32 x 32
// fragment is row 8 (i / 4) + 4 kh + i % 4, column l32.
template <int MR, int ACT>
__device__ __forceinline__ void pf_store_h(const FwdArgs& a, const Layout& L, const uint8_t* base, int inter,
                                           bool absent, int nt, const f32x16_t (&acc)[MR][kNJ], uint16_t* T,
                                           int wv, int kh, int l32) {
    const float nan = absent_nan();
    if constexpr (ACT == BRX_ACT_SILU_MLP) {
        constexpr int TS = kBlockN + 8;
#pragma unroll
        for (int nj = 0; nj < kNJ; ++nj) {
            const int fl = nj * 128 + wv * 32 + l32;
            const int f = min(nt * kBlockN + fl, inter - 1);
            const float bg = L.p[0].bias >= 0 ? bf2f(reinterpret_cast<const uint16_t*>(base + L.p[0].bias)[f]) : 0.f;
#pragma unroll
            for (int mi = 0; mi < MR; ++mi) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    float h = act_fixed<ACT>(acc[mi][nj][i] + bg, 0.f, a.alpha, a.limit);
                    h = absent ? nan : h;
                    T[(mi * 32 + 8 * (i >> 2) + 4 * kh + (i & 3)) * TS + fl] = __builtin_bit_cast(uint16_t, (__bf16)h);
                }
            }
        }
    } else {
        constexpr int TS = kBlockN / 2 + 8;
        const int fl = wv * (kWaveN / 2) + l32;
        const int f = min(nt * (kBlockN / 2) + fl, inter - 1);
        float bg = 0.f, bu = 0.f;
        if (L.p[0].bias >= 0) {
            bg = bf2f(reinterpret_cast<const uint16_t*>(base + L.p[0].bias)[f]);
            bu = bf2f(reinterpret_cast<const uint16_t*>(base + L.p[1].bias)[f]);
        }
#pragma unroll
        for (int mi = 0; mi < MR; ++mi) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float h = act_fixed<ACT>(acc[mi][0][i] + bg, acc[mi][1][i] + bu, a.alpha, a.limit);
                h = absent ? nan : h;
                T[(mi * 32 + 8 * (i >> 2) + 4 * kh + (i & 3)) * TS + fl] = __builtin_bit_cast(uint16_t, (__bf16)h);
            }
        }
    }
}

// The epilogue of a GEMM tile: MR x kNJ fragments of fp32 accumulators per wave go through LDS
// (`ring`, free once the caller has waited for every copy into it and synchronised) so the
// global stores are 16-byte chunks of contiguous row segments. KIND 0: the activation (one code
// path per rule, chosen once per tile) stored as bf16 h rows at their bucketed positions; KIND 1:
// + bias, each pair's row stored at its (token, k) position (dst_s). An absent expert's h rows
// are NaN.
template <int KIND, int MR>
__device__ __forceinline__ void pf_store(const FwdArgs& a, const Layout& L, const uint8_t* base, bool mlp, int inter,
                                         int slot, int nt, int m0, int rows, const f32x16_t (&acc)[MR][kNJ],
                                         uint8_t* ring, const int32_t* dst_s, uint16_t* __restrict__ hbuf,
                                         int hstride, uint16_t* __restrict__ y_routed,
                                         uint16_t* __restrict__ y_shared) {
    constexpr int MF = MR * 2;
    const int H = a.H;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kh = lane >> 5, l32 = lane & 31;
    uint16_t* T = reinterpret_cast<uint16_t*>(ring);
    if constexpr (KIND == 0) {
        const bool absent = slot == kAbsentCode;
        if (mlp)
            pf_store_h<MR, BRX_ACT_SILU_MLP>(a, L, base, inter, absent, nt, acc, T, wv, kh, l32);
        else if (a.act == BRX_ACT_SWIGLU_CLAMPED)
            pf_store_h<MR, BRX_ACT_SWIGLU_CLAMPED>(a, L, base, inter, absent, nt, acc, T, wv, kh, l32);
        else
            pf_store_h<MR, BRX_ACT_SWIGLU>(a, L, base, inter, absent, nt, acc, T, wv, kh, l32);
        lds_barrier();
        // a two-layer expert's tile holds kBlockN features, a gated one's kBlockN / 2
        const int fpb = mlp ? kBlockN : kBlockN / 2;
        const int TS = fpb + 8;
        const int CH = fpb / 8;
        for (int c = tid; c < MF * 16 * CH; c += kGemmThreads) {
            const int r = c / CH, f0 = nt * fpb + (c % CH) * 8;
            if (r < rows && f0 < inter)
                *reinterpret_cast<u32x4_t*>(hbuf + (int64_t)(m0 + r) * hstride + f0) =
                    *reinterpret_cast<const u32x4_t*>(T + r * TS + (c % CH) * 8);
        }
    } else {
        constexpr int TS = kBlockN + 8;
        constexpr int CH = kBlockN / 8;
#pragma unroll
        for (int nj = 0; nj < kNJ; ++nj) {
            const int nl = wv * kWaveN + nj * 32 + l32;
            float bd = 0.f;
            if (L.p[2].bias >= 0)
                bd = bf2f(reinterpret_cast<const uint16_t*>(base + L.p[2].bias)[min(nt * kBlockN + nl, H - 1)]);
#pragma unroll
            for (int mi = 0; mi < MR; ++mi) {
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    T[(mi * 32 + 8 * (i >> 2) + 4 * kh + (i & 3)) * TS + nl] =
                        __builtin_bit_cast(uint16_t, (__bf16)(acc[mi][nj][i] + bd));
            }
        }
        lds_barrier();
        for (int c = tid; c < MF * 16 * CH; c += kGemmThreads) {
            const int r = c / CH, n0 = nt * kBlockN + (c % CH) * 8;
            if (r < rows && n0 < H) {
                const int d = dst_s[r];
                uint16_t* dst = d >= 0 ? y_routed + (int64_t)d * H + n0 : y_shared + (int64_t)(-2 - d) * H + n0;
                *reinterpret_cast<u32x4_t*>(dst) = *reinterpret_cast<const u32x4_t*>(T + r * TS + (c % CH) * 8);
            }
        }
    }
}

// How a block copies its rows' scales into LDS: per row and stage one 16-bit affine scale and
// bias, or MXFP4's two e8m0 bytes. One copy ("unit") per row is 4 bytes holding stages 2u and
// 2u + 1 when every scale row and array of the block's matrices is 4-byte aligned and a group
// is one stage (affine groups of 64: K / 64 even; MXFP4: K a multiple of 128), else 2 bytes: the
// value of stage u, or of group u spanning stages 2u and 2u + 1 (affine groups of 128). A
// 16-bit copy into LDS fills a 32-bit slot, zero-extended.
struct ScalePlan {
    bool pair;
    int gs;         // stage -> group shift (1: groups of 128)
    int nu;         // units per row
    int pitch;      // scale-table slots per row: nu rounded up to odd, so 32 rows read conflict-free
    int rowbytes;   // bytes of one row of a scale array
};
template <int MODE, int KIND>
__device__ __forceinline__ ScalePlan scale_plan(const FwdArgs& a, const Layout& L, int K, bool mlp) {
    ScalePlan p;
    p.gs = kAffine<MODE> ? a.gshift : 0;
    p.rowbytes = kAffine<MODE> ? ((K / 64) >> p.gs) * 2 : K / 32;
    bool pair = (p.rowbytes & 3) == 0 && p.gs == 0;
#pragma unroll
    for (int pj = 0; pj < 3; ++pj)
        if (KIND == 0 ? (pj == 0 || (pj == 1 && !mlp)) : pj == 2)
            pair = pair && ((L.p[pj].s & 3) == 0) && (!kAffine<MODE> || (L.p[pj].b & 3) == 0);
    p.pair = pair;
    p.nu = p.rowbytes / (pair ? 4 : 2);
    p.pitch = p.nu | 1;
    return p;
}

// LDS bytes of a tile of MF x 16 rows: its A ring, plus the scale table when it has one
// (256 rows x pitch slots for each scale array; the per-stage copies sit in the ring otherwise).
template <int MODE>
__host__ __device__ constexpr int tile_lds(int MF, bool tbl, int pitch) {
    return tbl ? kNS * MF * 16 * kBK * 2 + (kAffine<MODE> ? 2 : 1) * 256 * pitch * 4
               : kNS * (MF * 16 * kBK * 2 + kStS);
}

template <int MODE, bool F16, int KIND, int MF, bool TBL>
__device__ __forceinline__ void pf_tile(const FwdArgs& a, const int32_t* __restrict__ order,
                                        uint16_t* __restrict__ hbuf, int hstride,
                                        uint16_t* __restrict__ y_routed, uint16_t* __restrict__ y_shared,
                                        uint8_t* ring, int32_t* dst_s, int e, int m0, int rows, int slot,
                                        int nt) {
    constexpr int NA = MF * 16 * 8 / 64 / kGemmWaves;   // A copies per wave per stage
    constexpr int NS = kNS;                             // stages in the ring
    constexpr int SA = MF * 16 * kBK * 2;               // A bytes per stage
    constexpr int SS = TBL ? SA : SA + kStS;            // stage bytes in the ring
    // loads per wave of an odd stage (A copies, B loads) and of an even stage (+ the scale copies
    // of it and the next stage, unless the tile reads its scales from the table)
    constexpr int NV1 = NA + kNJ * kBLoads<MODE>;
    constexpr int NV0 = NV1 + ((TBL || !kScaled<MODE>) ? 0 : kAffine<MODE> ? 2 : 1);
    // A (and scale) copies alone, of an even and an odd stage
    constexpr int NVA1 = NA;
    constexpr int NVA0 = NV0 - kNJ * kBLoads<MODE>;
    // 32-row tiles of 4-bit codes (affine or MXFP4) read B by stage pairs (below)
    constexpr bool BPAIR = MF == 2 && kBW<MODE> == 4;
    constexpr int B = kBits<MODE>;
    const bool sh = e >= a.E;
    const int inter = sh ? a.I_sh : a.I;
    const int H = a.H;
    const int K = KIND == 0 ? H : inter;
    const int nsteps = K / kBK;
    const Layout& L = sh ? a.lay_sh : a.lay;
    const uint8_t* base = sh ? a.shared : code_base(a, clamp_code(a, slot));
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kh = lane >> 5, l32 = lane & 31;

    // ---- A: wave wv fills 1 KB chunks [wv * NA, wv * NA + NA) of a stage's A tile; lane l of
    // chunk ii lands in 16-byte slot ii * 64 + l = (row, physical slot p) and carries the
    // row's logical K chunk p ^ key(row)
    // A rows past `rows` (the padding of an expert's last tile) are copied from past the end of
    // the buffer: the buffer unit's range check returns zeros without touching memory, so they
    // cost no cache traffic (their outputs are never stored) and every wave still issues the
    // same copies, which the stage waits count
    const uint32_t a_bytes = KIND == 0 ? (uint32_t)((int64_t)a.T * H * 2)
                                       : (uint32_t)((int64_t)(m0 + rows) * hstride * 2);
    const __amdgpu_buffer_rsrc_t ra_rsrc = make_rsrc(KIND == 0 ? (const void*)a.x : (const void*)hbuf, a_bytes);
    uint32_t va[NA];
#pragma unroll
    for (int i = 0; i < NA; ++i) {
        const int ci = (wv * NA + i) * 64 + lane;
        const int rl = ci >> 3;                            // LDS row
        const int r = min(rl, rows - 1);
        const int c = (ci & 7) ^ a_key(rl);
        if constexpr (KIND == 0) {
            va[i] = (uint32_t)pair_token(a, order[m0 + r]) * (uint32_t)(H * 2) + c * 16;
        } else {
            va[i] = (uint32_t)(m0 + r) * (uint32_t)(hstride * 2) + c * 16;
        }
        if (rl >= rows) va[i] = a_bytes;
    }
    // ---- B: the block's 256 weight rows (KIND 0: gate rows of features nt * 128 + [0, 128),
    // then the up rows of the same features; KIND 1: down rows nt * 256 + [0, 256)), 8 B bytes
    // of each per stage (64 codes). A lane loads its own operands straight into registers: the
    // half kh (4 B bytes) of the stage segment of row brow[nj] (fragment nj, column l32), so one
    // load instruction reads 32 rows x 8 B contiguous bytes. Rows past the matrix repeat its
    // last row.
    const __amdgpu_buffer_rsrc_t rb_rsrc = make_rsrc(base, (uint32_t)L.bytes);
    // a two-layer expert (fc1 / fc2): the block's 256 first-projection rows are 256 fc1
    // features, all from matrix 0, instead of 128 gate and the same 128 up features
    const bool mlp = KIND == 0 && a.act == BRX_ACT_SILU_MLP;
    auto mat_row = [&](int br) __attribute__((always_inline)) {
        return KIND == 0 ? (mlp ? min(nt * 256 + br, inter - 1) : min(nt * 128 + (br & 127), inter - 1))
                         : min(nt * 256 + br, H - 1);
    };
    int brow[kNJ];
    uint32_t vbw[kNJ];
#pragma unroll
    for (int nj = 0; nj < kNJ; ++nj) {
        brow[nj] = KIND == 0 ? nj * 128 + wv * 32 + l32 : wv * 64 + nj * 32 + l32;
        const int pj = KIND == 0 ? (mlp ? 0 : nj) : 2;
        vbw[nj] = (uint32_t)L.p[pj].w + (uint32_t)mat_row(brow[nj]) * (uint32_t)(K * B / 8) + kh * (4 * B);
    }
    // ---- scales (ScalePlan). Without the table, wave wv copies those of rows 64 wv + lane into
    // a 32-bit slot per row of the stage's ring slot, one unit per stage pair (paired) or stage;
    // the waits below assume the paired count, which unpaired makes them wait for one or two
    // more copies than they need. With the table (TBL), every unit of every row is copied once,
    // before the first stage, into [256 rows][pitch] slots after the A ring: lanes run along
    // each row's contiguous scale array, so a copy instruction touches a few cache lines rather
    // than one per lane, and no stage copies scales.
    const ScalePlan sp = scale_plan<MODE, KIND>(a, L, K, mlp);
    const int gs = sp.gs;
    const bool spair = sp.pair;
    const int p_w = KIND == 0 ? (mlp ? 0 : (wv >= 2 ? 1 : 0)) : 2;  // matrix of the rows this wave copies
    const int so = (int)L.p[p_w].s, bo = (int)L.p[p_w].b;
    const uint32_t vsc = (uint32_t)mat_row(wv * 64 + lane) * (uint32_t)sp.rowbytes;
    uint8_t* const tbl = ring + NS * SA;
    if constexpr (KIND == 1) {
        if (tid < kBM) {
            int d = -1;
            if (tid < rows) {
                const int pair = order[m0 + tid];
                d = pair < a.P ? pair_row(a, pair) : -2 - (pair - a.P);
            }
            dst_s[tid] = d;
        }
    }

    // the lane's B words of one stage (fragment nj: the B words of its half, 8 codes a piece)
    struct BReg {
        uint32_t w[kNJ][kBW<MODE>];
    };
    // issue the A and scale copies of stage s into ring slot s % NS
    auto issue_a = [&](int s) __attribute__((always_inline)) {
        const int g = min(s, nsteps - 1);
        uint8_t* st = ring + (s % NS) * SS;
#pragma unroll
        for (int i = 0; i < NA; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra_rsrc, (LDS_PTR)(st + (wv * NA + i) * 1024), 16,
                                                     va[i], g * 128, 0, 0);
        // scales: paired, an even stage's slot holds its 16-bit scale (and bias) value in the
        // low half and the next stage's in the high half and an odd stage copies nothing;
        // unpaired, every stage copies its own 16 bits
        if constexpr (TBL || !kScaled<MODE>) {
        } else if (spair) {
            if ((s & 1) == 0) {
                const int gp = g & ~1;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rb_rsrc, (LDS_PTR)(st + SA + wv * 256), 4, vsc,
                                                         so + gp * 2, 0, 0);
                if constexpr (kAffine<MODE>)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rb_rsrc, (LDS_PTR)(st + SA + 1024 + wv * 256), 4,
                                                             vsc, bo + gp * 2, 0, 0);
            }
        } else {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb_rsrc, (LDS_PTR)(st + SA + wv * 256), 2, vsc,
                                                     so + (g >> gs) * 2, 0, 0);
            if constexpr (kAffine<MODE>)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rb_rsrc, (LDS_PTR)(st + SA + 1024 + wv * 256), 2,
                                                         vsc, bo + (g >> gs) * 2, 0, 0);
        }
    };
    // issue the B loads of stage s into `br`: the lane's half of the stage segment, 4 B bytes
    // (kBLoads loads per fragment)
    auto issue_b = [&](int s, BReg& br) __attribute__((always_inline)) {
        const int g = min(s, nsteps - 1);
#pragma unroll
        for (int nj = 0; nj < kNJ; ++nj) {
            uint32_t* q = br.w[nj];
            const int go = g * (8 * B);
            if constexpr (B == 2) {
                const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(rb_rsrc, vbw[nj], go, 0);
                q[0] = v[0]; q[1] = v[1];
            } else if constexpr (B == 3) {
                const u32x3_t v = __builtin_amdgcn_raw_buffer_load_b96(rb_rsrc, vbw[nj], go, 0);
                q[0] = v[0]; q[1] = v[1]; q[2] = v[2];
            } else {
                const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(rb_rsrc, vbw[nj], go, 0);
                q[0] = v[0]; q[1] = v[1]; q[2] = v[2]; q[3] = v[3];
                if constexpr (B == 6) {
                    const u32x2_t u = __builtin_amdgcn_raw_buffer_load_b64(rb_rsrc, vbw[nj], go + 16, 0);
                    q[4] = u[0]; q[5] = u[1];
                } else if constexpr (B >= 8) {
#pragma unroll
                    for (int l = 1; l < B / 4; ++l) {
                        const u32x4_t u = __builtin_amdgcn_raw_buffer_load_b128(rb_rsrc, vbw[nj], go + 16 * l, 0);
                        q[4 * l] = u[0]; q[4 * l + 1] = u[1]; q[4 * l + 2] = u[2]; q[4 * l + 3] = u[3];
                    }
                }
            }
        }
    };
    // Fragments are 32 x 32 (v_mfma_f32_32x32x16_bf16): MR row blocks of 32 by kNJ column
    // blocks of 32 per wave. Lane l works on row / column l % 32 of a fragment and on K half
    // kh = l / 32: MFMA kk (0..3) of a stage takes the 8 K of chunk 4 kh + kk (8 K per chunk),
    // so a lane's B operands for the whole stage are the 4 consecutive words of the 16-byte
    // half kh of its weight row's stage segment, and its A operand for kk is the 16-byte
    // chunk 4 kh + kk of the activation row. Each output is still the sum over all K of the
    // stage.
    constexpr int MR = MF / 2;
    // the lane's scales of stage s, read from the ring
    // the lane's scales of one stage, as the dequantization takes them (converted once a stage):
    // affine s 2^24 (exact) and b; MXFP4 the e8m0 scale of the stage's 32-wide group kh, which
    // holds the lane's chunks 4 kh .. 4 kh + 3
    struct SReg {
        float s[kNJ], b[kNJ];
    };
    auto fetch_s = [&](SReg& f, int s) __attribute__((always_inline)) {
        // paired scales of an odd stage: the high halves of the previous (even) stage's slots
        const bool hi = spair && (s & 1);
        const int sh = hi ? 16 : 0;
        // per-stage copies: the slots of rows br in the stage's ring slot; the table: slot
        // br * pitch + unit of each array (a stage past the last reads the last unit)
        const uint8_t* ss = TBL ? tbl : ring + ((hi ? s - 1 : s) % NS) * SS + SA;
        const int unit = TBL ? min(spair ? s >> 1 : s >> gs, sp.nu - 1) : 0;
        const int rs = TBL ? sp.pitch : 1;          // slots between rows
        const int ab = TBL ? 256 * sp.pitch * 4 : 1024;   // bytes between the scale and bias arrays
#pragma unroll
        for (int nj = 0; nj < kNJ; ++nj) {
            const int br = brow[nj] * rs + unit;
            const uint32_t sv = (*reinterpret_cast<const uint32_t*>(ss + br * 4) >> sh) & 0xFFFFu;
            if constexpr (kAffine<MODE>) {
                const uint32_t bv = (*reinterpret_cast<const uint32_t*>(ss + ab + br * 4) >> sh) & 0xFFFFu;
                f.s[nj] = (F16 ? h2f(sv) : bf2f(sv)) * 16777216.0f;
                f.b[nj] = F16 ? h2f(bv) : bf2f(bv);
            } else if constexpr (!kScaled<MODE>) {
                f.s[nj] = f.b[nj] = 0.f;      // no scales: the slot read above is not used
            } else {
                f.s[nj] = e8m0_f32((sv >> (8 * kh)) & 0xFFu);
                f.b[nj] = 0.f;
            }
        }
    };
    // piece kk of the lane's stage half, dequantized into MFMA operands
    auto deq = [&](bf16x8_t (&bop)[kNJ], const BReg& bw, const SReg& f, int kk) __attribute__((always_inline)) {
#pragma unroll
        for (int nj = 0; nj < kNJ; ++nj) {
            const float sv = f.s[nj], bv = f.b[nj], sc = f.s[nj];
            bop[nj] = dq8<MODE>(bw.w[nj], kk, sv, bv, sc);
        }
    };

    f32x16_t acc[MR][kNJ];
#pragma unroll
    for (int i = 0; i < MR; ++i)
#pragma unroll
        for (int j = 0; j < kNJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // the A fragments of MFMA kk of stage s, read from the ring one K quarter ahead of their use
    auto lda = [&](int s, int kk, bf16x8_t (&af)[MR]) __attribute__((always_inline)) {
        const uint16_t* As = reinterpret_cast<const uint16_t*>(ring + (s % NS) * SS);
#pragma unroll
        for (int mi = 0; mi < MR; ++mi) {
            const int m = mi * 32 + l32;
            const int c = (4 * kh + kk) ^ a_key(m);
            af[mi] = *reinterpret_cast<const bf16x8_t*>(As + m * 64 + c * 8);
        }
    };
    auto mma = [&](const bf16x8_t (&af)[MR], const bf16x8_t (&bop)[kNJ]) __attribute__((always_inline)) {
#pragma unroll
        for (int mi = 0; mi < MR; ++mi)
#pragma unroll
            for (int nj = 0; nj < kNJ; ++nj)
                acc[mi][nj] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[mi], bop[nj], acc[mi][nj], 0, 0, 0);
    };

    // prologue: stages 0 .. NS - 2 in flight; wait for stages 0 and 1; B(0) kk 0 dequantized.
    // The B registers rotate through NS sets: stage t's words sit in set t % NS, so the loop
    // is unrolled NS times to keep every set index a constant.
    // (the empty asm with a memory clobber keeps each stage's copies into LDS after the previous
    // stage's: the wait counts them in issue order and the compiler cannot see their targets)
    if constexpr (TBL) {
        // the scale table: slot q = c * 256 + tid of copy c holds unit q % pitch of row
        // q / pitch (slot nu of an even nu is padding and repeats unit nu - 1); (r, u) advance by
        // 256 slots a copy
        const int pitch = sp.pitch, dr = 256 / pitch, du = 256 - dr * pitch;
        int r = tid / pitch, u = tid - r * pitch;
        uint8_t* const tb = tbl + 256 * pitch * 4;
        // the scale and bias arrays of rows 0..127 and 128..255 (gate / up for a gated expert),
        // read once as uniform values: indexing the layout by a per-lane matrix number would
        // read the kernel arguments per lane, a vector load the next copy would wait for
        const int plo = KIND == 0 ? 0 : 2, phi = KIND == 0 ? (mlp ? 0 : 1) : 2;
        const uint32_t s_lo = (uint32_t)L.p[plo].s, s_hi = (uint32_t)L.p[phi].s;
        const uint32_t b_lo = (uint32_t)L.p[plo].b, b_hi = (uint32_t)L.p[phi].b;
        for (int c = 0; c < pitch; ++c) {
            const bool up = r >= 128;
            const uint32_t vo = (uint32_t)mat_row(r) * (uint32_t)sp.rowbytes +
                                (uint32_t)min(u, sp.nu - 1) * (spair ? 4u : 2u);
            LDS_PTR ds = (LDS_PTR)(tbl + (c * 256 + wv * 64) * 4);
            LDS_PTR db = (LDS_PTR)(tb + (c * 256 + wv * 64) * 4);
            if (spair) {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rb_rsrc, ds, 4, vo + (up ? s_hi : s_lo), 0, 0, 0);
                if constexpr (kAffine<MODE>)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rb_rsrc, db, 4, vo + (up ? b_hi : b_lo), 0, 0, 0);
            } else {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rb_rsrc, ds, 2, vo + (up ? s_hi : s_lo), 0, 0, 0);
                if constexpr (kAffine<MODE>)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rb_rsrc, db, 2, vo + (up ? b_hi : b_lo), 0, 0, 0);
            }
            u += du;
            r += dr;
            if (u >= pitch) {
                u -= pitch;
                ++r;
            }
        }
        asm volatile("" ::: "memory");
    }
    bf16x8_t bop0[kNJ], bop1[kNJ];
    bf16x8_t a0[MR], a1[MR];
    SReg sc, sn;
    if constexpr (BPAIR) {
        // ---- B by stage pairs (32-row tiles of 4-bit codes): a load instruction reads 16 rows x
        // 64 contiguous bytes (lane L: row 16 h + L / 4 of the fragment, bytes [64 q + 16 (L % 4),
        // + 16) of stage pair q) instead of 32 rows x 32 bytes, and ds_bpermute hands each lane
        // the 16 bytes the MFMA operand layout gives it: stage 2q + t, half kh of row l32 is piece
        // 2 t + kh, in lane 4 (l32 % 16) + 2 t + kh of row half l32 / 16. The MFMA operands, and
        // so every output bit, are those of the per-stage loads. Pairs rotate through NPS
        // register sets; pair q is requested at stage 2q - 2 (NPS - 1), before that stage's A
        // copies.
        const int npairs = (nsteps + 1) / 2;
        struct PReg {
            u32x4_t w[kNJ][2];
        };
        uint32_t vbp[kNJ][2];
#pragma unroll
        for (int nj = 0; nj < kNJ; ++nj)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int fr = KIND == 0 ? nj * 128 + wv * 32 : wv * 64 + nj * 32;   // fragment's first row
                const int pj = KIND == 0 ? (mlp ? 0 : nj) : 2;
                vbp[nj][h] = (uint32_t)L.p[pj].w + (uint32_t)mat_row(fr + 16 * h + (lane >> 2)) * (uint32_t)(K / 2) +
                             (uint32_t)(lane & 3) * 16u;
            }
        auto issue_bp = [&](int q, PReg& pr) __attribute__((always_inline)) {
            const int qq = min(q, npairs - 1);
#pragma unroll
            for (int nj = 0; nj < kNJ; ++nj)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    pr.w[nj][h] = __builtin_amdgcn_raw_buffer_load_b128(rb_rsrc, vbp[nj][h], qq * 64, 0);
        };
        // the wave's pair goes through a 4 KB LDS area ([nj][row half][lane] x 16 bytes): written
        // once a pair, read back in the operand layout once a stage (same wave, in order)
        uint8_t* const bst = ring + kRing - kBPairLds + wv * (kBPairLds / kGemmWaves);
        // Load lane L = 4 r + c (row r of the half, piece c) sits in 16-byte slot L ^ (r >> 2) of
        // its 64: a stage's read (pieces c = 2 t + kh of rows r = 0..15) then touches 16
        // distinct slots mod 16, so neither the write nor the read has bank conflicts.
        auto stash = [&](const PReg& pr) __attribute__((always_inline)) {
            const int slot = lane ^ ((lane >> 4) & 3);
#pragma unroll
            for (int nj = 0; nj < kNJ; ++nj)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    *reinterpret_cast<u32x4_t*>(bst + ((nj * 2 + h) * 64 + slot) * 16) = pr.w[nj][h];
        };
        const int srow = ((l32 >> 4) * 64 + 4 * (l32 & 15)) * 16;   // row l32's four slots
        const int sx = (l32 & 15) >> 2;                              // their swizzle
        auto fetch_b = [&](int t, BReg& out) __attribute__((always_inline)) {
            const int so = srow + (((2 * t + kh) ^ sx) << 4);
#pragma unroll
            for (int nj = 0; nj < kNJ; ++nj) {
                const u32x4_t v = *reinterpret_cast<const u32x4_t*>(bst + nj * 2 * 64 * 16 + so);
#pragma unroll
                for (int w = 0; w < 4; ++w) out.w[nj][w] = v[w];
            }
        };
        constexpr int NVBP = kNJ * 2;   // loads of one pair
        constexpr int NPS = kBPairSets;
        PReg pq[NPS];
        BReg bs, bsn;
#pragma unroll
        for (int q = 0; q < NPS - 1; ++q) issue_bp(q, pq[q]);
#pragma unroll
        for (int t = 0; t < NS - 1; ++t) {
            issue_a(t);
            asm volatile("" ::: "memory");
        }
        dma_wait_barrier<NVA0>();   // stages 0 and 1: only stage 2's copies follow theirs
        fetch_s(sc, 0);
        stash(pq[0]);
        fetch_b(0, bs);
        deq(bop0, bs, sc, 0);
        lda(0, 0, a0);
        for (int s0 = 0; s0 < nsteps; s0 += 2 * NPS) {
#pragma unroll
            for (int u = 0; u < 2 * NPS; ++u) {
                const int s = s0 + u;
                if (s >= nsteps) break;
                // stage s + 1's copies landed in every wave: after them come iteration s - 1's
                // (B of pair (s - 1) / 2 + NPS - 1 when s - 1 is even, then A of stage s + 2), as
                // far as they were issued
                if (s + 2 < nsteps) {
                    if (u & 1) {
                        if ((s - 1) / 2 + NPS - 1 < npairs) dma_wait_barrier<NVBP + NVA1>();
                        else dma_wait_barrier<NVA1>();
                    } else {
                        dma_wait_barrier<NVA0>();
                    }
                } else {
                    dma_wait_barrier<0>();
                }
                if (!(u & 1) && s / 2 + NPS - 1 < npairs)
                    issue_bp(s / 2 + NPS - 1, pq[((u >> 1) + NPS - 1) % NPS]);
                if (s + NS - 1 < nsteps) issue_a(s + NS - 1);
                fetch_s(sn, s + 1);
                lda(s, 1, a1);
                mma(a0, bop0);
                deq(bop1, bs, sc, 1);
                lda(s, 2, a0);
                mma(a1, bop1);
                deq(bop0, bs, sc, 2);
                lda(s, 3, a1);
                mma(a0, bop0);
                deq(bop1, bs, sc, 3);
                lda(min(s + 1, nsteps - 1), 0, a0);
                mma(a1, bop1);
                if (u & 1) stash(pq[((u + 1) >> 1) % NPS]);   // stage s + 1 starts a pair
                fetch_b((u + 1) & 1, bsn);
                deq(bop0, bsn, sn, 0);
                bs = bsn;
                sc = sn;
            }
        }
    } else {
    BReg bq[NS];
#pragma unroll
    for (int t = 0; t < NS - 1; ++t) {
        issue_a(t);
        issue_b(t, bq[t]);
        asm volatile("" ::: "memory");
    }
    dma_wait_barrier<loads_after(NS, NV0, NV1, 0)>();
    fetch_s(sc, 0);
    deq(bop0, bq[0], sc, 0);
    lda(0, 0, a0);
    for (int s0 = 0; s0 < nsteps; s0 += NS) {
#pragma unroll
        for (int u = 0; u < NS; ++u) {
            const int s = s0 + u;
            if (s >= nsteps) break;
            // stage s + 1 landed in every wave; stage s - 1's slot and registers are free for
            // stage s + NS - 1 (NS is even, so s and u have the same parity). No stage past the
            // last is loaded: near the end fewer loads follow stage s + 1's, so the wait counts
            // only those issued (all of stage s + NS - 2's once it exists, else none).
            static_assert(NS == 4, "the tail waits below count the loads of one later stage");
            if (s + NS - 2 < nsteps) {
                if (u & 1)
                    dma_wait_barrier<loads_after(NS, NV0, NV1, 1)>();
                else
                    dma_wait_barrier<loads_after(NS, NV0, NV1, 0)>();
            } else {
                dma_wait_barrier<0>();
            }
            if (s + NS - 1 < nsteps) {
                issue_a(s + NS - 1);
                issue_b(s + NS - 1, bq[(u + NS - 1) % NS]);
            }
            fetch_s(sn, s + 1);
            lda(s, 1, a1);
            mma(a0, bop0);
            deq(bop1, bq[u], sc, 1);
            lda(s, 2, a0);
            mma(a1, bop1);
            deq(bop0, bq[u], sc, 2);
            lda(s, 3, a1);
            mma(a0, bop0);
            deq(bop1, bq[u], sc, 3);
            lda(min(s + 1, nsteps - 1), 0, a0);   // stage s + 1 landed at the top of this one
            mma(a1, bop1);
            deq(bop0, bq[(u + 1) % NS], sn, 0);
            sc = sn;
        }
    }
    }

    // ---- epilogue: the output tile goes through LDS (the ring, once every copy into it has
    // landed and every wave is done reading it) so that the global stores are 16-byte chunks
    // of contiguous row segments
    dma_wait_barrier<0>();
    pf_store<KIND, MR>(a, L, base, mlp, inter, slot, nt, m0, rows, acc, ring, dst_s, hbuf, hstride, y_routed,
                       y_shared);
}

template <int MODE, bool F16, int KIND>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void k_pf_gemm(FwdArgs a, const int32_t* __restrict__ order, const int32_t* __restrict__ tile_start,
               const int4* __restrict__ tinfo, int E_ext, int ntn, uint16_t* __restrict__ hbuf,
               int hstride, uint16_t* __restrict__ y_routed, uint16_t* __restrict__ y_shared) {
    __shared__ __attribute__((aligned(16))) uint8_t ring[kRing];
    __shared__ int32_t dst_s[KIND == 1 ? kBM : 1];
    const int blk = blockIdx.x;
    const int loc = blk / kXcd;
    const int nt = loc % ntn;
    const int mt = (loc / ntn) * kXcd + blk % kXcd;
    const int total = tile_start[E_ext];
    const int4 ti = tinfo[mt];
    if (mt >= total) return;
    const int e = ti.x, m0 = ti.y, rows = ti.z;
    if (KIND == 0) {
        const int inter = e >= a.E ? a.I_sh : a.I;
        if (nt * (a.act == BRX_ACT_SILU_MLP ? kBlockN : kBlockN / 2) >= inter) return;
    } else {
        if (nt * kBlockN >= a.H) return;
    }
    // A tile reads its scales from a table copied once per tile when the table fits beside its
    // A ring (gpt-oss's 512-token prefill 800 -> 615 us per layer, the Qwen3-shape gate/up
    // 168 -> 160 us); otherwise (128-row tiles of wide K) each stage's scales come with the stage.
    const bool sh = e >= a.E;
    const int K = KIND == 0 ? a.H : (sh ? a.I_sh : a.I);
    const ScalePlan sp = scale_plan<MODE, KIND>(a, sh ? a.lay_sh : a.lay, K, KIND == 0 && a.act == BRX_ACT_SILU_MLP);
#define BRX_TILE(MF, TBL) \
    pf_tile<MODE, F16, KIND, MF, TBL>(a, order, hbuf, hstride, y_routed, y_shared, ring, dst_s, e, m0, rows, ti.w, nt)
    if constexpr (!kScaled<MODE>) {       // bf16 weights: no scales to copy
        if (rows <= 32) BRX_TILE(2, false);
        else BRX_TILE(4, false);
    } else if (rows <= 32) {
        // (32-row tiles of 4-bit codes also keep kBPairLds for their paired B loads)
        constexpr int stage_b = kBW<MODE> == 4 ? kBPairLds : 0;
        if (tile_lds<MODE>(2, true, sp.pitch) + stage_b <= kRing) BRX_TILE(2, true);
        else BRX_TILE(2, false);
    } else if (kTileRows<MODE> == 64 || rows <= 64) {
        if (tile_lds<MODE>(4, true, sp.pitch) <= kRing) BRX_TILE(4, true);
        else BRX_TILE(4, false);
    } else if constexpr (kTileRows<MODE> == 128) {
        if (tile_lds<MODE>(8, true, sp.pitch) <= kRing) BRX_TILE(8, true);
        else BRX_TILE(8, false);
    }
#undef BRX_TILE
}

// ------------------------------------------------------------------ combine
// V consecutive outputs of one token per thread (V = 8: 16-byte loads and stores, every
// expert row's load issued before the sums; V = 2 when a pointer is not 16-byte aligned). Each
// output is fma(w[t, j], y[t, j], acc) over j = 0 .. k - 1 in order, then the shared term,
// whatever V is.
template <int V>
__global__ __launch_bounds__(kThreads) void k_combine(const uint16_t* __restrict__ y_routed,
                                                      const uint16_t* __restrict__ y_shared,
                                                      const float* __restrict__ w,
                                                      const float* __restrict__ sg, int T, int k,
                                                      int H, uint16_t* __restrict__ out) {
    using VT = typename std::conditional<V == 8, uint4, uint32_t>::type;
    constexpr int NW = V / 2;                      // 32-bit words per thread
    constexpr int KB = 8;                          // expert rows in flight per thread
    const int t = blockIdx.y;
    const int n = (blockIdx.x * kThreads + threadIdx.x) * V;
    if (n >= H) return;
    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.f;
    auto add = [&](float wj, const VT& v) __attribute__((always_inline)) {
        const uint32_t* q = reinterpret_cast<const uint32_t*>(&v);
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            acc[2 * i] = fmaf(wj, bf2f(q[i] & 0xFFFFu), acc[2 * i]);
            acc[2 * i + 1] = fmaf(wj, bf2f(q[i] >> 16), acc[2 * i + 1]);
        }
    };
    // the shared expert's row and gate are requested with the first routed rows (it is added
    // last, in the same order as before, but its round trip is not a second one)
    // (the load is unconditional -- from routed row 0 when there is no shared expert, and then
    // unused -- so no branch holds it back)
    const bool has_sh = y_shared && sg;   // uniform
    const uint16_t* shrow = has_sh ? y_shared + (int64_t)t * H + n : y_routed + (int64_t)t * k * H + n;
    const VT vsh = *reinterpret_cast<const VT*>(shrow);
    const float wsh = has_sh ? sg[t] : 0.f;
    auto batch = [&](int j0) __attribute__((always_inline)) {
        VT v[KB];
        float wj[KB];
#pragma unroll
        for (int u = 0; u < KB; ++u) {
            const int j = min(j0 + u, k - 1);
            v[u] = *reinterpret_cast<const VT*>(y_routed + ((int64_t)t * k + j) * H + n);
            wj[u] = w[t * k + j];
        }
#pragma unroll
        for (int u = 0; u < KB; ++u)
            if (j0 + u < k) add(wj[u], v[u]);
    };
    // the first KB rows outside the loop: straight-line code after the shared row's load, so
    // nothing makes them wait for it
    batch(0);
    for (int j0 = KB; j0 < k; j0 += KB) batch(j0);
    if (has_sh) add(wsh, vsh);
    uint32_t o[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) o[i] = f2bf(acc[2 * i]) | (f2bf(acc[2 * i + 1]) << 16);
    *reinterpret_cast<VT*>(out + (int64_t)t * H + n) = *reinterpret_cast<const VT*>(o);
}

struct PfWs {
    int32_t* order;
    int32_t* offsets;
    int32_t* tile_start;
    int4* tinfo;
    uint16_t* hbuf;
    uint16_t* y_routed;
    uint16_t* y_shared;
    int mt_pad;                 // M tiles the grids cover (a multiple of kXcd)
    size_t bytes;
};

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// The M tile height of a kernel mode (kTileRows on the host).
inline int tile_rows(int mode) {
    return mode == kModeAffine6 || mode == kModeAffine8 || mode == kModeBf16 ? 64 : kBM;
}

PfWs carve(const FwdArgs& a, void* ws) {
    const int P = a.P;
    const int T_sh = a.auto_shared ? a.T : 0;
    const int P_ext = P + T_sh;
    const int E_ext = a.E + (a.shared ? 1 : 0);
    const int Imax = a.I > a.I_sh ? a.I : a.I_sh;
    // at most ceil(P_ext / BM) full tiles plus one partial tile per expert
    const int BM = tile_rows(a.quant_mode);
    const int mt_max = (P_ext + BM - 1) / BM + E_ext;
    PfWs w{};
    w.mt_pad = (mt_max + kXcd - 1) / kXcd * kXcd;
    size_t off = 0;
    char* b = reinterpret_cast<char*>(ws);
    w.order = reinterpret_cast<int32_t*>(b + off); off = align256(off + sizeof(int32_t) * P_ext);
    w.offsets = reinterpret_cast<int32_t*>(b + off); off = align256(off + sizeof(int32_t) * (E_ext + 1));
    w.tile_start = reinterpret_cast<int32_t*>(b + off); off = align256(off + sizeof(int32_t) * (E_ext + 1));
    w.tinfo = reinterpret_cast<int4*>(b + off); off = align256(off + sizeof(int4) * w.mt_pad);
    w.hbuf = reinterpret_cast<uint16_t*>(b + off); off = align256(off + 2ull * P_ext * Imax);
    w.y_routed = reinterpret_cast<uint16_t*>(b + off); off = align256(off + 2ull * P * a.H);
    w.y_shared = reinterpret_cast<uint16_t*>(b + off); off = align256(off + 2ull * T_sh * a.H);
    w.bytes = off;
    return w;
}

template <int MODE, bool F16>
hipError_t launch_gemm(const FwdArgs& a, const PfWs& w, int E_ext, int Imax, uint16_t* y_routed,
                       int phases, hipStream_t s) {
    if (phases & 1) {
        const int fpb = a.act == BRX_ACT_SILU_MLP ? kBlockN : kBlockN / 2;   // features per block
        const int ntn = (Imax + fpb - 1) / fpb;
        hipLaunchKernelGGL((k_pf_gemm<MODE, F16, 0>), dim3(w.mt_pad * ntn), dim3(kGemmThreads), 0, s,
                           a, w.order, w.tile_start, w.tinfo, E_ext, ntn, w.hbuf, Imax, y_routed, w.y_shared);
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
    }
    if (phases & 2) {
        const int ntn = (a.H + kBlockN - 1) / kBlockN;
        hipLaunchKernelGGL((k_pf_gemm<MODE, F16, 1>), dim3(w.mt_pad * ntn), dim3(kGemmThreads), 0, s,
                           a, w.order, w.tile_start, w.tinfo, E_ext, ntn, w.hbuf, Imax, y_routed, w.y_shared);
        return hipGetLastError();
    }
    return hipSuccess;
}

hipError_t launch_bucket(const int32_t* pexp, int P, int E, int E_ext, int T_sh, int BM,
                         const int32_t* g2s, int capacity, int host, int32_t* err, int32_t* order,
                         int32_t* offsets, int32_t* tile_start, int4* tinfo, hipStream_t s) {
    // each block lists its expert's pairs in LDS during the histogram pass, up to lcap of them;
    // an expert with more takes a second pass over the pairs
    const int P_ext = P + T_sh;
    const int lcap = P_ext < kBucketListMax ? P_ext : kBucketListMax;
    hipLaunchKernelGGL(k_bucket, dim3(E_ext), dim3(kBucketThreads), sizeof(int32_t) * (E_ext + lcap), s, pexp, P,
                       E, E_ext, T_sh, BM, g2s, capacity, host, err, order, offsets, tile_start, tinfo, lcap);
    return hipGetLastError();
}

}  // namespace

size_t prefill_workspace_bytes(const FwdArgs& a) { return carve(a, nullptr).bytes; }

hipError_t launch_sort_pairs(const int32_t* pexp, int P, int E, int E_ext, int T_sh, int BM,
                             int32_t* order, int32_t* offsets, int32_t* tile_start, hipStream_t s) {
    return launch_bucket(pexp, P, E, E_ext, T_sh, BM, nullptr, 1, 0, nullptr, order, offsets, tile_start, nullptr,
                         s);
}

hipError_t launch_combine(const uint16_t* y_routed, const uint16_t* y_shared, const float* w,
                          const float* sg, int T, int k, int H, uint16_t* out, hipStream_t s) {
    // H is a multiple of 64, so 8 outputs a thread tile every row
    if ((((uintptr_t)y_routed | (uintptr_t)y_shared | (uintptr_t)out) & 15) == 0)
        hipLaunchKernelGGL(k_combine<8>, dim3((H / 8 + kThreads - 1) / kThreads, T), dim3(kThreads), 0, s,
                           y_routed, y_shared, w, sg, T, k, H, out);
    else
        hipLaunchKernelGGL(k_combine<2>, dim3((H / 2 + kThreads - 1) / kThreads, T), dim3(kThreads), 0, s,
                           y_routed, y_shared, w, sg, T, k, H, out);
    return hipGetLastError();
}

hipError_t launch_prefill(const FwdArgs& a, void* ws, size_t ws_bytes, int phases, hipStream_t s) {
    PfWs w = carve(a, ws);
    if (w.bytes > ws_bytes) return hipErrorInvalidValue;
    const int P = a.P;
    const int T_sh = a.auto_shared ? a.T : 0;
    const int E_ext = a.E + (a.shared ? 1 : 0);
    const int Imax = a.I > a.I_sh ? a.I : a.I_sh;
    // the GEMMs address activations and h rows with 32-bit buffer offsets
    if ((int64_t)a.T * a.H * 2 >= (int64_t)1 << 32 || (int64_t)(P + T_sh) * Imax * 2 >= (int64_t)1 << 32)
        return hipErrorInvalidValue;
    uint16_t* y_routed = a.yun ? a.yun : w.y_routed;
    hipError_t err = hipSuccess;
    if (phases & 1) {
        err = launch_bucket(a.pexp, P, a.E, E_ext, T_sh, tile_rows(a.quant_mode), a.g2s, a.capacity, a.host != nullptr, a.err, w.order, w.offsets,
                            w.tile_start, w.tinfo, s);
        if (err != hipSuccess) return err;
    }
#define BRX_GEMM(M) (a.scale_f16 ? launch_gemm<M, true>(a, w, E_ext, Imax, y_routed, phases, s) \
                                 : launch_gemm<M, false>(a, w, E_ext, Imax, y_routed, phases, s))
    switch (a.quant_mode) {
        case kModeAffine4: err = BRX_GEMM(kModeAffine4); break;
        case kModeAffine3: err = BRX_GEMM(kModeAffine3); break;
        case kModeAffine2: err = BRX_GEMM(kModeAffine2); break;
        case kModeAffine6: err = BRX_GEMM(kModeAffine6); break;
        case kModeAffine8: err = BRX_GEMM(kModeAffine8); break;
        case BRX_QUANT_MXFP4: err = launch_gemm<BRX_QUANT_MXFP4, false>(a, w, E_ext, Imax, y_routed, phases, s); break;
        case kModeBf16: err = launch_gemm<kModeBf16, false>(a, w, E_ext, Imax, y_routed, phases, s); break;
        default: err = hipErrorInvalidValue;
    }
#undef BRX_GEMM
    if (err != hipSuccess) return err;
    if ((phases & 2) && a.out)
        err = launch_combine(y_routed, a.auto_shared ? w.y_shared : nullptr, a.w, a.sgate, a.T, a.k,
                             a.H, a.out, s);
    return err;
}

}  // namespace brx
