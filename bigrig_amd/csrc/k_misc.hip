// fp32 dequantization of one projection (test hook; replaces mx.dequantize,
// bigrig_engine/precision.py:186-189). w = s*q + b for affine (s*q exact in fp32, one
// rounding), w = e2m1(q) * 2^(e-127) for mxfp4, the bf16 weight for unquantized experts.
#include "brx_internal.h"

namespace brx {
namespace {

// Code k of a row sits at bits [bits k, bits k + bits) of the row's bytes, least significant
// bit first (a 3- or 6-bit code may straddle two bytes); affine scale groups hold `group` codes.
template <int MODE>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t* __restrict__ base, Proj P,
                                                 int scale_f16, int bits, int group,
                                                 float* __restrict__ out) {
    const int row = blockIdx.x;
    const int n_in = P.n_in;
    const uint8_t* wrow = base + P.w + (int64_t)row * (n_in * bits / 8);
    if constexpr (MODE == BRX_QUANT_NONE) {    // unquantized: the bf16 weights themselves
        for (int k = threadIdx.x; k < n_in; k += blockDim.x)
            out[(int64_t)row * n_in + k] = bf2f(reinterpret_cast<const uint16_t*>(wrow)[k]);
        return;
    }
    for (int k = threadIdx.x; k < n_in; k += blockDim.x) {
        const int bit = k * bits;
        uint32_t two = wrow[bit >> 3];
        if ((bit & 7) + bits > 8) two |= (uint32_t)wrow[(bit >> 3) + 1] << 8;
        const uint32_t q = (two >> (bit & 7)) & ((1u << bits) - 1u);
        float v;
        if constexpr (MODE == BRX_QUANT_AFFINE) {
            const int G = n_in / group;
            float s = load_scale(base + P.s, (int64_t)row * G + k / group, scale_f16);
            float b = load_scale(base + P.b, (int64_t)row * G + k / group, scale_f16);
            v = fmaf(s, (float)q, b);
        } else {
            const int G = n_in / 32;
            v = e2m1_f32(q) * e8m0_f32(base[P.s + (int64_t)row * G + k / 32]);
        }
        out[(int64_t)row * n_in + k] = v;
    }
}

// A batch of expert-table entries set in stream order (the values travel as kernel arguments,
// so nothing on the host has to outlive the call). Entries are distinct.
__global__ __launch_bounds__(64) void k_table_set(int32_t* __restrict__ g2s, TableEdits ed) {
    const int i = threadIdx.x;
    if (i < ed.n) g2s[ed.e[i]] = ed.v[i];
}

}  // namespace

hipError_t launch_table_set(int32_t* g2s, const TableEdits& ed, hipStream_t s) {
    hipLaunchKernelGGL(k_table_set, dim3(1), dim3(64), 0, s, g2s, ed);
    return hipGetLastError();
}

hipError_t launch_dequant(const brx_layer_desc& d, const Layout& L, const uint8_t* expert,
                          int proj, float* out, hipStream_t s) {
    const Proj& P = L.p[proj];
    if (d.quant_mode == BRX_QUANT_AFFINE)
        hipLaunchKernelGGL(k_dequant<BRX_QUANT_AFFINE>, dim3(P.n_out), dim3(256), 0, s, expert, P,
                           d.scale_dtype == BRX_SCALE_F16 ? 1 : 0, d.bits, d.group_size, out);
    else if (d.quant_mode == BRX_QUANT_NONE)
        hipLaunchKernelGGL(k_dequant<BRX_QUANT_NONE>, dim3(P.n_out), dim3(256), 0, s, expert, P, 0,
                           16, 0, out);
    else
        hipLaunchKernelGGL(k_dequant<BRX_QUANT_MXFP4>, dim3(P.n_out), dim3(256), 0, s, expert, P, 0,
                           4, 32, out);
    return hipGetLastError();
}

}  // namespace brx
