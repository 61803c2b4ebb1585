// Decode launches for 4-bit affine, MXFP4 and 3-bit affine weights, and the dispatch over every
// weight mode (2-, 6- and 8-bit affine and bf16 weights are compiled in k_decode_wide.hip).
#include "dec_kernels.h"

namespace brx {

size_t decode_workspace_bytes(const FwdArgs& a) { return dec_carve(a, nullptr).bytes; }

hipError_t launch_decode(const FwdArgs& a, void* ws, int phases, hipStream_t s) {
    const DecWs w = dec_carve(a, ws);
    switch (a.quant_mode) {
        case kModeAffine4:
            return launch_mode<kModeAffine4>(a, w.hbuf, w.table, w.y_routed, w.y_shared, phases, s);
        case BRX_QUANT_MXFP4:
            return launch_mode<BRX_QUANT_MXFP4>(a, w.hbuf, w.table, w.y_routed, w.y_shared, phases, s);
        case kModeAffine3:
            return launch_mode<kModeAffine3>(a, w.hbuf, w.table, w.y_routed, w.y_shared, phases, s);
        default:
            return launch_decode_wide(a, ws, phases, s);
    }
}

}  // namespace brx
