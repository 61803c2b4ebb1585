// Decode launches for 2-, 6- and 8-bit affine and unquantized bf16 weights (the kernels of
// dec_kernels.h; a translation unit of its own so the modes compile in parallel).
#include "dec_kernels.h"

namespace brx {

hipError_t launch_decode_wide(const FwdArgs& a, void* ws, int phases, hipStream_t s) {
    const DecWs w = dec_carve(a, ws);
    switch (a.quant_mode) {
        case kModeAffine2:
            return launch_mode<kModeAffine2>(a, w.hbuf, w.table, w.y_routed, w.y_shared, phases, s);
        case kModeAffine6:
            return launch_mode<kModeAffine6>(a, w.hbuf, w.table, w.y_routed, w.y_shared, phases, s);
        case kModeAffine8:
            return launch_mode<kModeAffine8>(a, w.hbuf, w.table, w.y_routed, w.y_shared, phases, s);
        case kModeBf16:
            return launch_mode<kModeBf16>(a, w.hbuf, w.table, w.y_routed, w.y_shared, phases, s);
        default:
            return hipErrorInvalidValue;
    }
}

}  // namespace brx
