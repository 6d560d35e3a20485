// fpa_fwd16.hip -- the forward kernel of First Passage Attention (fpa_fwd.h) for fp16 operands.
#include "fpa_fwd.h"

namespace fpa {

hipError_t launch_fwd_f16(const FwdParams &p, int D, hipStream_t s) {
    switch (D) {
        case 16: return launch_fwd_t<f16, 16>(p, s);
        case 32: return launch_fwd_t<f16, 32>(p, s);
        case 64: return launch_fwd_t<f16, 64>(p, s);
        case 128: return launch_fwd_t<f16, 128>(p, s);
        case 256: return launch_fwd_t<f16, 256>(p, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_fwd_merge_f16(const FwdParams &p, int D, hipStream_t s) {
    switch (D) {
        case 16: return launch_fwd_merge_t<f16, 16>(p, s);
        case 32: return launch_fwd_merge_t<f16, 32>(p, s);
        case 64: return launch_fwd_merge_t<f16, 64>(p, s);
        case 128: return launch_fwd_merge_t<f16, 128>(p, s);
        case 256: return launch_fwd_merge_t<f16, 256>(p, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace fpa
