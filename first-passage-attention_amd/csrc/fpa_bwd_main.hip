// fpa_bwd_main.hip -- the single-pass backward kernel (fp16, D <= 64); the tile is in fpa_bwd_main.h.
//
// Reference behaviour: _bwd_kv (kernel.py:177-265) and _bwd_q (kernel.py:286-340) of
// yliu-fort/first-passage-attention, in one pass over the causal pairs.
#include "fpa_bwd_main.h"

namespace fpa {

static_assert(MAIN_NW * 32 == MAIN_BK, "keys per workgroup");

template <int D, int NW>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2)))
fpa_bwd_main_kernel(BwdParams p) {
    __shared__ MainShared<D, NW> sm;
    int rank, bh;
    xcd_work_item(rank, bh, p.BH, p.nkt);
    bwd_main_tile<D, NW>(p, sm, rank, bh);  // rank 0: key tile 0, the one with the most query blocks
}

template <int D>
static hipError_t launch_main_t(const BwdParams &p, hipStream_t s) {
    hipLaunchKernelGGL((fpa_bwd_main_kernel<D, MAIN_NW>), dim3(p.nkt, p.BH), dim3(64 * MAIN_NW), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_bwd_main(const BwdParams &p, int dtype, int D, hipStream_t s) {
    if (dtype != 0 || p.nkt < 1) return hipErrorInvalidValue;
    switch (D) {
        case 16: return launch_main_t<16>(p, s);
        case 32: return launch_main_t<32>(p, s);
        case 64: return launch_main_t<64>(p, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace fpa
