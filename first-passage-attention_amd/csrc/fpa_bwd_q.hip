// fpa_bwd_q.hip -- the query-side kernel of the backward.
//
// Reference behaviour: _bwd_q (kernel.py:286-340) of yliu-fort/first-passage-attention.
// The query-side tile itself is in fpa_bwd_q.h.
#include "fpa_bwd_q.h"

namespace fpa {

template <typename T, int D, int WPE, int NW>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
fpa_bwd_q_kernel(BwdParams p) {
    __shared__ QShared<T, D, NW> sm;
    const int nqt = (p.T + 32 * NW - 1) / (32 * NW);
    int rank, bh;
    xcd_work_item(rank, bh, p.BH, p.H, nqt);
    bwd_q_tile<T, D, NW>(p, sm, nqt - 1 - rank, bh);  // rank 0: the longest rows
}

template <typename T, int D>
static hipError_t launch_q_t(const BwdParams &p, hipStream_t s) {
    constexpr int NW = FPA_NW;
    const int nqt = (p.T + 32 * NW - 1) / (32 * NW);
    constexpr int WPE = q_wpe<T, D>();
    hipLaunchKernelGGL((fpa_bwd_q_kernel<T, D, WPE, NW>), head_grid(nqt, p.H, p.BH), dim3(64 * NW), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_bwd_q(const BwdParams &p, int dtype, int D, hipStream_t s) {
    if (dtype == 0) {
        switch (D) {
            case 16: return launch_q_t<f16, 16>(p, s);
            case 32: return launch_q_t<f16, 32>(p, s);
            case 64: return launch_q_t<f16, 64>(p, s);
            case 128: return launch_q_t<f16, 128>(p, s);
            case 256: return launch_q_t<f16, 256>(p, s);
        }
    } else {
        switch (D) {
            case 16: return launch_q_t<float, 16>(p, s);
            case 32: return launch_q_t<float, 32>(p, s);
            case 64: return launch_q_t<float, 64>(p, s);
            case 128: return launch_q_t<float, 128>(p, s);
            case 256: return launch_q_t<float, 256>(p, s);
        }
    }
    return hipErrorInvalidValue;
}

}  // namespace fpa
