// fpa_bwd_fused.hip -- the key-side and query-side backward tiles in one launch.
//
// Reference behaviour: _bwd_kv (kernel.py:177-265) and _bwd_q (kernel.py:286-340) of
// yliu-fort/first-passage-attention, which run as two launches there.  The two sides depend
// on the per-query preparation only, not on each other.  Their work is triangular (key tiles
// near 0 and query tiles near T cover the most blocks), so a launch of either side alone
// ends with the chip partly idle while its longest workgroups finish.  One grid holding both
// kinds of workgroup, ordered longest first by an estimate of their cost, keeps every CU busy
// to the end.  Each workgroup computes exactly what it computes in the separate kernels.
#include <algorithm>

#include "fpa_bwd_kv.h"
#include "fpa_bwd_q.h"

// Relative cost of one block iteration of the key side and of the query side, for the order
// of the fused grid (measured alone at D = 64 fp16: about 1.2; the fused launch is fastest with
// weights 5:4 to 6:5, 1% ahead of 3:2 and 4% ahead of 1:1 at cfg2, level at cfg4).
#ifndef FPA_FUSE_WKV
#define FPA_FUSE_WKV 5
#endif
#ifndef FPA_FUSE_WQ
#define FPA_FUSE_WQ 4
#endif

namespace fpa {

// Workgroup slots of the fused grid (per head): key tiles and query tiles together.
constexpr int FUSED_MAX = 1024;

// Slot -> tile: a key tile index, or a query tile index with bit 15 set.  Passed by value
// (2 KB of kernel arguments); the index is uniform, so each workgroup reads one entry with a
// scalar load.
struct BwdOrder {
    uint16_t e[FUSED_MAX];
};

template <typename T, int D, int NW>
union BwdShared {
    KvShared<T, D, NW> kv;
    QShared<T, D, NW> q;
};

template <typename T, int D, int WPE, int NW>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
fpa_bwd_kvq_kernel(BwdParams p, BwdOrder ord) {
    __shared__ BwdShared<T, D, NW> sm;
    int slot, bh;
    xcd_work_item(slot, bh, p.BH, p.H, 2 * ((p.T + 32 * NW - 1) / (32 * NW)));
    const int e = __builtin_amdgcn_readfirstlane((int)ord.e[slot]);
    if (e & 0x8000)
        bwd_q_tile<T, D, NW>(p, sm.q, e & 0x7fff, bh);
    else
        bwd_kv_tile<T, D, NW>(p, sm.kv, e, bh);
}

template <typename T, int D>
static hipError_t launch_kvq_t(const BwdParams &p, hipStream_t s) {
    constexpr int NW = FPA_NW, BT = 32 * NW, WPE = kv_wpe<T, D>();
    const int nt = (p.T + BT - 1) / BT;  // key tiles; as many query tiles
    auto two_launches = [&]() {
        hipError_t e = launch_bwd_kv(p, sizeof(T) == 2 ? 0 : 1, D, s);
        return e != hipSuccess ? e : launch_bwd_q(p, sizeof(T) == 2 ? 0 : 1, D, s);
    };
    // No common launch shape, or (fp32 at D = 64, one wave per SIMD) two launches measured 2% faster.
    if constexpr (WPE != q_wpe<T, D>() || kv_parts<T, D>() > 1 || (sizeof(T) == 4 && D == 64)) {
        return two_launches();
    } else {
        if (2 * nt > FUSED_MAX) return two_launches();
        // Block iterations of key tile kt (query blocks from its diagonal block to the end) and of
        // query tile qt (key blocks from its diagonal block down to 0), weighted by their cost.
        auto c_kv = [&](int kt) { return FPA_FUSE_WKV * (p.NB - kt * BT / G); };
        auto c_q = [&](int qt) { return FPA_FUSE_WQ * (std::min(p.NB - 1, (qt * BT + BT - 1) / G) + 1); };
        BwdOrder ord;
        int n = 0;
        for (int kt = 0, qt = nt - 1; kt < nt || qt >= 0;) {  // merge, costliest first
            if (qt < 0 || (kt < nt && c_kv(kt) >= c_q(qt)))
                ord.e[n++] = (uint16_t)kt++;
            else
                ord.e[n++] = (uint16_t)(0x8000 | qt--);
        }
        hipLaunchKernelGGL((fpa_bwd_kvq_kernel<T, D, WPE, NW>), head_grid(2 * nt, p.H, p.BH), dim3(64 * NW), 0, s, p,
                           ord);
        return hipGetLastError();
    }
}

hipError_t launch_bwd_kvq(const BwdParams &p, int dtype, int D, hipStream_t s) {
    if (dtype == 0) {
        switch (D) {
            case 16: return launch_kvq_t<f16, 16>(p, s);
            case 32: return launch_kvq_t<f16, 32>(p, s);
            case 64: return launch_kvq_t<f16, 64>(p, s);
            case 128: return launch_kvq_t<f16, 128>(p, s);
            case 256: return launch_kvq_t<f16, 256>(p, s);
        }
    } else {
        switch (D) {
            case 16: return launch_kvq_t<float, 16>(p, s);
            case 32: return launch_kvq_t<float, 32>(p, s);
            case 64: return launch_kvq_t<float, 64>(p, s);
            case 128: return launch_kvq_t<float, 128>(p, s);
            case 256: return launch_kvq_t<float, 256>(p, s);
        }
    }
    return hipErrorInvalidValue;
}

}  // namespace fpa
