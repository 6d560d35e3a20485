// fpa_bwd_kv.hip -- per-query preparation and the key-side kernel of the backward.
//
// Reference behaviour: _bwd_delta (kernel.py:165-174) and _bwd_kv (kernel.py:177-265)
// of yliu-fort/first-passage-attention.  The key-side tile itself is in fpa_bwd_kv.h.
#include "fpa_bwd_kv.h"

namespace fpa {

template <typename T, int D>
__global__ void __launch_bounds__(NTHREADS) fpa_bwd_prep_kernel(BwdParams p) {
    constexpr int CE = MT<T>::CHUNK;
    constexpr int CPR = (D + CE - 1) / CE;
    const int bh = group_bh(p.H), b = bh / p.H, h = bh % p.H;
    const int row = group_x() * 64 + thread_x() / 4, part = thread_x() % 4;
    const StateLayout L{p.BH, p.TP, p.NB};
    const bool ok = row < p.T;
    // The row's statistics first: their loads overlap those of O and dO below.
    constexpr bool XB = exact_bias<T>();
    float blse = 0.f, prel0 = 0.f, prel = 0.f, pre = pinf(), bmin = 0.f, lse = 0.f, lsl = 0.f;
    const bool writer = part == 0 && row < p.TP;
    if (writer) {
        blse = p.state[L.bplane(BP_LSE) + (int64_t)bh * p.NB + row / G];
        prel0 = p.state[L.at(PL_PREL, bh, (row / G) * G)];
        if (ok) {
            prel = p.state[L.at(PL_PREL, bh, row)];
            pre = p.state[L.at(PL_PRE, bh, row)];
            lse = p.lse[(int64_t)bh * p.TP + row];
            if constexpr (XB) lsl = p.lse[((int64_t)p.BH + bh) * p.TP + row];
        }
        if (row % G == 0) bmin = p.state[L.bplane(BP_MIN) + (int64_t)bh * p.NB + row / G];
    }
    float acc = 0.f;
    if (ok) {
        const T *Or = static_cast<const T *>(p.o) + b * p.so.b + h * p.so.h + (int64_t)row * p.so.t;
        const T *Dr = static_cast<const T *>(p.dout) + b * p.sdo.b + h * p.sdo.h + (int64_t)row * p.sdo.t;
#pragma unroll
        for (int i = 0; i < (CPR + 3) / 4; ++i) {  // unrolled: every chunk's loads issued together
            const int cc = part + 4 * i;
            if (cc >= CPR) break;
            if constexpr (sizeof(T) == 2) {
                h8 ov = *reinterpret_cast<const h8 *>(Or + cc * CE);
                h8 dv = *reinterpret_cast<const h8 *>(Dr + cc * CE);
#pragma unroll
                for (int e = 0; e < 8; ++e) acc += (float)ov[e] * (float)dv[e];
            } else {
                f32x4 ov = *reinterpret_cast<const f32x4 *>(Or + cc * CE);
                f32x4 dv = *reinterpret_cast<const f32x4 *>(Dr + cc * CE);
#pragma unroll
                for (int e = 0; e < 4; ++e) acc += ov[e] * dv[e];
            }
        }
    }
    acc += __shfl_xor(acc, 1, 64);
    acc += __shfl_xor(acc, 2, 64);
    if (writer) {
        const float prl = ok ? prel - blse : 0.f;
        const float spread = blse - prel0;
        if constexpr (XB) {  // the row's running maximum (+inf past T: P = 0) and log2 l
            p.qinfo[qi_at(bh, p.NB, row, QI_LQ)] = ok ? lse : pinf();
            p.qinfo[qi_at(bh, p.NB, row, QI_LL)] = ok ? lsl : 0.f;
        } else {
            p.qinfo[qi_at(bh, p.NB, row, QI_LQ)] = ok ? -lse / p.sc2 : ninf();
        }
        p.qinfo[qi_at(bh, p.NB, row, QI_DL)] = ok ? -acc : 0.f;
        p.qinfo[qi_at(bh, p.NB, row, QI_PRE)] = ok ? pre : pinf();
        p.qinfo[qi_at(bh, p.NB, row, QI_ZQ)] = (FPA_KV_PROD && spread <= PROD_SPREAD) ? fexp2(prl) : prl;
        // The block's BMIN and BLSE for the key side's loop (plane QI_BST, positions 0 and 1).
        if (row % G < 2) p.qinfo[qi_at(bh, p.NB, row, QI_BST)] = (row % G == 0) ? bmin : blse;
    }
}

template <typename T, int D, int WPE, int NW>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
fpa_bwd_kv_kernel(BwdParams p) {
    __shared__ KvShared<T, D, NW> sm;
    constexpr int NP = kv_parts<T, D>();
    int rank, bh;
    xcd_work_item(rank, bh, p.BH, p.H, NP * ((p.T + 32 * NW - 1) / (32 * NW)));
    bwd_kv_tile<T, D, NW>(p, sm, rank / NP, bh, rank % NP);  // rank 0: the heaviest key tile (most query blocks)
}

template <typename T, int D>
static hipError_t launch_prep_t(const BwdParams &p, hipStream_t s) {
    hipLaunchKernelGGL((fpa_bwd_prep_kernel<T, D>), head_grid(p.TP / 64, p.H, p.BH), dim3(NTHREADS), 0, s, p);
    return hipGetLastError();
}

template <typename T, int D>
static hipError_t launch_kv_t(const BwdParams &p, hipStream_t s) {
    constexpr int NW = FPA_NW, WPE = kv_wpe<T, D>();
    const int nkt = kv_parts<T, D>() * ((p.T + 32 * NW - 1) / (32 * NW));
    hipLaunchKernelGGL((fpa_bwd_kv_kernel<T, D, WPE, NW>), head_grid(nkt, p.H, p.BH), dim3(64 * NW), 0, s, p);
    return hipGetLastError();
}

#define FPA_DISPATCH(FN)                                   \
    if (dtype == 0) {                                      \
        switch (D) {                                       \
            case 16: return FN<f16, 16>(p, s);             \
            case 32: return FN<f16, 32>(p, s);             \
            case 64: return FN<f16, 64>(p, s);             \
            case 128: return FN<f16, 128>(p, s);           \
            case 256: return FN<f16, 256>(p, s);           \
        }                                                  \
    } else {                                               \
        switch (D) {                                       \
            case 16: return FN<float, 16>(p, s);           \
            case 32: return FN<float, 32>(p, s);           \
            case 64: return FN<float, 64>(p, s);           \
            case 128: return FN<float, 128>(p, s);         \
            case 256: return FN<float, 256>(p, s);         \
        }                                                  \
    }                                                      \
    return hipErrorInvalidValue;

hipError_t launch_bwd_prep(const BwdParams &p, int dtype, int D, hipStream_t s) { FPA_DISPATCH(launch_prep_t) }
hipError_t launch_bwd_kv(const BwdParams &p, int dtype, int D, hipStream_t s) { FPA_DISPATCH(launch_kv_t) }

}  // namespace fpa
