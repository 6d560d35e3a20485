// fpa_fwd.hip -- block statistics and the fp32 forward pass of First Passage Attention.
//
// Reference behaviour: kernel.py:83-100 (_stats) and kernel.py:103-162 (_fwd) of
// yliu-fort/first-passage-attention.  Same maths, gfx950 design:
//   * statistics: one wave per block of G = 64 positions, prefix/suffix min and
//     base-2 log-sum-exp by wave shuffles;
//   * forward: the kernel template of fpa_fwd.h, instantiated here for fp32 operands
//     (fpa_fwd16.hip holds the fp16 ones); launch_fwd dispatches on the operand type.
#include "fpa_fwd.h"

namespace fpa {

// ---------------------------------------------------------------------------
// Block statistics (per head, per 64-block):
//   PHI, PSI  : contiguous float copies (phi = +inf past T)
//   PRE_t     = min phi[sb .. t]           PREL_t = log2 sum 2^a[sb .. t]
//   SUF_s     = min phi(s .. eb)           SUFL_s = log2 sum 2^a(s .. eb)
//   BMIN, BLSE: the whole block.           a_u = -phi_u * log2(e) / tau
//   CA, CP    : beta*log2e*min(SUF - psi, 0) and beta*log2e*psi (the forward's per-key terms)
//   BSUF      : beta*log2e*SUF (the query side's per-key term)
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(64) fpa_stats_kernel(StatsParams p) {
    const int blk = group_x(), bh = group_bh(p.H);
    const int b = bh / p.H, h = bh % p.H;
    const int lane = thread_x();
    const int u = blk * G + lane;
    float ph = pinf(), ps = 0.f;
    if (u < p.T) {
        ph = p.phi[b * p.sphi.b + h * p.sphi.h + (int64_t)u * p.sphi.t];
        ps = p.psi[b * p.spsi.b + h * p.spsi.h + (int64_t)u * p.spsi.t];
    }
    const float a = (u < p.T) ? -ph * p.il2 : ninf();

    float pm = ph, pl = a;  // inclusive prefix
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float ym = __shfl_up(pm, o, 64);
        const float yl = __shfl_up(pl, o, 64);
        if (lane >= o) {
            pm = fminf(pm, ym);
            pl = lse2_pair(pl, yl);
        }
    }
    float sm = ph, sl = a;  // inclusive suffix
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float ym = __shfl_down(sm, o, 64);
        const float yl = __shfl_down(sl, o, 64);
        if (lane + o < 64) {
            sm = fminf(sm, ym);
            sl = lse2_pair(sl, yl);
        }
    }
    float suf = __shfl_down(sm, 1, 64), sufl = __shfl_down(sl, 1, 64);  // strictly after
    if (lane == 63) {
        suf = pinf();
        sufl = ninf();
    }
    StateLayout L{p.BH, p.TP, p.NB};
    p.state[L.at(PL_PHI, bh, u)] = ph;
    p.state[L.at(PL_PSI, bh, u)] = ps;
    p.state[L.at(PL_PRE, bh, u)] = pm;
    p.state[L.at(PL_PREL, bh, u)] = pl;
    p.state[L.at(PL_SUF, bh, u)] = suf;
    p.state[L.at(PL_SUFL, bh, u)] = sufl;
    const float betal = p.beta[bh % p.H] * LOG2E;
    p.state[L.at(PL_CA, bh, u)] = betal * fminf(suf - ps, 0.f);
    p.state[L.at(PL_CP, bh, u)] = betal * ps;
    p.state[L.at(PL_BSUF, bh, u)] = (suf < pinf()) ? betal * suf : (betal > 0.f ? pinf() : betal < 0.f ? ninf() : 0.f);
    const float bmin = __shfl(pm, 63, 64), blse = __shfl(pl, 63, 64), suf0 = __shfl(suf, 0, 64);
    p.state[L.at(PL_BST, bh, u)] = (lane == 0) ? bmin : (lane == 1) ? blse : (lane == 2) ? suf0 : 0.f;
    if (lane == 63) {
        p.state[L.bplane(BP_MIN) + (int64_t)bh * p.NB + blk] = pm;
        p.state[L.bplane(BP_LSE) + (int64_t)bh * p.NB + blk] = pl;
    }
}

hipError_t launch_stats(const StatsParams &p, hipStream_t s) {
    hipLaunchKernelGGL(fpa_stats_kernel, head_grid(p.NB, p.H, p.BH), dim3(64), 0, s, p);
    return hipGetLastError();
}

int fwd_split_tiles(int64_t BH, int64_t T, int dtype, int D) {
    const int64_t nqt = (T + 32 * FPA_NW - 1) / (32 * FPA_NW);
    const int wpe = (D == 128) ? 2 : (D >= 128) ? 1 : (dtype == 0 ? FPA_FWD_WPE : (D <= 32 ? 3 : FPA_FWD_WPE32));  // fwd_wpe
    if (nqt < 4 || 100 * BH * nqt > (int64_t)FPA_FWD_SPLIT_FILL * 8 * XCD_CUS * wpe) return 0;
    return (int)(nqt / 2);
}

hipError_t launch_fwd_merge(const FwdParams &p, int dtype, int D, hipStream_t s) {
    if (dtype == 0) return launch_fwd_merge_f16(p, D, s);
    switch (D) {
        case 16: return launch_fwd_merge_t<float, 16>(p, s);
        case 32: return launch_fwd_merge_t<float, 32>(p, s);
        case 64: return launch_fwd_merge_t<float, 64>(p, s);
        case 128: return launch_fwd_merge_t<float, 128>(p, s);
        case 256: return launch_fwd_merge_t<float, 256>(p, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_fwd(const FwdParams &p, int dtype, int D, hipStream_t s) {
    if (dtype == 0) return launch_fwd_f16(p, D, s);
    switch (D) {
        case 16: return launch_fwd_t<float, 16>(p, s);
        case 32: return launch_fwd_t<float, 32>(p, s);
        case 64: return launch_fwd_t<float, 64>(p, s);
        case 128: return launch_fwd_t<float, 128>(p, s);
        case 256: return launch_fwd_t<float, 256>(p, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace fpa
