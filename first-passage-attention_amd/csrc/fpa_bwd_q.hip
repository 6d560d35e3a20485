// fpa_bwd_q.hip -- query-side backward of First Passage Attention.
//
// Reference behaviour: _bwd_q (kernel.py:286-340) of yliu-fort/first-passage-attention.
// gfx950 design: a workgroup of 4 waves owns 128 queries (one query per lane column)
// and streams 32-key tiles from the diagonal down to key 0 through LDS (K row-major
// and transposed, V row-major).  Each wave recomputes S^T = K Q^T and dP^T = V dO^T
// with Q, dO in registers, accumulates dQ^T += K^T dS^T on the 32x32 MFMA, and
// reduces per query the query-block soft-min sum
//   R_t = sum_{s outside blk(t)} g_ts 2^{c_t} / Z_ts,   c_t = max a over [start of blk(t), t].
// The diagonal block (keys and query in one 64-block) uses the in-block range minimum.
#include "fpa_common.h"
#include "fpa_params.h"

namespace fpa {

template <typename T, int D>
__global__ void __launch_bounds__(NTHREADS) fpa_bwd_q_kernel(BwdParams p) {
    constexpr int BM = 128, BK = 32;
    constexpr int DT = D < 32 ? 32 : D;
    constexpr int NDT = DT / 32;
    constexpr int PK = D + (sizeof(T) == 2 ? 8 : 4);
    constexpr int PT = BK + 4;
    __shared__ __attribute__((aligned(16))) T Ks[BK * PK];
    __shared__ __attribute__((aligned(16))) T Vs[BK * PK];
    __shared__ __attribute__((aligned(16))) T KT[DT * PT];
    __shared__ float kSUF[BK], kSUFL[BK], kPSI[BK];
    __shared__ float bPHI[G];

    const int tid = threadIdx.x, w = tid / 64, lane = tid % 64, g = lane / 32, c = lane % 32;
    const int qt = gridDim.x - 1 - blockIdx.x;  // longest rows first
    const int bh = blockIdx.y, b = bh / p.H, h = bh % p.H;
    const int q0 = qt * BM, qw0 = q0 + 32 * w, tq = qw0 + c;
    const int ib = qw0 / G;
    const bool wave_active = qw0 < p.T;
    const bool t_valid = tq < p.T;
    const StateLayout L{p.BH, p.TP, p.NB};
    const int64_t rowbase = (int64_t)bh * p.TP;
    const int64_t brow = (int64_t)bh * p.NB;

    const T *Qb = static_cast<const T *>(p.q) + b * p.sq.b + h * p.sq.h;
    const T *Kb = static_cast<const T *>(p.k) + b * p.sk.b + h * p.sk.h;
    const T *Vb = static_cast<const T *>(p.v) + b * p.sv.b + h * p.sv.h;
    const T *DOb = static_cast<const T *>(p.dout) + b * p.sdo.b + h * p.sdo.h;

    OpRow<T, D> qreg, doreg;
    load_row_p1<T, D>(qreg, Qb + (int64_t)tq * p.sq.t, t_valid, g);
    load_row_p1<T, D>(doreg, DOb + (int64_t)tq * p.sdo.t, t_valid, g);

    const float betal = p.beta[h] * LOG2E;
    float lse = 0.f, del = 0.f, pre = 0.f, prel = 0.f;
    if (t_valid) {
        lse = p.lse[rowbase + tq];
        del = p.delta[rowbase + tq];
        pre = p.state[L.plane(PL_PRE) + rowbase + tq];
        prel = p.state[L.plane(PL_PREL) + rowbase + tq];
    }
    const float ct = -pre * p.il2;  // max a over [start of blk(t), t]
    const float prel_ct = fexp2(prel - ct);

    if constexpr (D < DT) {
        for (int i = tid; i < (DT - D) * PT; i += NTHREADS) KT[D * PT + i] = (T)0.f;
    }

    f32x16 dqacc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) dqacc[dt] = zero16();
    float racc = 0.f;
    float mid = pinf(), midl = ninf();  // over blocks strictly between jb and ib
    float mterm = prel_ct;
    int cur_jb = -1;

    const int nk = (p.T + BK - 1) / BK;
    const int ktmax = min(nk - 1, (q0 + BM - 1) / BK);
    for (int kt = ktmax; kt >= 0; --kt) {
        const int k0 = kt * BK;
        const int jb = k0 / G;
        if (jb != cur_jb) {
            // Entering key block jb from jb + 1: block jb + 1 joins the middle if it lies below ib.
            if (cur_jb >= 0 && cur_jb < ib) {
                mid = fminf(mid, p.state[L.bplane(BP_MIN) + brow + cur_jb]);
                midl = lse2_pair(midl, p.state[L.bplane(BP_LSE) + brow + cur_jb]);
            }
            cur_jb = jb;
            mterm = fexp2(midl - ct) + prel_ct;
        }
        __syncthreads();
        stage_rows<T, D, BK, PK>(Ks, Kb, p.sk.t, k0, p.T);
        stage_rows<T, D, BK, PK>(Vs, Vb, p.sv.t, k0, p.T);
        stage_rows_t<T, D, BK, PT>(KT, Kb, p.sk.t, k0, p.T);
        if (tid < BK) {
            kSUF[tid] = p.state[L.plane(PL_SUF) + rowbase + k0 + tid];
            kSUFL[tid] = p.state[L.plane(PL_SUFL) + rowbase + k0 + tid];
            kPSI[tid] = p.state[L.plane(PL_PSI) + rowbase + k0 + tid];
        } else if (tid >= 64 && tid < 64 + G) {
            bPHI[tid - 64] = p.state[L.plane(PL_PHI) + rowbase + jb * G + (tid - 64)];
        }
        __syncthreads();
        if (!wave_active || k0 > qw0 + 31) continue;

        f32x16 S = mma_p1_lds_reg<T, D>(zero16(), Ks + c * PK, g, qreg);    // [s][t]
        f32x16 dP = mma_p1_lds_reg<T, D>(zero16(), Vs + c * PK, g, doreg);

        const bool diag = (jb == ib);
        float Xd[16];
        if (diag) {
            // X_ts = min phi(s, t] inside the block: descending scan down to s+1.
            const int tr = tq - jb * G, kh = (k0 - jb * G) >> 5;
#pragma unroll
            for (int j = 0; j < 16; ++j) Xd[j] = pinf();
            float r = pinf();
#pragma unroll
            for (int u = G - 1; u >= 1; --u) {
                r = (u <= tr) ? fminf(r, bPHI[u]) : r;
                const int sr = u - 1, jj = sr & 31, gg = (jj >> 2) & 1, j = (jj >> 3) * 4 + (jj & 3);
                if ((sr >> 5) == kh && gg == g) Xd[j] = r;
            }
        }
        const float Y = fminf(pre, mid);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int sr = acc_row(j, g), s = k0 + sr;
            const bool valid = t_valid && (s <= tq);
            const bool strict = valid && (s < tq);
            const float psi_s = kPSI[sr];
            float x;
            if (diag)
                x = Xd[j] - psi_s;
            else
                x = fminf(kSUF[sr] - psi_s, Y - psi_s);
            const float xm = strict ? fminf(x, 0.f) : 0.f;
            const float z = S[j] * p.sc2 + betal * xm - lse;
            const float P = valid ? fexp2(z) : 0.f;
            const float dS = P * (dP[j] - del);
            const float gg = (strict && x <= 0.f) ? dS : 0.f;
            if (!diag) racc += gg * frcp(fexp2(kSUFL[sr] - ct) + mterm);
            S[j] = dS;
        }
        // dQ^T[d][t] += K^T[d][s] dS^T[s][t]
        const f32x16 dSt[1] = {S};
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) dqacc[dt] = mma_p2_p3<T, 1, true>(dqacc[dt], dSt, KT + (32 * dt + c) * PT, g);
    }

    racc += __shfl_xor(racc, 32, 64);
    if (!wave_active) return;
    if (g == 0 && tq < p.TP) p.rsum[rowbase + tq] = t_valid ? racc : 0.f;
    if (!t_valid) return;
    T *dQr = static_cast<T *>(p.dq) + b * p.sdq.b + h * p.sdq.h + (int64_t)tq * p.sdq.t;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int jq = 0; jq < 4; ++jq) {
            const int d0 = 32 * dt + 8 * jq + 4 * g;
            if (d0 < D) {
                if constexpr (sizeof(T) == 2) {
                    h4 v4 = {(f16)(dqacc[dt][4 * jq + 0] * p.smscale), (f16)(dqacc[dt][4 * jq + 1] * p.smscale),
                             (f16)(dqacc[dt][4 * jq + 2] * p.smscale), (f16)(dqacc[dt][4 * jq + 3] * p.smscale)};
                    *reinterpret_cast<h4 *>(dQr + d0) = v4;
                } else {
                    f32x4 v4 = {dqacc[dt][4 * jq + 0] * p.smscale, dqacc[dt][4 * jq + 1] * p.smscale,
                                dqacc[dt][4 * jq + 2] * p.smscale, dqacc[dt][4 * jq + 3] * p.smscale};
                    *reinterpret_cast<f32x4 *>(dQr + d0) = v4;
                }
            }
        }
}

template <typename T, int D>
static hipError_t launch_q_t(const BwdParams &p, hipStream_t s) {
    const int nqt = (p.T + 127) / 128;
    hipLaunchKernelGGL((fpa_bwd_q_kernel<T, D>), dim3(nqt, p.BH), dim3(NTHREADS), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_bwd_q(const BwdParams &p, int dtype, int D, hipStream_t s) {
    if (dtype == 0) {
        switch (D) {
            case 16: return launch_q_t<f16, 16>(p, s);
            case 32: return launch_q_t<f16, 32>(p, s);
            case 64: return launch_q_t<f16, 64>(p, s);
            case 128: return launch_q_t<f16, 128>(p, s);
        }
    } else {
        switch (D) {
            case 16: return launch_q_t<float, 16>(p, s);
            case 32: return launch_q_t<float, 32>(p, s);
            case 64: return launch_q_t<float, 64>(p, s);
            case 128: return launch_q_t<float, 128>(p, s);
        }
    }
    return hipErrorInvalidValue;
}

}  // namespace fpa
