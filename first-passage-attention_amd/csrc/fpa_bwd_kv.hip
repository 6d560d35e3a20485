// fpa_bwd_kv.hip -- key-side backward of First Passage Attention.
//
// Reference behaviour: _bwd_delta (kernel.py:165-174) and _bwd_kv (kernel.py:177-265)
// of yliu-fort/first-passage-attention.  gfx950 design: a workgroup of 4 waves owns
// 128 keys (32 per wave, one key per lane column) and streams 32-query tiles from
// the diagonal to T through LDS (Q and dO both row-major and transposed).  Each
// wave computes S = Q K^T and dP = dO V^T with K, V held in registers, then
// dV^T += dO^T P and dK^T += Q^T dS on the 32x32 MFMA.  Per key it also reduces
//   dpsi_s  = -beta * sum_t g_ts                       (g = [x <= 0] dS, strict t > s)
//   dbeta   = sum_{t>s} dS_ts min(0, x_ts)             (per-wave partials, summed later)
//   W_s     = sum_{t outside blk(s)} g_ts 2^{C_s} / Z_ts   (key-block soft-min sums)
//   TBUF    = middle-block soft-min sums per (query block, key block, key half)
// and writes the in-block gated dS to GD for the in-block soft-min recurrence.
#include "fpa_common.h"
#include "fpa_params.h"

namespace fpa {

// Delta_t = sum_d dO_td O_td (fp32), zero for padded rows.
template <typename T, int D>
__global__ void __launch_bounds__(NTHREADS) fpa_bwd_prep_kernel(BwdParams p) {
    constexpr int CE = MT<T>::CHUNK;
    constexpr int CPR = (D + CE - 1) / CE;
    const int bh = blockIdx.y, b = bh / p.H, h = bh % p.H;
    const int row = blockIdx.x * 64 + threadIdx.x / 4, part = threadIdx.x % 4;
    float acc = 0.f;
    if (row < p.T) {
        const T *Or = static_cast<const T *>(p.o) + b * p.so.b + h * p.so.h + (int64_t)row * p.so.t;
        const T *Dr = static_cast<const T *>(p.dout) + b * p.sdo.b + h * p.sdo.h + (int64_t)row * p.sdo.t;
        for (int cc = part; cc < CPR; cc += 4) {
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
    if (part == 0 && row < p.TP) p.delta[(int64_t)bh * p.TP + row] = acc;
}

template <typename T, int D>
__global__ void __launch_bounds__(NTHREADS) fpa_bwd_kv_kernel(BwdParams p) {
    constexpr int BK = 128, BQ = 32;
    constexpr int DT = D < 32 ? 32 : D;
    constexpr int NDT = DT / 32;
    constexpr int PQ = D + (sizeof(T) == 2 ? 8 : 4);  // row-major tile pitch
    constexpr int PT = BQ + 4;                          // transposed tile pitch
    __shared__ __attribute__((aligned(16))) T Qs[BQ * PQ];
    __shared__ __attribute__((aligned(16))) T dOs[BQ * PQ];
    __shared__ __attribute__((aligned(16))) T QT[DT * PT];
    __shared__ __attribute__((aligned(16))) T dOT[DT * PT];
    __shared__ float rLSE[BQ], rDEL[BQ], rPRE[BQ], rPREL[BQ];
    __shared__ float kPHI[BK];

    const int tid = threadIdx.x, w = tid / 64, lane = tid % 64, g = lane / 32, c = lane % 32;
    const int kt = blockIdx.x;  // heaviest (most query tiles) first
    const int bh = blockIdx.y, b = bh / p.H, h = bh % p.H;
    const int k0 = kt * BK, kw0 = k0 + 32 * w, s = kw0 + c;
    const int jb = kw0 / G, sb = jb * G;
    const bool wave_active = kw0 < p.T;
    const bool s_valid = s < p.T;
    const StateLayout L{p.BH, p.TP, p.NB};
    const int64_t rowbase = (int64_t)bh * p.TP;
    const int64_t brow = (int64_t)bh * p.NB;

    const T *Qb = static_cast<const T *>(p.q) + b * p.sq.b + h * p.sq.h;
    const T *Kb = static_cast<const T *>(p.k) + b * p.sk.b + h * p.sk.h;
    const T *Vb = static_cast<const T *>(p.v) + b * p.sv.b + h * p.sv.h;
    const T *DOb = static_cast<const T *>(p.dout) + b * p.sdo.b + h * p.sdo.h;

    OpRow<T, D> kreg, vreg;
    load_row_p1<T, D>(kreg, Kb + (int64_t)s * p.sk.t, s_valid, g);
    load_row_p1<T, D>(vreg, Vb + (int64_t)s * p.sv.t, s_valid, g);

    const float beta = p.beta[h], betal = beta * LOG2E;
    float psi_s = 0.f, suf = pinf(), sufl = ninf();
    if (s < p.TP) {
        psi_s = p.state[L.plane(PL_PSI) + rowbase + s];
        suf = p.state[L.plane(PL_SUF) + rowbase + s];
        sufl = p.state[L.plane(PL_SUFL) + rowbase + s];
    }
    const float Cs = (suf < pinf()) ? -suf * p.il2 : ninf();  // max a over (s, end of block)
    const float sufpsi = suf - psi_s;

    if constexpr (D < DT) {
        for (int i = tid; i < (DT - D) * PT; i += NTHREADS) {
            QT[D * PT + i] = (T)0.f;
            dOT[D * PT + i] = (T)0.f;
        }
    }
    if (tid < BK) kPHI[tid] = (k0 + tid < p.TP) ? p.state[L.plane(PL_PHI) + rowbase + k0 + tid] : pinf();

    f32x16 dkacc[NDT], dvacc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
        dkacc[dt] = zero16();
        dvacc[dt] = zero16();
    }
    float gsum = 0.f, dbacc = 0.f, Wacc = 0.f, wblk = 0.f;
    float mid = pinf(), midl = ninf(), cmid = ninf();  // over blocks strictly between jb and ib
    float rs = ninf(), sv = 0.f;
    int cur_ib = -1;
    const float *phiblk = kPHI + (sb - k0);  // phi of this wave's key block (64 values)

    for (int q0 = k0; q0 < p.T; q0 += BQ) {
        const int ib = q0 / G;
        if (ib != cur_ib) {
            if (cur_ib > jb) {  // close the previous query block: W and middle-block sums
                if (rs > ninf()) Wacc += fexp2(Cs - rs) * wblk;
                if (cur_ib > jb + 1) {
                    const float tp = wave_sum((rs > ninf()) ? fexp2(cmid - rs) * wblk : 0.f);
                    if (lane == 0 && wave_active)
                        p.tbuf[((brow + cur_ib) * p.NB + jb) * 2 + (w & 1)] = tp;
                }
                const float bm = p.state[L.bplane(BP_MIN) + brow + cur_ib];
                mid = fminf(mid, bm);
                midl = lse2_pair(midl, p.state[L.bplane(BP_LSE) + brow + cur_ib]);
                cmid = fmaxf(cmid, -bm * p.il2);
            }
            wblk = 0.f;
            cur_ib = ib;
            if (ib > jb) {
                rs = fmaxf(Cs, cmid);
                sv = (rs > ninf()) ? fexp2(sufl - rs) + fexp2(midl - rs) : 0.f;
            }
        }

        __syncthreads();
        stage_rows<T, D, BQ, PQ>(Qs, Qb, p.sq.t, q0, p.T);
        stage_rows<T, D, BQ, PQ>(dOs, DOb, p.sdo.t, q0, p.T);
        stage_rows_t<T, D, BQ, PT>(QT, Qb, p.sq.t, q0, p.T);
        stage_rows_t<T, D, BQ, PT>(dOT, DOb, p.sdo.t, q0, p.T);
        if (tid < BQ) {
            rLSE[tid] = p.lse[rowbase + q0 + tid];
            rDEL[tid] = p.delta[rowbase + q0 + tid];
            rPRE[tid] = p.state[L.plane(PL_PRE) + rowbase + q0 + tid];
            rPREL[tid] = p.state[L.plane(PL_PREL) + rowbase + q0 + tid];
        }
        __syncthreads();
        if (!wave_active || q0 + BQ - 1 < kw0) continue;

        f32x16 S = mma_p1_lds_reg<T, D>(zero16(), Qs + c * PQ, g, kreg);   // [t][s]
        f32x16 dP = mma_p1_lds_reg<T, D>(zero16(), dOs + c * PQ, g, vreg);

        const bool diag = (ib == jb);
        float Xd[16];
        if (diag) {
            // X_ts = min phi(s, t] inside the block: ascending scan from s+1.
            const int sr = s - sb, qh = (q0 - sb) >> 5;
#pragma unroll
            for (int j = 0; j < 16; ++j) Xd[j] = pinf();
            float r = pinf();
#pragma unroll
            for (int u = 0; u < G; ++u) {
                r = (u > sr) ? fminf(r, phiblk[u]) : r;
                const int jj = u & 31, gg = (jj >> 2) & 1, j = (jj >> 3) * 4 + (jj & 3);
                if ((u >> 5) == qh && gg == g) Xd[j] = r;
            }
        }
        const float Y0 = mid;
        float tile_g[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int tr = acc_row(j, g), t = q0 + tr;
            const bool valid = (t < p.T) && (t >= s) && s_valid;
            const bool strict = valid && (t > s);
            float x;
            if (diag)
                x = Xd[j] - psi_s;
            else
                x = fminf(sufpsi, fminf(rPRE[tr], Y0) - psi_s);
            const float xm = strict ? fminf(x, 0.f) : 0.f;
            const float z = S[j] * p.sc2 + betal * xm - rLSE[tr];
            const float P = valid ? fexp2(z) : 0.f;
            const float dS = P * (dP[j] - rDEL[tr]);
            const float gg = (strict && x <= 0.f) ? dS : 0.f;
            gsum += gg;
            dbacc += dS * xm;
            if (!diag && rs > ninf()) wblk += gg * frcp(sv + fexp2(rPREL[tr] - rs));
            tile_g[j] = gg;
            S[j] = P;
            dP[j] = dS;
        }
        if (diag && s_valid) {
            float *gdrow = p.gd + ((brow + jb) * G + (s - sb)) * G + (q0 - sb);
#pragma unroll
            for (int jq = 0; jq < 4; ++jq) {
                f32x4 v4 = {tile_g[4 * jq + 0], tile_g[4 * jq + 1], tile_g[4 * jq + 2], tile_g[4 * jq + 3]};
                *reinterpret_cast<f32x4 *>(gdrow + 8 * jq + 4 * g) = v4;
            }
        }

        // dV^T[d][s] += dO^T[d][t] P[t][s];  dK^T[d][s] += Q^T[d][t] dS[t][s]
        const f32x16 Pt[1] = {S};
        const f32x16 dSt[1] = {dP};
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
            dvacc[dt] = mma_p2_p3<T, 1, true>(dvacc[dt], Pt, dOT + (32 * dt + c) * PT, g);
            dkacc[dt] = mma_p2_p3<T, 1, true>(dkacc[dt], dSt, QT + (32 * dt + c) * PT, g);
        }
    }
    if (cur_ib > jb) {
        if (rs > ninf()) Wacc += fexp2(Cs - rs) * wblk;
        if (cur_ib > jb + 1) {
            const float tp = wave_sum((rs > ninf()) ? fexp2(cmid - rs) * wblk : 0.f);
            if (lane == 0 && wave_active) p.tbuf[((brow + cur_ib) * p.NB + jb) * 2 + (w & 1)] = tp;
        }
    }

    // Per-key outputs (lanes c and c + 32 hold the same key, different queries).
    gsum += __shfl_xor(gsum, 32, 64);
    Wacc += __shfl_xor(Wacc, 32, 64);
    const float dbw = wave_sum(dbacc);
    if (lane == 0) p.dbp[((int64_t)bh * p.NKV + kt) * 4 + w] = dbw;  // 0 for waves past T
    if (!wave_active) return;
    if (g == 0 && s < p.TP) p.wsum[rowbase + s] = Wacc;
    if (g == 0 && s_valid) p.dpsi[(int64_t)bh * p.T + s] = -beta * gsum;
    if (!s_valid) return;
    T *dKr = static_cast<T *>(p.dk) + b * p.sdk.b + h * p.sdk.h + (int64_t)s * p.sdk.t;
    T *dVr = static_cast<T *>(p.dv) + b * p.sdv.b + h * p.sdv.h + (int64_t)s * p.sdv.t;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int jq = 0; jq < 4; ++jq) {
            const int d0 = 32 * dt + 8 * jq + 4 * g;
            if (d0 < D) {
                if constexpr (sizeof(T) == 2) {
                    h4 kv4 = {(f16)(dkacc[dt][4 * jq + 0] * p.smscale), (f16)(dkacc[dt][4 * jq + 1] * p.smscale),
                              (f16)(dkacc[dt][4 * jq + 2] * p.smscale), (f16)(dkacc[dt][4 * jq + 3] * p.smscale)};
                    h4 vv4 = {(f16)dvacc[dt][4 * jq + 0], (f16)dvacc[dt][4 * jq + 1], (f16)dvacc[dt][4 * jq + 2],
                              (f16)dvacc[dt][4 * jq + 3]};
                    *reinterpret_cast<h4 *>(dKr + d0) = kv4;
                    *reinterpret_cast<h4 *>(dVr + d0) = vv4;
                } else {
                    f32x4 kv4 = {dkacc[dt][4 * jq + 0] * p.smscale, dkacc[dt][4 * jq + 1] * p.smscale,
                                 dkacc[dt][4 * jq + 2] * p.smscale, dkacc[dt][4 * jq + 3] * p.smscale};
                    f32x4 vv4 = {dvacc[dt][4 * jq + 0], dvacc[dt][4 * jq + 1], dvacc[dt][4 * jq + 2],
                                 dvacc[dt][4 * jq + 3]};
                    *reinterpret_cast<f32x4 *>(dKr + d0) = kv4;
                    *reinterpret_cast<f32x4 *>(dVr + d0) = vv4;
                }
            }
        }
}

template <typename T, int D>
static hipError_t launch_prep_t(const BwdParams &p, hipStream_t s) {
    hipLaunchKernelGGL((fpa_bwd_prep_kernel<T, D>), dim3(p.TP / 64, p.BH), dim3(NTHREADS), 0, s, p);
    return hipGetLastError();
}

template <typename T, int D>
static hipError_t launch_kv_t(const BwdParams &p, hipStream_t s) {
    hipLaunchKernelGGL((fpa_bwd_kv_kernel<T, D>), dim3(p.NKV, p.BH), dim3(NTHREADS), 0, s, p);
    return hipGetLastError();
}

#define FPA_DISPATCH(FN)                                   \
    if (dtype == 0) {                                      \
        switch (D) {                                       \
            case 16: return FN<f16, 16>(p, s);             \
            case 32: return FN<f16, 32>(p, s);             \
            case 64: return FN<f16, 64>(p, s);             \
            case 128: return FN<f16, 128>(p, s);           \
        }                                                  \
    } else {                                               \
        switch (D) {                                       \
            case 16: return FN<float, 16>(p, s);           \
            case 32: return FN<float, 32>(p, s);           \
            case 64: return FN<float, 64>(p, s);           \
            case 128: return FN<float, 128>(p, s);         \
        }                                                  \
    }                                                      \
    return hipErrorInvalidValue;

hipError_t launch_bwd_prep(const BwdParams &p, int dtype, int D, hipStream_t s) { FPA_DISPATCH(launch_prep_t) }
hipError_t launch_bwd_kv(const BwdParams &p, int dtype, int D, hipStream_t s) { FPA_DISPATCH(launch_kv_t) }

}  // namespace fpa
