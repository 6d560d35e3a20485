// fpa_bwd_kv.hip -- key-side backward of First Passage Attention.
//
// Reference behaviour: _bwd_delta (kernel.py:165-174) and _bwd_kv (kernel.py:177-265)
// of yliu-fort/first-passage-attention.  gfx950 design: a workgroup of 4 waves owns
// 128 keys (32 per wave, one key per lane column) and streams 64-query blocks from
// the diagonal to T through double-buffered LDS (register prefetch of the next block,
// one barrier per block).  Each wave computes S = Q K^T and dP = dO V^T with K, V
// held in registers, then dV^T += dO^T P and dK^T += Q^T dS on the 32x32 MFMA (dO^T
// and Q^T read from the row-major tiles with LDS transpose reads).  Per key it reduces
//   dpsi_s  = -beta * sum_t g_ts                       (g = [x <= 0] dS, strict t > s)
//   dbeta   = sum_{t>s} dS_ts min(0, x_ts)             (per-wave partials, summed later)
//   W_s     = sum_{t outside blk(s)} g_ts 2^{C_s} / Z_ts   (key-block soft-min sums)
//   TBUF    = middle-block soft-min sums per (query block, key block, key half)
// and writes the in-block gated dS to GD for the in-block soft-min recurrence.
#include <type_traits>

#include "fpa_common.h"
#include "fpa_params.h"

// Tuning knobs (build-time): waves per SIMD of the fp16 D <= 64 key-side kernel, and whether
// well-conditioned tiles use the shared-reference soft-min path.
#ifndef FPA_KV_WPE
#define FPA_KV_WPE 2
#endif
#ifndef FPA_KV_FAST
#define FPA_KV_FAST 0
#endif

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

template <typename T, int D, int WPE>
__global__ void __launch_bounds__(NTHREADS) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
fpa_bwd_kv_kernel(BwdParams p) {
    constexpr int BK = 128, BQ = 64;   // keys per workgroup, queries per iteration (one block)
    constexpr int DT = D < 32 ? 32 : D;
    constexpr int NDT = DT / 32;
    constexpr int PQ = D + (sizeof(T) == 2 ? 8 : 4);  // tile pitch (elements)
    constexpr int TS = BQ * PQ;
    __shared__ __attribute__((aligned(16))) T Qs[2 * TS + (DT - D)];
    __shared__ __attribute__((aligned(16))) T dOs[2 * TS + (DT - D)];
    __shared__ __attribute__((aligned(16))) float rLSE[2][BQ], rDEL[2][BQ], rPRE[2][BQ], rPREL[2][BQ];
    __shared__ __attribute__((aligned(16))) float kPHI[BK];
    __shared__ __attribute__((aligned(16))) float Bw[4][BQ];  // per-wave query factors of the shared-reference path

    const int tid = threadIdx.x, lane = tid % 64, g = lane / 32, c = lane % 32;
    const int w = __builtin_amdgcn_readfirstlane(tid / 64);  // wave index, uniform across the wave
    int rank, bh;
    xcd_work_item(rank, bh, p.BH);
    const int kt = rank;  // heaviest (most query blocks) first
    const int b = bh / p.H, h = bh % p.H;
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

    if constexpr (D < DT) {  // columns D..31 read by the padded transpose reads stay zero
        for (int i = tid; i < 2 * TS + (DT - D); i += NTHREADS) {
            Qs[i] = (T)0.f;
            dOs[i] = (T)0.f;
        }
    }
    if (tid < BK) kPHI[tid] = (k0 + tid < p.TP) ? p.state[L.plane(PL_PHI) + rowbase + k0 + tid] : pinf();

    f32x16 dkacc[NDT], dvacc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
        dkacc[dt] = zero16();
        dvacc[dt] = zero16();
    }
    float gsum = 0.f, dbacc = 0.f, Wacc = 0.f;
    float mid = pinf(), midl = ninf(), cmid = ninf();  // over blocks strictly between jb and ib
    const float *phiblk = kPHI + (sb - k0);

    TileRegs<T, D, BQ> qr, dor;
    float pf_lse = 0.f, pf_del = 0.f, pf_pre = 0.f, pf_prel = 0.f;
    auto gload = [&](int ib) {
        qr.load(Qb, p.sq.t, ib * BQ, p.T);
        dor.load(DOb, p.sdo.t, ib * BQ, p.T);
        if (tid < BQ) {
            const int64_t r = rowbase + ib * BQ + tid;
            pf_lse = p.lse[r];
            pf_del = p.delta[r];
            pf_pre = p.state[L.plane(PL_PRE) + r];
            pf_prel = p.state[L.plane(PL_PREL) + r];
        }
    };
    auto lstore = [&](int buf) {
        qr.store(Qs + buf * TS, PQ);
        dor.store(dOs + buf * TS, PQ);
        if (tid < BQ) {
            rLSE[buf][tid] = pf_lse;
            rDEL[buf][tid] = pf_del;
            rPRE[buf][tid] = pf_pre;
            rPREL[buf][tid] = pf_prel;
        }
    };

    const int ib0 = k0 / G;
    gload(ib0);
    lstore(0);
    __syncthreads();
    for (int ib = ib0, it = 0; ib < p.NB; ++ib, ++it) {
        const int buf = it & 1;
        if (ib + 1 < p.NB) gload(ib + 1);
        if (wave_active && ib >= jb) {
            float rs = ninf(), sv = 0.f;
            bool fast = false;
            if (ib > jb) {
                if (ib - 1 > jb) {  // block ib - 1 joins the middle
                    const float bm = p.state[L.bplane(BP_MIN) + brow + ib - 1];
                    mid = fminf(mid, bm);
                    midl = lse2_pair(midl, p.state[L.bplane(BP_LSE) + brow + ib - 1]);
                    cmid = fmaxf(cmid, -bm * p.il2);
                }
                // Shared reference R >= every exponent of the tile; the smallest pair maximum is
                // at least max(cmid, a of the block's first query).
                const float cfirst = uniform_f(Cs);  // lane 0 holds the wave's first key: largest C_s
                const float R = fmaxf(fmaxf(cfirst, cmid), -p.state[L.bplane(BP_MIN) + brow + ib] * p.il2);
                const float lo = fmaxf(cmid, -p.state[L.plane(PL_PHI) + rowbase + ib * BQ] * p.il2);
                fast = FPA_KV_FAST && (R - lo) < FAST_SPREAD;
                if (fast) {
                    rs = R;  // W_s and TBUF are scaled by 2^{. - R} at the end of the block
                    sv = fexp2(sufl - R) + fexp2(midl - R);
                    Bw[w][lane] = fexp2(rPREL[buf][lane] - R);
                } else {
                    rs = fmaxf(Cs, cmid);
                    sv = (rs > ninf()) ? fexp2(sufl - rs) + fexp2(midl - rs) : 0.f;
                }
            }
            const float Ap = fminf(sufpsi, mid - psi_s);  // min(SUF_s, MID) - psi_s
            const bool full = (ib + 1) * BQ <= p.T;
            const T *Qt = Qs + buf * TS;
            const T *Dt = dOs + buf * TS;
            const bool diag = (ib == jb);
            const int sr = s - sb;
            float r = pinf();  // running min of phi over (s, u] for the in-block scan
            float wblk = 0.f;
#pragma unroll 1
            for (int mt = 0; mt < 2; ++mt) {
                f32x16 S[1], dP[1];
                S[0] = mma_p1_lds_reg<T, D>(zero16(), Qt + (32 * mt + c) * PQ, g, kreg);   // [t][s]
                dP[0] = mma_p1_lds_reg<T, D>(zero16(), Dt + (32 * mt + c) * PQ, g, vreg);
                float X[16];
                if (diag) diag_x_queries(X, r, phiblk, mt, sr, g);  // X_ts = min phi(s, t] in the block
                if (!diag) {
                    // Off the diagonal block every key is valid and every query is later than
                    // every key; only the rows of a ragged last block are past T.
                    auto offdiag = [&](auto fast_c) {
                        constexpr bool FAST = decltype(fast_c)::value;
#pragma unroll
                        for (int jq = 0; jq < 4; ++jq) {
                            const int t4 = 32 * mt + 8 * jq + 4 * g;
                            const f32x4 lse4 = *reinterpret_cast<const f32x4 *>(&rLSE[buf][t4]);
                            const f32x4 del4 = *reinterpret_cast<const f32x4 *>(&rDEL[buf][t4]);
                            const f32x4 pre4 = *reinterpret_cast<const f32x4 *>(&rPRE[buf][t4]);
                            const f32x4 zq4 = FAST ? *reinterpret_cast<const f32x4 *>(&Bw[w][t4])
                                                   : *reinterpret_cast<const f32x4 *>(&rPREL[buf][t4]);
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                const int j = 4 * jq + e;
                                const float x = fminf(Ap, pre4[e] - psi_s);  // min(SUF_s, MID, PRE_t) - psi_s
                                const float xm = fminf(x, 0.f);
                                float P = fexp2(fmaf(S[0][j], p.sc2, fmaf(betal, xm, -lse4[e])));
                                if (!full) P = (ib * BQ + t4 + e < p.T) ? P : 0.f;
                                const float dS = P * (dP[0][j] - del4[e]);
                                const float gg = (x <= 0.f) ? dS : 0.f;
                                gsum += gg;
                                dbacc = fmaf(gg, x, dbacc);
                                // Z_ts 2^{-r} = sv + 2^{PREL_t - r}, r shared (FAST) or per key
                                const float zq = FAST ? zq4[e] : fexp2(zq4[e] - rs);
                                wblk = fmaf(gg, frcp(sv + zq), wblk);
                                S[0][j] = P;
                                dP[0][j] = dS;
                            }
                        }
                    };
#if FPA_KV_FAST
                    if (fast)
                        offdiag(std::true_type{});
                    else
#endif
                        offdiag(std::false_type{});
                } else {
#pragma unroll
                    for (int jq = 0; jq < 4; ++jq) {
                        const int t4 = 32 * mt + 8 * jq + 4 * g;
                        const f32x4 lse4 = *reinterpret_cast<const f32x4 *>(&rLSE[buf][t4]);
                        const f32x4 del4 = *reinterpret_cast<const f32x4 *>(&rDEL[buf][t4]);
                        f32x4 g4;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int j = 4 * jq + e;
                            const int t = ib * BQ + t4 + e;
                            const bool valid = (t < p.T) && (t >= s) && s_valid;
                            const bool strict = valid && (t > s);
                            const float x = X[j] - psi_s;
                            const float xm = strict ? fminf(x, 0.f) : 0.f;
                            const float P = valid ? fexp2(fmaf(S[0][j], p.sc2, fmaf(betal, xm, -lse4[e]))) : 0.f;
                            const float dS = P * (dP[0][j] - del4[e]);
                            const float gg = (strict && x <= 0.f) ? dS : 0.f;
                            gsum += gg;
                            dbacc = fmaf(dS, xm, dbacc);  // x is +inf where the range is empty
                            g4[e] = gg;
                            S[0][j] = P;
                            dP[0][j] = dS;
                        }
                        if (s_valid) *reinterpret_cast<f32x4 *>(p.gd + ((brow + jb) * G + sr) * G + t4) = g4;
                    }
                }
                // dV^T[d][s] += dO^T[d][t] P[t][s];  dK^T[d][s] += Q^T[d][t] dS[t][s]
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) {
                    dvacc[dt] = mma_p2_p3<T, 1, true>(dvacc[dt], S, Dt + 32 * mt * PQ, PQ, 32 * dt, lane);
                    dkacc[dt] = mma_p2_p3<T, 1, true>(dkacc[dt], dP, Qt + 32 * mt * PQ, PQ, 32 * dt, lane);
                }
            }
            if (ib > jb) {  // close query block ib: key-block and middle-block soft-min sums
                if (rs > ninf()) Wacc = fmaf(fexp2(Cs - rs), wblk, Wacc);
                if (ib > jb + 1) {
                    const float tp = wave_sum((rs > ninf()) ? fexp2(cmid - rs) * wblk : 0.f);
                    if (lane == 0) p.tbuf[((brow + ib) * p.NB + jb) * 2 + (w & 1)] = tp;
                }
            }
        }
        if (ib + 1 < p.NB) lstore(buf ^ 1);
        __syncthreads();
    }

    // Per-key outputs (lanes c and c + 32 hold the same key, different queries).
    gsum = sum_halves(gsum);
    Wacc = sum_halves(Wacc);
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
    constexpr int WPE = (D >= 128 || (sizeof(T) == 4 && D >= 64)) ? 1 : FPA_KV_WPE;
    hipLaunchKernelGGL((fpa_bwd_kv_kernel<T, D, WPE>), dim3(p.NKV, p.BH), dim3(NTHREADS), 0, s, p);
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
