// fpa_bwd_q.h -- the query-side backward tile of First Passage Attention.
//
// Reference behaviour: _bwd_q (kernel.py:286-340) of yliu-fort/first-passage-attention.
// gfx950 design: a workgroup of FPA_NW waves owns 32 queries per wave (one query per lane
// column) and streams 64-key blocks from the diagonal down to key 0 through
// double-buffered (single-buffered where two stages do not fit in LDS: fp32 at D = 256),
// padded LDS tiles filled by direct global->LDS loads (one barrier per
// block).  Each wave
// recomputes S^T = K Q^T and dP^T = V dO^T with Q, dO in registers, accumulates
// dQ^T += K^T dS^T on the 32x32 MFMA (K^T read from the row-major tile with LDS
// transpose reads), and reduces per query the query-block soft-min sum
//   R_t = sum_{s outside blk(t)} g_ts 2^{c_t} / Z_ts,   c_t = max a over [start of blk(t), t].
// The diagonal block (keys and query in one 64-block) uses the in-block range minimum.
#pragma once

#include <type_traits>

#include "fpa_common.h"
#include "fpa_params.h"

// Tuning knobs (build-time): waves per SIMD of the D <= 64 query-side kernel, and whether
// well-conditioned tiles use the shared-reference soft-min path.
#ifndef FPA_Q_WPE
#define FPA_Q_WPE 2
#endif
#ifndef FPA_Q_FAST
#define FPA_Q_FAST 1
#endif
// Per-key fast paths of off-diagonal blocks on the shared-reference path; 0 turns them off.
#ifndef FPA_Q_CLASSES
#define FPA_Q_CLASSES 1
#endif

namespace fpa {

// Waves per SIMD of the query-side tile (fp32 at D = 64 spills 50 VGPRs at two waves and runs 41%
// faster at one).
template <typename T, int D>
constexpr int q_wpe() { return (D >= 128 || (sizeof(T) == 4 && D >= 64)) ? 1 : FPA_Q_WPE; }

// LDS of one query-side workgroup.
template <typename T, int D, int NW>
struct QShared {
    static constexpr int TB = Pad<T, (D < 32 ? 32 : D)>::template bytes<64>();  // one padded K or V tile
    static constexpr int NS = tile_stages<TB>(2 * 8 * 64 * 4 + NW * 64 * 4);
    __attribute__((aligned(1024))) char Ks[NS][TB];
    __attribute__((aligned(1024))) char Vs[NS][TB];
    // Per-key values of a block: BSUF, CP (= betal * psi; SUF and PSI for fp32), SUFL, PHI, and BST (BMIN, BLSE, SUF of the
    // first key at [4][0..2]; planes 4-7 are four copies, so the two halves are one 1 KB load each
    // from the even and the odd waves).
    __attribute__((aligned(1024))) float kst[NS][8][64];
    __attribute__((aligned(16))) float Aw[NW][64];  // per-wave key factors of the shared-reference path
    __attribute__((aligned(16))) float Bw[NW][64];  // per-wave per-key bias of classes 1, 2
};

// Queries [32 NW qt, 32 NW (qt + 1)) of head bh: every key block from their diagonal block down to 0.
// SPLIT (small fused launches): half 1 takes the key blocks from jbmax down to jbs = jbmax + 1 -
// max(2, (jbmax + 1) / 2) (both diagonal blocks of the tile), half 2 the blocks below jbs; each writes
// its dQ accumulators and R to the split-tile partials (pq, pqr) for the merge kernel.
template <typename T, int D, int NW, bool SPLIT = false>
__device__ __forceinline__ void bwd_q_tile(const BwdParams &p, QShared<T, D, NW> &sm, const int qt, const int bh,
                                           const int half = 0) {
    constexpr int BM = 32 * NW, BK = 64;  // queries per workgroup, keys per iteration (one block)
    constexpr int DT = D < 32 ? 32 : D;
    constexpr int NDT = DT / 32;
    auto &Ks = sm.Ks;
    auto &Vs = sm.Vs;
    auto &kst = sm.kst;
    auto &Aw = sm.Aw;
    auto &Bw = sm.Bw;

    const int tid = thread_x(), lane = tid % 64, g = lane / 32, c = lane % 32;
    const int w = __builtin_amdgcn_readfirstlane(tid / 64);  // wave index, uniform across the wave
    const int b = bh / p.H, h = bh % p.H;
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
    // lanes 0-15: BSUF, 16-31: CP, 32-47: SUFL, 48-63: PHI.  With fp32 operands SUF and PSI take the
    // places of BSUF and CP: x = min(SUF_s, MID, PRE_t) - psi_s is formed before the scaling by betal.
    constexpr bool XB = exact_bias<T>();
    const int kpl = (lane < 16) ? (XB ? PL_SUF : PL_BSUF) : (lane < 32) ? (XB ? PL_PSI : PL_CP) : (lane < 48) ? PL_SUFL : PL_PHI;
    const float *st_head = p.state + L.at(0, bh, 0);
    const uint32_t kst_off = (uint32_t)((kpl * p.TP + 4 * (lane & 15)) * 4);  // bytes from plane 0 of the head
    const uint32_t bst_off = (uint32_t)((PL_BST * p.TP + 4 * (lane & 15)) * 4);  // four copies of BST

    TileLoader<T, D, DT, BK, NW> kld, vld;
    kld.init(p.sk.t, w, lane);
    vld.init(p.sv.t, w, lane);
    const uint32_t aK = lds_addr(&Ks[0][0]), aV = lds_addr(&Vs[0][0]), aS = lds_addr(&kst[0][0][0]);
    auto issue = [&](int jb, int buf) {
        kld.issue(aK + buf * sizeof(Ks[0]), Kb, p.sk.t, jb * BK, p.T, w, lane);
        vld.issue(aV + buf * sizeof(Vs[0]), Vb, p.sv.t, jb * BK, p.T, w, lane);
#pragma unroll
        for (int hq = (NW >= 2 ? w % 2 : 0); hq < 2; hq += (NW >= 2 ? 2 : 1))
            buf_lds16(buf_rsrc(st_head + jb * BK), hq ? bst_off : kst_off, aS + buf * sizeof(kst[0]) + 1024 * hq);
    };
    const int jbmax = umin_i(p.NB - 1, (q0 + BM - 1) / BK);
    int jbhi = jbmax, jblo = 0;
    if constexpr (SPLIT) {
        if (half != 0) {
            const int jbs = jbmax + 1 - max(2, (jbmax + 1) / 2);
            if (half == 1)
                jblo = jbs;
            else
                jbhi = jbs - 1;
        }
    }
    issue(jbhi, 0);

    OpRow<T, D> qreg, doreg;
    load_row_p1<T, D>(qreg, Qb + (int64_t)tq * p.sq.t, t_valid, g);
    load_row_p1<T, D>(doreg, DOb + (int64_t)tq * p.sdo.t, t_valid, g);

    const float betal = p.beta[h] * LOG2E;
    float lse = pinf(), lsl = 0.f, del = 0.f, pre = 0.f, prel = 0.f;
    if (t_valid) {
        lse = p.lse[rowbase + tq];  // fp32: the row's running maximum
        if constexpr (XB) lsl = p.lse[(int64_t)p.BH * p.TP + rowbase + tq];
        del = -p.qinfo[qi_at(bh, p.NB, tq, QI_DL)];
        pre = p.state[L.at(PL_PRE, bh, tq)];
        prel = p.state[L.at(PL_PREL, bh, tq)];
    }
    const float ct = -pre * p.il2;  // max a over [start of blk(t), t]
    // PRE_t is non-increasing along a block: this is the largest PRE of the wave's queries.
    const float premax = wave_max(t_valid ? pre : ninf());
    const float prel_ct = fexp2(prel - ct);
    const float E = (betal >= 0.f) ? ninf() : pinf();  // med3(x, y, E) = min (beta >= 0) or max (beta < 0)

    // The S and dP accumulators start at -lse_t / sc2 and -Delta_t (this lane's query, the same in
    // all 16 registers): the MFMA chains subtract them for free.  Rows past T get lse = +inf, so
    // their scores are -inf and P = 0 with no per-element mask.  fp32: S starts at 0, and the
    // logit is formed as in the forward and shifted by the forward's running maximum and log2 l,
    // P = 2^{(s - m) - log2 l}, so that P is the forward's to a few ulps whatever the size of s.
    f32x16 lq16, dl16;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        lq16[j] = XB ? 0.f : -lse / p.sc2;
        dl16[j] = -del;
    }

    f32x16 dqacc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) dqacc[dt] = zero16();
    float racc = 0.f;
    float mid = pinf(), midl = ninf(), cmid = ninf();  // over blocks strictly between jb and ib
    const int ibc = umin_i(ib, p.NB - 1);  // waves past T keep ib in range for these reads
    const float a_first = -ld_uniform(p.state, L.at(PL_PHI, bh, ibc * G)) * p.il2;  // a of the block's first query
    const float c_blk = -ld_uniform(p.state, L.bplane(BP_MIN) + brow + ibc) * p.il2;          // max a over block ib

    // BMIN / BLSE of block jb + 1 (which joins the middle), from the previous block's staged values.
    float bm_prev = 0.f, bl_prev = 0.f;
    if constexpr (SPLIT) {
        if (half == 2 && wave_active) {  // blocks jbs + 1 .. ib - 1 are between; block jbs joins them first
            const int jbs = jbhi + 1;
            const float *bmin = p.state + L.bplane(BP_MIN) + brow, *blse = p.state + L.bplane(BP_LSE) + brow;
            float m = pinf(), l = ninf();
            for (int j0 = jbs + 1; j0 < ib; j0 += 64) {
                const int j = j0 + lane;
                if (j < ib) {
                    m = fminf(m, bmin[j]);
                    l = lse2_pair(l, blse[j]);
                }
            }
            mid = wave_min(m);
            midl = wave_reduce(l, [](float a, float b) { return lse2_pair(a, b); });
            cmid = (mid < pinf()) ? -mid * p.il2 : ninf();
            bm_prev = ld_uniform(bmin, jbs);
            bl_prev = ld_uniform(blse, jbs);
        }
    }
    wait_loads();
    __syncthreads();
    constexpr int NS = QShared<T, D, NW>::NS;
    for (int jb = jbhi, it = 0; jb >= jblo; --jb, ++it) {
        const int buf = (NS == 2) ? (it & 1) : 0;
        const int s0 = jb * BK;
        if constexpr (NS == 2) issue(jb > 0 ? jb - 1 : 0, buf ^ 1);
        const float bm_here = kst[buf][4][0], bl_here = kst[buf][4][1], suf_first = kst[buf][4][2];
        if (wave_active && jb <= ib) {
            const float *kSUF = kst[buf][0], *kPSI = kst[buf][1], *kSUFL = kst[buf][2], *kPHI = kst[buf][3];
            if (jb + 1 < ib) {  // block jb + 1 joins the middle
                mid = fminf(mid, bm_prev);
                midl = lse2_pair(midl, bl_prev);
                cmid = fmaxf(cmid, -bm_prev * p.il2);
            }
            const float mterm = fexp2(midl - ct) + prel_ct;
            // Shared reference R >= every exponent of the tile (largest C_s is at the block's first key).
            bool fast = false;
            float R = 0.f, bq = 0.f;
            if (jb < ib) {
                const float cfirst = -suf_first * p.il2;  // SUF of the block's first key
                R = fmaxf(fmaxf(cfirst, cmid), c_blk);
                fast = FPA_Q_FAST && (R - fmaxf(cmid, a_first)) < FAST_SPREAD;
                if (fast) {
                    Aw[w][lane] = fexp2(kSUFL[lane] - R) + fexp2(midl - R);
                    bq = t_valid ? fexp2(prel - R) : 1.f;  // rows past T: any positive factor (g = 0)
                }
            }
            float rblk = 0.f;  // sum of g / (Z 2^{-R}) over this key block (shared-reference path)
            const float bY = XB ? fminf(pre, mid) : betal * fminf(pre, mid);
            // Shared-reference path, when every query of the wave has PRE_t >= MID (the largest
            // min(SUF_s, MID) of a block is MID: its last key has an empty suffix), x_ts =
            // min(SUF_s, MID) - psi_s for all t: bias and gate are per key, tabled once per block
            // in Bw (class 1).  When moreover 2^{PREL_t - MIDL} <= 2^-25 for every query,
            // Z_ts 2^{-R} = Aw_s + bq_t equals Aw_s to within 2^-25 (Aw_s >= 2^{MIDL - R}): the
            // reciprocal is per key too (class 2, 1 / Aw_s in Aw).  The per-key gate goes into Aw:
            // a closed gate makes the class-2 factor 0 and the class-1 denominator +inf (reciprocal
            // 0), so g / Z is dS / Z with no per-element gate.
            int cls = 0;
            if (FPA_Q_CLASSES && fast && __all(!t_valid || pre >= mid)) {
                cls = __all(!t_valid || prel - midl <= -25.f) ? 2 : 1;
                bool open;
                if constexpr (XB) {
                    const float x = fminf(kSUF[lane], mid) - kPSI[lane];
                    Bw[w][lane] = betal * fminf(x, 0.f);
                    open = x <= 0.f;
                } else {
                    const float v = __builtin_amdgcn_fmed3f(kSUF[lane], betal * mid, E) - kPSI[lane];
                    const float bmk = __builtin_amdgcn_fmed3f(v, 0.f, E);
                    Bw[w][lane] = bmk;
                    open = bmk == v;
                }
                const float aw = Aw[w][lane];
                Aw[w][lane] = (cls == 2) ? (open ? 1.f / aw : 0.f) : (open ? aw : pinf());
            } else if (FPA_Q_CLASSES && fast) {
                // Class 3: the gate x_ts <= 0 open for every pair.  x grows with PRE_t, so it is
                // enough that it holds at the wave's largest PRE for every key of the block (lane =
                // key); then bm = v and g = dS.
                bool open;
                if constexpr (XB) {
                    open = fminf(kSUF[lane], fminf(premax, mid)) <= kPSI[lane];
                } else {
                    const float v = __builtin_amdgcn_fmed3f(kSUF[lane], betal * fminf(premax, mid), E) - kPSI[lane];
                    open = __builtin_amdgcn_fmed3f(v, 0.f, E) == v;
                }
                if (__all(open)) cls = 3;
            }
            const bool diag = (jb == ib);
            const bool upper = (qw0 - ib * G) >= 32;  // this wave holds queries 32-63 of its block
            const int tr = tq - s0;
            const char *Kt = Ks[buf];
            const char *Vt = Vs[buf];
            float r = pinf();  // running min of phi over [u, t] for the in-block scan
            // On the diagonal the upper 32 keys come after every one of the first 32 queries: that
            // quarter (all P = 0) is skipped.
#pragma unroll 1
            for (int mt = (diag && !upper) ? 0 : 1; mt >= 0; --mt) {
                // S' = S - lse_t / sc2 and dP' = dP - Delta_t  ([s][t])
                f32x16 S = lq16, dP = dl16;
                mma_p1_pad_reg2<T, D, DT>(S, Kt, 32 * mt + c, qreg, dP, Vt, 32 * mt + c, doreg, g);
                float X[16];
                if (diag) {  // X_ts = min phi(s, t] in the block; the upper queries' first half is all before them
                    if (mt == 0 && upper)
                        diag_x_keys<true>(X, r, kPHI, mt, tr, g);
                    else
                        diag_x_keys(X, r, kPHI, mt, tr, g);
                }
                if (!diag) {
                    // Off the diagonal block every key is valid and earlier than every query.
                    auto offdiag = [&](auto fast_c, auto cls_c) {
                        constexpr bool FAST = decltype(fast_c)::value;
                        constexpr int CLS = decltype(cls_c)::value;
#pragma unroll
                        for (int jq = 0; jq < 4; ++jq) {
                            const int s4 = 32 * mt + 8 * jq + 4 * g;
                            const f32x4 zk4 = FAST ? *reinterpret_cast<const f32x4 *>(&Aw[w][s4])
                                                   : *reinterpret_cast<const f32x4 *>(&kSUFL[s4]);
                            if constexpr (CLS == 1 || CLS == 2) {
                                const f32x4 bm4 = *reinterpret_cast<const f32x4 *>(&Bw[w][s4]);
#pragma unroll
                                for (int e = 0; e < 4; ++e) {
                                    const int j = 4 * jq + e;
                                    const float P = fexp2(XB ? (fmaf(S[j], p.sc2, bm4[e]) - lse) - lsl : fmaf(S[j], p.sc2, bm4[e]));
                                    const float dS = P * dP[j];
                                    rblk = fmaf(dS, (CLS == 2) ? zk4[e] : frcp(zk4[e] + bq), rblk);
                                    S[j] = dS;
                                }
                                continue;
                            }
                            const f32x4 bsuf4 = *reinterpret_cast<const f32x4 *>(&kSUF[s4]);
                            const f32x4 bpsi4 = *reinterpret_cast<const f32x4 *>(&kPSI[s4]);
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                const int j = 4 * jq + e;
                                // v = betal * x with x = min(SUF_s, MID, PRE_t) - psi_s, and the bias
                                // bm = betal * min(x, 0); the gate x <= 0 is bm == v for either sign.
                                float bm;
                                bool open;
                                if constexpr (XB) {  // bsuf4, bpsi4 hold SUF and psi, bY min(PRE_t, MID)
                                    const float x = fminf(bsuf4[e], bY) - bpsi4[e];
                                    bm = betal * ((CLS == 3) ? x : fminf(x, 0.f));
                                    open = x <= 0.f;
                                } else {
                                    const float v = __builtin_amdgcn_fmed3f(bsuf4[e], bY, E) - bpsi4[e];
                                    bm = (CLS == 3) ? v : __builtin_amdgcn_fmed3f(v, 0.f, E);
                                    open = bm == v;
                                }
                                const float P = fexp2(XB ? (fmaf(S[j], p.sc2, bm) - lse) - lsl : fmaf(S[j], p.sc2, bm));
                                const float dS = P * dP[j];
                                const float gg = (CLS == 3 || open) ? dS : 0.f;
                                if constexpr (FAST)
                                    rblk = fmaf(gg, frcp(zk4[e] + bq), rblk);
                                else
                                    racc = fmaf(gg, frcp(fexp2(zk4[e] - ct) + mterm), racc);
                                S[j] = dS;
                            }
                        }
                    };
                    using C0 = std::integral_constant<int, 0>;
#if FPA_Q_FAST
                    if (cls == 2)
                        offdiag(std::true_type{}, std::integral_constant<int, 2>{});
                    else if (cls == 3)
                        offdiag(std::true_type{}, std::integral_constant<int, 3>{});
                    else if (cls == 1)
                        offdiag(std::true_type{}, std::integral_constant<int, 1>{});
                    else if (fast)
                        offdiag(std::true_type{}, C0{});
                    else
#endif
                        offdiag(std::false_type{}, C0{});
                } else {
#pragma unroll
                    for (int jq = 0; jq < 4; ++jq) {
                        const int s4 = 32 * mt + 8 * jq + 4 * g;
                        const f32x4 bpsi4 = *reinterpret_cast<const f32x4 *>(&kPSI[s4]);
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int j = 4 * jq + e;
                            const int s = s0 + s4 + e;
                            const bool valid = t_valid && (s <= tq);
                            const bool strict = valid && (s < tq);
                            const float bm = !strict ? 0.f
                                             : XB ? betal * fminf(X[j] - bpsi4[e], 0.f)
                                                  : __builtin_amdgcn_fmed3f(fmaf(betal, X[j], -bpsi4[e]), 0.f, E);
                            const float P = !valid ? 0.f
                                            : fexp2(XB ? (fmaf(S[j], p.sc2, bm) - lse) - lsl : fmaf(S[j], p.sc2, bm));
                            S[j] = P * dP[j];
                        }
                    }
                }
                // dQ^T[d][t] += K^T[d][s] dS^T[s][t]   (K read transposed from its natural layout)
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt)
                    dqacc[dt] = mma_p2_p3_pad<T, DT, true>(dqacc[dt], S, Kt, 32 * mt, 32 * dt, lane);
            }
            if (fast) racc = fmaf(fexp2(ct - R), rblk, racc);  // R_t gets 2^{c_t} sum g / Z
        }
        bm_prev = bm_here;
        bl_prev = bl_here;
        if constexpr (NS == 1) {  // every wave is done with the tiles: load the next block in their place
            __syncthreads();
            issue(jb > 0 ? jb - 1 : 0, 0);
        }
        wait_loads();
        __syncthreads();
    }

    racc = sum_halves(racc);
    if (!wave_active) return;
    if constexpr (SPLIT) {
        if (half != 0) {  // partial sums of a split tile (queries QS .. T - 1): raw dQ accumulators and R
            if (!t_valid) return;
            const int64_t qs = ((int64_t)(half - 1) * p.BH + bh) * (p.T - p.QS) + (tq - p.QS);
            if (g == 0) p.pqr[qs] = racc;
            float *row = p.pq + qs * D;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int jq = 0; jq < 4; ++jq) {
                    const int d0 = 32 * dt + 8 * jq + 4 * g;
                    if (d0 < D)
                        *reinterpret_cast<f32x4 *>(row + d0) = f32x4{dqacc[dt][4 * jq + 0], dqacc[dt][4 * jq + 1],
                                                                     dqacc[dt][4 * jq + 2], dqacc[dt][4 * jq + 3]};
                }
            return;
        }
    }
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

}  // namespace fpa
