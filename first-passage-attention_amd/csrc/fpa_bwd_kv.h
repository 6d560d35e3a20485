// fpa_bwd_kv.h -- the key-side backward tile of First Passage Attention.
//
// Reference behaviour: _bwd_kv (kernel.py:177-265) of yliu-fort/first-passage-attention.
// gfx950 design: a workgroup of FPA_NW waves owns
// 32 keys per wave (one key per lane column) and streams 64-query blocks from the
// diagonal to T through double-buffered (single-buffered where two stages do not fit in LDS:
// fp32 at D = 256), padded LDS tiles filled by direct global->LDS
// loads (one barrier per block).  Each wave computes S = Q K^T and dP = dO V^T with K, V
// held in registers, then dV^T += dO^T P and dK^T += Q^T dS on the 32x32 MFMA (dO^T
// and Q^T read from the row-major tiles with LDS transpose reads).  Per key it reduces
//   dpsi_s  = -beta * sum_t g_ts                       (g = [x <= 0] dS, strict t > s)
//   dbeta   = sum_{t>s} dS_ts min(0, x_ts)             (per-wave partials, summed later)
//   W_s     = sum_{t outside blk(s)} g_ts 2^{C_s} / Z_ts   (key-block soft-min sums)
//   TBUF    = middle-block soft-min sums per (query block, key block)
// and writes the in-block gated dS to GD for the in-block soft-min recurrence.
#pragma once

#include <type_traits>

#include "fpa_common.h"
#include "fpa_params.h"

// Tuning knobs (build-time): waves per SIMD of the fp16 D <= 64 key-side kernel, and whether
// well-conditioned tiles use the shared-reference soft-min path.
#ifndef FPA_KV_WPE
#define FPA_KV_WPE 2
#endif
#ifndef FPA_KV_PROD
#define FPA_KV_PROD 1
#endif
// Per-key fast paths of off-diagonal blocks (see bwd_kv_tile); 0 turns them off.
#ifndef FPA_KV_CLASSES
#define FPA_KV_CLASSES 1
#endif

namespace fpa {

// Per-query planes of the backward (QI_*), for t < TP:
//   LQ    -lse_t / sc2 (-inf past T) and DL = -Delta_t (0 past T), Delta_t = sum_d dO_td O_td: the
//         start values of the S and dP accumulators, so the MFMA chains subtract them for free;
//         rows past T get -inf scores and P = 0 with no per-element mask
//   PRE   PRE_t, the running minimum of phi from the start of t's block (+inf past T)
//   ZQ    with PRL_t = PREL_t - BLSE <= 0 (BLSE = log2 sum 2^a over t's block; 0 past T):
//         2^{PRL_t} > 0 when the block's spread -PRL_{first row} is at most PROD_SPREAD
//         (product form of the soft-min denominators), else PRL_t <= 0 (exact form).  The sign
//         of the block's first entry tells the two apart.
//   BST   the block's BMIN and BLSE (positions 0 and 1).
__device__ __forceinline__ float beta_eff(float betal) { return betal != 0.f ? betal : 0x1p-100f; }

// Waves per SIMD of the key-side tile: wide tiles need the registers of one wave per SIMD.
template <typename T, int D>
constexpr int kv_wpe() { return (D >= 128 || (sizeof(T) == 4 && D >= 64)) ? 1 : FPA_KV_WPE; }

// Parts of the head dimension whose dK / dV accumulators one workgroup holds: at D = 256 the
// accumulators and the K, V rows together exceed the registers of a wave, so each key tile is
// run twice (four times in fp32), each run accumulating dK and dV over one part of D and
// recomputing S and dP; the per-key scalars (dpsi, dbeta, W, TBUF, GD) come from part 0.
template <typename T, int D>
constexpr int kv_parts() { return D >= 256 ? (sizeof(T) == 2 ? 2 : 4) : 1; }

// LDS of one key-side workgroup.
template <typename T, int D, int NW>
struct KvShared {
    static constexpr int TB = Pad<T, (D < 32 ? 32 : D)>::template bytes<64>();  // one padded Q or dO tile
    static constexpr int NS = tile_stages<TB>(2 * QI_PLANES * 64 * 4 + 32 * NW * 4);
    __attribute__((aligned(1024))) char Qs[NS][TB];
    __attribute__((aligned(1024))) char dOs[NS][TB];
    __attribute__((aligned(1024))) float qi[NS][QI_PLANES][64];  // per-query values of a block: LQ, DL, PRE, ZQ, BST
    __attribute__((aligned(16))) float kPHI[32 * NW];
    float tpx[2][NW];  // each wave's middle-block sum of the last two query blocks (by parity)
};

// Keys [32 NW kt, 32 NW (kt + 1)) of head bh: every query block from the keys' diagonal block to T.
// SPLIT (small fused launches): half 1 takes the query blocks from the diagonal one up to ibs =
// ib0 + max(2, (NB - ib0) / 2) (both diagonal blocks of the tile), half 2 the blocks from ibs on; each
// writes its sums to the split-tile partials (pkv, pks, the second half of dbp) for the merge kernel.
template <typename T, int D, int NW, bool SPLIT = false>
__device__ __forceinline__ void bwd_kv_tile(const BwdParams &p, KvShared<T, D, NW> &sm, const int kt, const int bh,
                                            const int part = 0, const int half = 0) {
    constexpr int BK = 32 * NW, BQ = 64;   // keys per workgroup, queries per iteration (one block)
    constexpr int DT = D < 32 ? 32 : D;
    constexpr int NDT = DT / 32 / kv_parts<T, D>();  // dK / dV column tiles of this part
    const int dt0 = part * NDT;
    const bool scalars = part == 0;  // this run writes the per-key scalars
    auto &Qs = sm.Qs;
    auto &dOs = sm.dOs;
    auto &qi = sm.qi;
    float *const kPHI = sm.kPHI;

    const int tid = thread_x(), lane = tid % 64, g = lane / 32, c = lane % 32;
    const int w = __builtin_amdgcn_readfirstlane(tid / 64);  // wave index, uniform across the wave
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
    // A block's per-query values: planes 0-3 (LQ, DL, PRE, ZQ) and 4-7 (BST, three unused) with one
    // 1 KB load each, from the even and the odd waves (no wave-dependent branch).  After the last
    // block the prefetch repeats it into a buffer that is not read again.
    const float *qi_head = p.qinfo + qi_at(bh, p.NB, 0, 0);

    TileLoader<T, D, DT, BQ, NW> qld, dld;
    qld.init(p.sq.t, w, lane);
    dld.init(p.sdo.t, w, lane);
    const uint32_t aQ = lds_addr(&Qs[0][0]), aD = lds_addr(&dOs[0][0]), aI = lds_addr(&qi[0][0][0]);
    auto issue = [&](int ib, int buf) {
        qld.issue(aQ + buf * sizeof(Qs[0]), Qb, p.sq.t, ib * BQ, p.T, w, lane);
        dld.issue(aD + buf * sizeof(dOs[0]), DOb, p.sdo.t, ib * BQ, p.T, w, lane);
#pragma unroll
        for (int hq = (NW >= 2 ? w % 2 : 0); hq < 2; hq += (NW >= 2 ? 2 : 1))
            buf_lds16(buf_rsrc(qi_head + (int64_t)ib * QI_PLANES * 64), 1024 * hq + 16 * lane, aI + buf * sizeof(qi[0]) + 1024 * hq);
    };
    const int ib0 = k0 / G;
    int iblo = ib0, ibhi = p.NB;
    if constexpr (SPLIT) {
        if (half != 0) {
            const int ibs = ib0 + max(2, (p.NB - ib0) / 2);
            if (half == 1)
                ibhi = ibs;
            else
                iblo = ibs;
        }
    }
    issue(iblo, 0);

    OpRow<T, D> kreg, vreg;
    load_row_p1<T, D>(kreg, Kb + (int64_t)s * p.sk.t, s_valid, g);
    load_row_p1<T, D>(vreg, Vb + (int64_t)s * p.sv.t, s_valid, g);

    // Bias terms scaled by beff = beta * log2e (2^-100 for beta = 0, below fp32 resolution in the
    // exponent).  Off the diagonal, x = min(SUF_s, MID, PRE_t) - psi_s splits into a per-key part
    // and a per-query part: bm = beff * min(x, 0) = med3(beff PRE_t - beff psi_s, cAz, E) with
    // cAz = beff * min(SUF_s - psi_s, MID - psi_s, 0), and the gate x <= 0 is PRE_t <= thr with
    // thr = +inf when min(SUF_s, MID) <= psi_s (every query passes), else psi_s.  With fp32
    // operands x is formed before the scaling: x = min(PRE_t, mS) - psi_s with mS = min(SUF_s, MID,
    // psi_s), bm = beff * x, cAz = beff * cx with cx = mS - psi_s, and dbeta sums dS x directly.
    const float beta = p.beta[h], beff = beta_eff(beta * LOG2E);
    const float E = (beff > 0.f) ? ninf() : pinf();  // med3(x, y, E) = min (beff > 0) or max
    float psi_s = 0.f, suf = pinf(), sufl = ninf();
    if (s < p.TP) {
        psi_s = p.state[L.at(PL_PSI, bh, s)];
        suf = p.state[L.at(PL_SUF, bh, s)];
        sufl = p.state[L.at(PL_SUFL, bh, s)];
    }
    const float Cs = (suf < pinf()) ? -suf * p.il2 : ninf();  // max a over (s, end of block)
    const float bsuf = beff * suf, bpsi = beff * psi_s;
    constexpr bool XB = exact_bias<T>();
    // Accumulator start values from a per-query plane of the staged block: register j of this
    // lane holds row 32 mt + 8 (j / 4) + 4 g + j % 4.
    auto rows16 = [&](const float *plane, int mt) {
        f32x16 r;
#pragma unroll
        for (int jq = 0; jq < 4; ++jq) {
            const f32x4 v = *reinterpret_cast<const f32x4 *>(&plane[32 * mt + 8 * jq + 4 * g]);
#pragma unroll
            for (int e = 0; e < 4; ++e) r[4 * jq + e] = v[e];
        }
        return r;
    };
    if (tid < BK) kPHI[tid] = (k0 + tid < p.TP) ? p.state[L.at(PL_PHI, bh, k0 + tid)] : pinf();

    f32x16 dkacc[NDT], dvacc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
        dkacc[dt] = zero16();
        dvacc[dt] = zero16();
    }
    float gsum = 0.f, dbacc = 0.f, Wacc = 0.f;
    float mid = pinf(), midl = ninf(), cmid = ninf();  // over blocks strictly between jb and ib
    const float *phiblk = kPHI + (sb - k0);

    // The soft-min reference rs = max(C_s, cmid) and sv = 2^{SUFL_s - rs} + 2^{MIDL - rs} of the
    // current query block.  After a block the middle takes in its BMIN / BLSE (staged with the
    // block's per-query values) and both are recomputed for the next block, before its barrier.
    float rs = Cs, sv = (Cs > ninf()) ? fexp2(sufl - Cs) : 0.f;
    if constexpr (SPLIT) {
        if (half == 2 && wave_active) {  // blocks jb + 1 .. iblo - 1 are between the keys and the first query block
            const float *bmin = p.state + L.bplane(BP_MIN) + brow, *blse = p.state + L.bplane(BP_LSE) + brow;
            float m = pinf(), l = ninf();
            for (int j0 = jb + 1; j0 < iblo; j0 += 64) {
                const int j = j0 + lane;
                if (j < iblo) {
                    m = fminf(m, bmin[j]);
                    l = lse2_pair(l, blse[j]);
                }
            }
            mid = wave_min(m);
            midl = wave_reduce(l, [](float a, float b) { return lse2_pair(a, b); });
            cmid = (mid < pinf()) ? -mid * p.il2 : ninf();
            rs = fmaxf(Cs, cmid);
            sv = (rs > ninf()) ? fexp2(sufl - rs) + fexp2(midl - rs) : 0.f;
        }
    }
    wait_loads();
    __syncthreads();
    constexpr int NS = KvShared<T, D, NW>::NS;
    // TBUF holds one middle-block sum per (query block, key block) pair: the two waves of a 64-key
    // block (2 h, 2 h + 1) add their halves through LDS once the barrier that ends the query block has
    // passed, and the even wave writes the sum.
    static_assert(NW % 2 == 0, "two waves per 64-key block");
    auto flush_tbuf = [&](int ibp, int par) {
        if ((w & 1) == 0 && lane == 0 && scalars && wave_active && ibp > jb + 1)
            p.tbuf[(brow + ibp) * p.NB + jb] = sm.tpx[par][w] + sm.tpx[par][w + 1];
    };
    for (int ib = iblo, it = 0; ib < ibhi; ++ib, ++it) {
        const int buf = (NS == 2) ? (it & 1) : 0;
        if constexpr (NS == 2) issue(umin_i(ib + 1, p.NB - 1), buf ^ 1);
        if (it > 0) flush_tbuf(ib - 1, (it - 1) & 1);
        float tpw = 0.f;
        const float bm_here = qi[buf][QI_BST][0], bl_cur = qi[buf][QI_BST][1];  // block ib
        if (wave_active && ib >= jb) {
            // Soft-min denominators off the diagonal: Z_ts 2^{-rs} = sv + 2^{PREL_t - rs} with the
            // per-key reference rs = max(C_s, cmid) (sv >= 1 when rs is finite).  With
            // rsb = rs - BLSE, 2^{PREL_t - rs} = 2^{PRL_t - rsb}; when the block's PRL spread is at
            // most PROD_SPREAD this is ZQ_t * ck with ZQ_t = 2^{PRL_t} and ck = 2^{min(-rsb, 126)}:
            // one FMA per element instead of an exp2.  The clamp only changes terms whose
            // 2^{PREL_t - rs} exceeds 2^{126 - PROD_SPREAD}, where 1/Z is already below 2^{-26} of
            // the other terms.
            float rsb = ninf(), ck = 0.f;
            bool prod = false;
            if (ib > jb) {
                rsb = rs - bl_cur;
                ck = fexp2(fminf(-rsb, 126.f));
                prod = uniform_f(qi[buf][QI_ZQ][0]) > 0.f;
            }
            const float mS = fminf(fminf(suf, mid), psi_s), cx = mS - psi_s;
            const float cAz = XB ? beff * cx
                                 : __builtin_amdgcn_fmed3f(__builtin_amdgcn_fmed3f(bsuf, beff * mid, E) - bpsi, 0.f, E);
            const float thr = (fminf(suf, mid) <= psi_s) ? pinf() : psi_s;
            const float nbpsi = -bpsi;
            const char *Qt = Qs[buf];
            const char *Dt = dOs[buf];
            const float *rPRE = qi[buf][QI_PRE];
            const bool diag = (ib == jb);
            const bool upper = (kw0 - sb) >= 32;  // this wave holds keys 32-63 of its block
            const int sr = s - sb;
            float r = pinf();  // running min of phi over (s, u] for the in-block scan
            float wblk = 0.f;
            // Off the diagonal, when every query of block ib has PRE_t >= m_s = min(SUF_s, MID) for
            // every key of the wave (the block's minimum BMIN >= m_s), x_ts = m_s - psi_s for all t:
            // the bias is cAz per key and the gate m_s <= psi_s is per key, so the block needs only
            // sum_t dS_ts per key (class 1).  When moreover 2^{BLSE - rs} <= 2^-25 for every key, each
            // Z_ts 2^{-rs} = sv + 2^{PREL_t - rs} equals sv to within 2^-25 (sv >= 1), below fp32
            // resolution: the soft-min sum is sum_t g_ts / sv (class 2).  Otherwise, when the gate
            // PRE_t <= thr is open for every row (PRE_t is non-increasing along the block, so it is
            // enough that the block's first row passes for every key), g = dS (class 3, on the
            // product form of Z only).
            int cls = 0;
            if (FPA_KV_CLASSES && !diag) {
                if (__all(bm_here >= fminf(suf, mid)))
                    cls = __all(bl_cur - rs <= -25.f) ? 2 : 1;
                else if (prod && __all(rPRE[0] <= thr))
                    cls = 3;
            }
            float dsum = 0.f;  // classes 1, 2: sum of dS over the block
            // fp32: the block's dbeta terms dS x are summed on their own and added to dbacc once per
            // block (the terms cancel: every row of dS sums to zero, and |x| reaches hundreds).
            float dbblk = 0.f;
            // On the diagonal the upper 32 keys come after every one of the first 32 queries: that
            // quarter (all P = 0; its gd entries are never read) is skipped.
#pragma unroll 1
            for (int mt = (diag && upper) ? 1 : 0; mt < 2; ++mt) {
                f32x16 S, dP;
                // S - lse / sc2 and dP - Delta, rows t, columns s
                S = XB ? zero16() : rows16(qi[buf][QI_LQ], mt);
                dP = rows16(qi[buf][QI_DL], mt);
                mma_p1_pad_reg2<T, D, DT>(S, Qt, 32 * mt + c, kreg, dP, Dt, 32 * mt + c, vreg, g);
                float X[16];
                if (diag) {  // X_ts = min phi(s, t] in the block; the lower keys' second half is all after them
                    if (mt == 1 && !upper)
                        diag_x_queries<true>(X, r, phiblk, mt, sr, g);
                    else
                        diag_x_queries(X, r, phiblk, mt, sr, g);
                }
                if (!diag) {
                    // Off the diagonal block every key is valid and every query is later than
                    // every key; rows of a ragged last block are past T and have P = 0.
                    auto offdiag = [&](auto prod_c, auto cls_c) {
                        constexpr bool PROD = decltype(prod_c)::value;
                        constexpr int CLS = decltype(cls_c)::value;
                        const float *rZQ = qi[buf][QI_ZQ];
#pragma unroll
                        for (int jq = 0; jq < 4; ++jq) {
                            const int t4 = 32 * mt + 8 * jq + 4 * g;
                            const f32x4 pre4 = *reinterpret_cast<const f32x4 *>(&rPRE[t4]);
                            f32x4 m4, l4;  // fp32: the rows' running maxima and log2 l
                            if constexpr (XB) {
                                m4 = *reinterpret_cast<const f32x4 *>(&qi[buf][QI_LQ][t4]);
                                l4 = *reinterpret_cast<const f32x4 *>(&qi[buf][QI_LL][t4]);
                            }
                            const f32x4 zq4 = *reinterpret_cast<const f32x4 *>(&rZQ[t4]);
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                const int j = 4 * jq + e;
                                if constexpr (CLS == 0 || CLS == 3) {
                                    const float xb = XB ? fminf(pre4[e], mS) - psi_s : 0.f;
                                    const float bm = XB ? beff * xb : __builtin_amdgcn_fmed3f(fmaf(pre4[e], beff, nbpsi), cAz, E);
                                    const float P = fexp2(XB ? (fmaf(S[j], p.sc2, bm) - m4[e]) - l4[e] : fmaf(S[j], p.sc2, bm));
                                    const float dS = P * dP[j];
                                    const float gg = (CLS == 3 || pre4[e] <= thr) ? dS : 0.f;
                                    gsum += gg;
                                    if constexpr (XB)
                                        dbblk = fmaf(dS, xb, dbblk);
                                    else
                                        dbacc = fmaf(dS, bm, dbacc);
                                    const float z = PROD ? fmaf(zq4[e], ck, sv) : sv + fexp2(zq4[e] - rsb);
                                    wblk = fmaf(gg, frcp(z), wblk);
                                    S[j] = P;
                                    dP[j] = dS;
                                } else {
                                    const float P = fexp2(XB ? (fmaf(S[j], p.sc2, cAz) - m4[e]) - l4[e] : fmaf(S[j], p.sc2, cAz));
                                    const float dS = P * dP[j];
                                    dsum += dS;
                                    if constexpr (CLS == 1) {
                                        const float z = PROD ? fmaf(zq4[e], ck, sv) : sv + fexp2(zq4[e] - rsb);
                                        wblk = fmaf(dS, frcp(z), wblk);
                                    }
                                    S[j] = P;
                                    dP[j] = dS;
                                }
                            }
                        }
                    };
                    using C0 = std::integral_constant<int, 0>;
                    using C1 = std::integral_constant<int, 1>;
                    using C2 = std::integral_constant<int, 2>;
                    if (cls == 2)
                        offdiag(std::true_type{}, C2{});
                    else if (cls == 3)
                        offdiag(std::true_type{}, std::integral_constant<int, 3>{});
                    else if (cls == 1)
                        prod ? offdiag(std::true_type{}, C1{}) : offdiag(std::false_type{}, C1{});
                    else
                        prod ? offdiag(std::true_type{}, C0{}) : offdiag(std::false_type{}, C0{});
                } else {
#pragma unroll
                    for (int jq = 0; jq < 4; ++jq) {
                        const int t4 = 32 * mt + 8 * jq + 4 * g;
                        f32x4 g4, m4, l4;
                        if constexpr (XB) {
                            m4 = *reinterpret_cast<const f32x4 *>(&qi[buf][QI_LQ][t4]);
                            l4 = *reinterpret_cast<const f32x4 *>(&qi[buf][QI_LL][t4]);
                        }
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int j = 4 * jq + e;
                            const int t = ib * BQ + t4 + e;
                            // X is +inf where the range (s, t] is empty (t <= s): there x = +inf, the bias
                            // beff * min(x, 0) is 0 and the gate x <= 0 is off, as for b_tt = 0.
                            const bool valid = (t >= s) && s_valid;  // rows past T have -inf scores: P = 0
                            const float x = X[j] - psi_s;
                            const float bm = beff * fminf(x, 0.f);
                            const float P = !valid ? 0.f
                                            : fexp2(XB ? (fmaf(S[j], p.sc2, bm) - m4[e]) - l4[e] : fmaf(S[j], p.sc2, bm));
                            const float dS = P * dP[j];
                            const float gg = (x <= 0.f) ? dS : 0.f;
                            gsum += gg;
                            if constexpr (XB)
                                dbblk = fmaf(dS, fminf(x, 0.f), dbblk);
                            else
                                dbacc = fmaf(dS, bm, dbacc);
                            g4[e] = gg;
                            S[j] = P;
                            dP[j] = dS;
                        }
                        if (s_valid && scalars) *reinterpret_cast<f32x4 *>(p.gd + ((brow + jb) * G + sr) * G + t4) = g4;
                    }
                }
                // dV^T[d][s] += dO^T[d][t] P[t][s];  dK^T[d][s] += Q^T[d][t] dS[t][s]
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) {
                    dvacc[dt] = mma_p2_p3_pad<T, DT, true>(dvacc[dt], S, Dt, 32 * mt, 32 * (dt0 + dt), lane);
                    dkacc[dt] = mma_p2_p3_pad<T, DT, true>(dkacc[dt], dP, Qt, 32 * mt, 32 * (dt0 + dt), lane);
                }
            }
            if constexpr (XB) dbacc += dbblk;
            if (cls == 1 || cls == 2) {  // the per-key sums of classes 1 and 2
                const bool gate = fminf(suf, mid) <= psi_s;
                gsum += gate ? dsum : 0.f;
                dbacc = fmaf(dsum, XB ? cx : cAz, dbacc);
                wblk = !gate ? 0.f : (cls == 2) ? dsum / sv : wblk;
            }
            if (ib > jb) {  // close query block ib: key-block and middle-block soft-min sums
                if (rs > ninf()) Wacc = fmaf(fexp2(Cs - rs), wblk, Wacc);
                if (ib > jb + 1) tpw = wave_sum((rs > ninf()) ? fexp2(cmid - rs) * wblk : 0.f);
            }
        }
        if (lane == 0) sm.tpx[it & 1][w] = tpw;
        if (wave_active && ib > jb) {  // block ib joins the middle of the blocks after it
            mid = fminf(mid, bm_here);
            midl = lse2_pair(midl, bl_cur);
            cmid = fmaxf(cmid, -bm_here * p.il2);
            rs = fmaxf(Cs, cmid);
            sv = (rs > ninf()) ? fexp2(sufl - rs) + fexp2(midl - rs) : 0.f;
        }
        if constexpr (NS == 1) {  // every wave is done with the tiles: load the next block in their place
            __syncthreads();
            issue(umin_i(ib + 1, p.NB - 1), 0);
        }
        wait_loads();
        __syncthreads();
    }

    flush_tbuf(ibhi - 1, (ibhi - 1 - iblo) & 1);
    // Per-key outputs (lanes c and c + 32 hold the same key, different queries).
    gsum = sum_halves(gsum);
    Wacc = sum_halves(Wacc);
    const float dbw = XB ? wave_sum(dbacc) : wave_sum(dbacc) / beff;
    if (!wave_active) return;
    if constexpr (SPLIT) {
        if (half != 0) {  // partial sums of a split tile (keys < KS < T): raw dK / dV accumulators
            const int hp = half - 1;
            if (lane == 0) p.dbp[((int64_t)hp * p.BH + bh) * p.NK32 + kw0 / 32] = dbw;
            const int64_t ks = ((int64_t)hp * p.BH + bh) * p.KS + s;
            if (g == 0) *reinterpret_cast<f32x2 *>(p.pks + 2 * ks) = f32x2{Wacc, gsum};
            float *row = p.pkv + ks * 2 * D;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int jq = 0; jq < 4; ++jq) {
                    const int d0 = 32 * (dt0 + dt) + 8 * jq + 4 * g;
                    if (d0 < D) {
                        *reinterpret_cast<f32x4 *>(row + d0) = f32x4{dkacc[dt][4 * jq + 0], dkacc[dt][4 * jq + 1],
                                                                     dkacc[dt][4 * jq + 2], dkacc[dt][4 * jq + 3]};
                        *reinterpret_cast<f32x4 *>(row + D + d0) = f32x4{dvacc[dt][4 * jq + 0], dvacc[dt][4 * jq + 1],
                                                                         dvacc[dt][4 * jq + 2], dvacc[dt][4 * jq + 3]};
                    }
                }
            return;
        }
    }
    if (scalars) {
        if (lane == 0) p.dbp[(int64_t)bh * p.NK32 + kw0 / 32] = dbw;  // one partial per 32-key group
        if (g == 0 && s < p.TP) p.wsum[rowbase + s] = Wacc;
        if (g == 0 && s_valid) p.dpsi[(int64_t)bh * p.T + s] = -beta * gsum;
    }
    if (!s_valid) return;
    T *dKr = static_cast<T *>(p.dk) + b * p.sdk.b + h * p.sdk.h + (int64_t)s * p.sdk.t;
    T *dVr = static_cast<T *>(p.dv) + b * p.sdv.b + h * p.sdv.h + (int64_t)s * p.sdv.t;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int jq = 0; jq < 4; ++jq) {
            const int d0 = 32 * (dt0 + dt) + 8 * jq + 4 * g;
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

}  // namespace fpa
