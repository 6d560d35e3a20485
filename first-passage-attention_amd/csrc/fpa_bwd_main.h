// fpa_bwd_main.h -- the single-pass backward tile of First Passage Attention (fp16, D <= 64).
//
// Reference behaviour: _bwd_kv (kernel.py:177-265) and _bwd_q (kernel.py:286-340) of
// yliu-fort/first-passage-attention.  The reference runs a key-side and a query-side kernel that
// both recompute the scores, probabilities and dS of every causal pair.  Here each pair is
// computed once.  A workgroup of MAIN_NW waves owns 32 keys per wave (256 keys) and streams
// 64-query blocks from the keys' diagonal block to T.  Per block and wave it computes, on the
// 32x32 MFMA and the VALU:
//   S = Q K^T, dP = dO V^T, P, dS, the gate g = [x <= 0] dS and the soft-min terms y = g / Z;
//   dV^T += dO^T P, dK^T += Q^T dS (registers, the whole key range of the tile);
//   per key: dpsi, dbeta, W (sums of y over the queries); per block pair: TBUF (sums of y);
//   the in-block gated dS of the diagonal block (gd).
// The two sums over keys, which the query side of the reference computes, come from the same
// values: dS goes to LDS transposed (fp16) and, one block later, a 16x16x32 MFMA pass contracts it
// with K into this tile's partial dQ of the block; the soft-min sums R_t = sum_s y_ts are reduced
// across the 32 key lanes of each wave with DPP / permlane steps and across the waves through
// LDS.  Both partials go to the workspace and the combine kernel adds the tiles' partials in a
// fixed order, so the backward stays deterministic.
//
// Soft-min reference: with Z_ts = 2^SUFL_s + 2^MIDL + 2^PREL_t, one reciprocal per pair serves W,
// R and TBUF when every term is taken relative to one wave-uniform reference rho = max(SUFL of the
// wave's first key, MIDL, BLSE of the query block): z = Z 2^-rho <= 3, and z >= 2^-PROD_SPREAD
// when rho - max(MIDL, a of the block's first query) <= PROD_SPREAD.  Tiles outside that range
// take the exact path: a per-key reference for W and TBUF and a per-query reference for R (two
// reciprocals per pair, as the two-sided formulation).
#pragma once

#include <type_traits>

#include "fpa_bwd_kv.h"
#include "fpa_common.h"
#include "fpa_params.h"

namespace fpa {

constexpr int MAIN_NW = MAIN_BK / 32;  // waves per workgroup of the single-pass backward

// The partial dQ of a block (64 queries x D) is 4 * D / 16 tiles of 16 x 16; each wave with dQ work
// takes NTILE tiles of one 16-wide d range.
template <int D> struct DqSplit {
    static constexpr int ND = D / 16;
    static constexpr int NTILE = (ND * 4 >= MAIN_NW) ? ND * 4 / MAIN_NW : 1;
    static constexpr int NACT = ND * 4 / NTILE;  // waves with dQ work
};

template <int D, int NW>
struct MainShared {
    static constexpr int DT = D < 32 ? 32 : D;
    static constexpr int TB = Pad<f16, DT>::template bytes<64>();  // one padded Q or dO tile
    static constexpr int DSP = 72;  // row pitch of the transposed dS tile in halves (144 bytes)
    __attribute__((aligned(1024))) char Qs[2][TB];
    __attribute__((aligned(1024))) char dOs[2][TB];
    __attribute__((aligned(1024))) float qi[2][QI_PLANES][64];
    __attribute__((aligned(16))) f16 dsT[2][32 * NW][DSP];  // dS^T of a block: [key][query]
    __attribute__((aligned(16))) float rst[2][NW][64];      // per-wave soft-min row sums of a block
    __attribute__((aligned(16))) float kPHI[32 * NW];
    __attribute__((aligned(1024))) char Ks[Pad<f16, DT>::template bytes<32 * NW>()];  // the tile's keys (dQ operand)
};

// 16x16x32 f16 MFMA operand from a natural-layout LDS tile X[krow][n] (pitch in elements): lane l
// gets column n0 + l % 16 of k rows R0 + 8 (l / 16) + 0..7 (two transposing reads of four rows).
__device__ __forceinline__ h8 tr_op16(const f16 *X, int pitch, int R0, int n0, int lane) {
    const int j = lane & 15, q = lane >> 4;
    const f16 *p0 = X + (R0 + 8 * q + (j >> 2)) * pitch + n0 + 4 * (j & 3);
    const h4 lo = ds_read_tr16(p0);
    const h4 hi = ds_read_tr16(p0 + 4 * pitch);
    return h8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Lane exchange partners for the reduce-scatter of the soft-min row sums (rows of 16 lanes).
template <int CTRL> __device__ __forceinline__ float dpp_mov(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// Sums over the 32 key lanes of each half-wave of v[0..15] (register j = query row of the 32x32
// accumulator layout), in a fixed order.  On return lanes c and c ^ 1 of each half hold the sum of
// register c >> 1.  Steps: lane bit 4 (permlane16 swap), then bits 3, 2, 1 (row_mirror,
// row_half_mirror, quad_perm [2,3,0,1]: each pairs lanes across the bit), then bit 0.
__device__ __forceinline__ float rowsum_scatter(const float (&v)[16], int c) {
    float a[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[j]), __float_as_uint(v[j + 8]), false, false);
        a[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);  // bit 4 = 0: register j, else j + 8
    }
    const bool b3 = c & 8, b2 = c & 4, b1 = c & 2;
    float b[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float keep = b3 ? a[j + 4] : a[j], send = b3 ? a[j] : a[j + 4];
        b[j] = keep + dpp_mov<0x140>(send);  // row_mirror: lane 15 - c
    }
    float d[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const float keep = b2 ? b[j + 2] : b[j], send = b2 ? b[j] : b[j + 2];
        d[j] = keep + dpp_mov<0x141>(send);  // row_half_mirror: lane 7 - c within 8
    }
    const float keep = b1 ? d[1] : d[0], send = b1 ? d[0] : d[1];
    const float e = keep + dpp_mov<0x4E>(send);  // quad_perm [2,3,0,1]: lane c ^ 2
    return e + dpp_mov<0xB1>(e);                  // quad_perm [1,0,3,2]: lane c ^ 1
}

// Keys [32 NW kt, 32 NW (kt + 1)) of head bh: every query block from the keys' first diagonal block
// to T.
template <int D, int NW>
__device__ __forceinline__ void bwd_main_tile(const BwdParams &p, MainShared<D, NW> &sm, const int kt, const int bh) {
    using T = f16;
    constexpr int BK = 32 * NW, BQ = 64;
    constexpr int DT = D < 32 ? 32 : D;
    constexpr int NDT = DT / 32;
    constexpr int BPT = BK / G;
    constexpr int DSP = MainShared<D, NW>::DSP;
    using SPL = DqSplit<D>;
    auto &Qs = sm.Qs;
    auto &dOs = sm.dOs;
    auto &qi = sm.qi;
    float *const kPHI = sm.kPHI;

    const int tid = thread_x(), lane = tid % 64, g = lane / 32, c = lane % 32;
    const int w = __builtin_amdgcn_readfirstlane(tid / 64);
    const int b = bh / p.H, h = bh % p.H;
    const int k0 = kt * BK, kw0 = k0 + 32 * w, s = kw0 + c;
    const int jb = kw0 / G, sb = jb * G;
    const bool wave_active = kw0 < p.T;
    const bool s_valid = s < p.T;
    const StateLayout L{p.BH, p.TP, p.NB};
    const int64_t rowbase = (int64_t)bh * p.TP;
    const int64_t brow = (int64_t)bh * p.NB;
    const int64_t per_head = dqp_per_head(p.NB, p.nkt, BPT);

    const T *Qb = static_cast<const T *>(p.q) + b * p.sq.b + h * p.sq.h;
    const T *Kb = static_cast<const T *>(p.k) + b * p.sk.b + h * p.sk.h;
    const T *Vb = static_cast<const T *>(p.v) + b * p.sv.b + h * p.sv.h;
    const T *DOb = static_cast<const T *>(p.dout) + b * p.sdo.b + h * p.sdo.h;
    const float *qi_head = p.qinfo + qi_at(bh, p.NB, 0, 0);

    TileLoader<T, D, DT, BQ, NW> qld, dld;
    qld.init(p.sq.t, w, lane);
    dld.init(p.sdo.t, w, lane);
    const uint32_t aQ = lds_addr(&Qs[0][0]), aD = lds_addr(&dOs[0][0]), aI = lds_addr(&qi[0][0][0]);
    auto issue = [&](int ib, int buf) {
        qld.issue(aQ + buf * sizeof(Qs[0]), Qb, p.sq.t, ib * BQ, p.T, w, lane);
        dld.issue(aD + buf * sizeof(dOs[0]), DOb, p.sdo.t, ib * BQ, p.T, w, lane);
        buf_lds16(buf_rsrc(qi_head + (int64_t)ib * QI_PLANES * 64), 1024 * (w % 2) + 16 * lane,
                  aI + buf * sizeof(qi[0]) + 1024 * (w % 2));
    };
    const int ib0 = k0 / G;
    issue(ib0, 0);

    OpRow<T, D> vreg;  // V in registers; K is read from the resident LDS tile
    load_row_p1<T, D>(vreg, Vb + (int64_t)s * p.sv.t, s_valid, g);

    // The tile's keys stay in LDS for the dQ pass (its K^T operand), loaded with the first block.
    const bool dq_wave = w < SPL::NACT;
    const int dr = (w * SPL::NTILE) / 4, tq0 = (w * SPL::NTILE) % 4;
    const int q16 = lane / 16, i16 = lane % 16;
    {
        TileLoader<T, D, DT, BK, NW> kld;
        kld.init(p.sk.t, w, lane);
        kld.issue(lds_addr(&sm.Ks[0]), Kb, p.sk.t, k0, p.T, w, lane);
    }
    constexpr int KP = Pad<T, DT>::PITCH;

    const float beta = p.beta[h], beff = beta_eff(beta * LOG2E);
    const float E = (beff > 0.f) ? ninf() : pinf();
    float psi_s = 0.f, suf = pinf(), sufl = ninf();
    if (s < p.TP) {
        psi_s = p.state[L.at(PL_PSI, bh, s)];
        suf = p.state[L.at(PL_SUF, bh, s)];
        sufl = p.state[L.at(PL_SUFL, bh, s)];
    }
    const float sufl0 = uniform_f(sufl);  // SUFL of the wave's first key: the largest of the wave
    const float Cs = (suf < pinf()) ? -suf * p.il2 : ninf();
    const float bsuf = beff * suf, bpsi = beff * psi_s;
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

    // Partial dQ and soft-min row sums of block ibp from the staged buffers of iteration itp.
    auto flush = [&](int itp, int ibp) {
        const int pb = itp & 1;
        if (w == 0) {
            float r = 0.f;
#pragma unroll
            for (int v = 0; v < NW; ++v) r += sm.rst[pb][v][lane];
            p.rp[((int64_t)bh * p.nkt + kt) * p.TP + ibp * BQ + lane] = r;
        }
        if (dq_wave) {
            f32x4 acc[SPL::NTILE];
#pragma unroll
            for (int u = 0; u < SPL::NTILE; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
            const f16 *X = &sm.dsT[pb][0][0];
            const f16 *KX = reinterpret_cast<const f16 *>(&sm.Ks[0]);
#pragma unroll 2
            for (int ks = 0; ks < NW; ++ks) {
                const h8 kT = tr_op16(KX, KP, 32 * ks, 16 * dr, lane);  // K^T: rows d, contraction over keys
#pragma unroll
                for (int u = 0; u < SPL::NTILE; ++u)
                    acc[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kT, tr_op16(X, DSP, 32 * ks, 16 * (tq0 + u), lane),
                                                                    acc[u], 0, 0, 0);
            }
            float *dst = p.dqp + dqp_block(bh, kt, ibp, p.NB, BPT, per_head) * (BQ * D);
#pragma unroll
            for (int u = 0; u < SPL::NTILE; ++u)
                *reinterpret_cast<f32x4 *>(dst + (16 * (tq0 + u) + i16) * D + 16 * dr + 4 * q16) = acc[u];
        }
    };

    wait_loads();
    __syncthreads();
    int it = 0;
    for (int ib = ib0; ib < p.NB; ++ib, ++it) {
        const int buf = it & 1;
        issue(umin_i(ib + 1, p.NB - 1), buf ^ 1);
        const float bm_here = qi[buf][QI_BST][0], bl_cur = qi[buf][QI_BST][1];  // block ib
        if (it > 0) flush(it - 1, ib - 1);
        f16 *dsw = &sm.dsT[buf][32 * w + c][0];  // this lane's row (key) of dS^T
        float *rsw = sm.rst[buf][w];
        if (wave_active && ib >= jb) {
            const bool diag = (ib == jb);
            // Soft-min reference of the block (see the file comment).
            float rho = 0.f, ck = 0.f, sv = 0.f, rs = ninf(), rsb = ninf();
            bool prod = false, fast = false;
            if (!diag) {
                prod = uniform_f(qi[buf][QI_ZQ][0]) > 0.f;
                const float prel0 = -uniform_f(qi[buf][QI_PRE][0]) * p.il2;  // a of the block's first query
                rho = fmaxf(fmaxf(sufl0, midl), bl_cur);
                fast = prod && (rho - fmaxf(midl, prel0) <= PROD_SPREAD);
                if (fast) {
                    ck = fexp2(bl_cur - rho);
                    sv = fexp2(sufl - rho) + fexp2(midl - rho);
                } else {
                    rs = fmaxf(Cs, cmid);
                    rsb = rs - bl_cur;
                    ck = fexp2(fminf(-rsb, 126.f));
                    sv = (rs > ninf()) ? fexp2(sufl - rs) + fexp2(midl - rs) : 0.f;
                }
            }
            const float cAz = __builtin_amdgcn_fmed3f(__builtin_amdgcn_fmed3f(bsuf, beff * mid, E) - bpsi, 0.f, E);
            const float thr = (fminf(suf, mid) <= psi_s) ? pinf() : psi_s;
            const float nbpsi = -bpsi;
            const char *Qt = Qs[buf];
            const char *Dt = dOs[buf];
            const float *rPRE = qi[buf][QI_PRE];
            const float *rZQ = qi[buf][QI_ZQ];
            const float *rPREL = qi[buf][QI_PREL];
            const float *rCT = qi[buf][QI_CT];
            const int sr = s - sb;
            float r = pinf();
            float wblk = 0.f;
#pragma unroll 1
            for (int mt = 0; mt < 2; ++mt) {
                // S - lse / sc2: A = Q rows, B = this lane's key row of the resident K tile (rows past T
                // hold row T - 1, whose scores are masked: such keys only occur in the diagonal block).
                f32x16 S = rows16(qi[buf][QI_LQ], mt);
                {
                    const T *qrow = reinterpret_cast<const T *>(Qt) + (32 * mt + c) * Pad<T, DT>::PITCH;
                    const T *krow = reinterpret_cast<const T *>(&sm.Ks[0]) + (32 * w + c) * Pad<T, DT>::PITCH;
#pragma unroll
                    for (int i = 0; i < D / 16; ++i)
                        S = MT<T>::mma(*reinterpret_cast<const h8 *>(qrow + 16 * i + 8 * g),
                                       *reinterpret_cast<const h8 *>(krow + 16 * i + 8 * g), S);
                }
                f32x16 dP = mma_p1_pad_reg<T, D, DT>(rows16(qi[buf][QI_DL], mt), Dt, 32 * mt + c, g, vreg);
                float yv[16];
                if (!diag) {
                    auto offdiag = [&](auto fast_c, auto prod_c) {
                        constexpr bool FAST = decltype(fast_c)::value;
                        constexpr bool PROD = decltype(prod_c)::value;
#pragma unroll
                        for (int jq = 0; jq < 4; ++jq) {
                            const int t4 = 32 * mt + 8 * jq + 4 * g;
                            const f32x4 pre4 = *reinterpret_cast<const f32x4 *>(&rPRE[t4]);
                            const f32x4 zq4 = *reinterpret_cast<const f32x4 *>(&rZQ[t4]);
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                const int j = 4 * jq + e;
                                const float bm = __builtin_amdgcn_fmed3f(fmaf(pre4[e], beff, nbpsi), cAz, E);
                                const float P = fexp2(fmaf(S[j], p.sc2, bm));
                                const float dS = P * dP[j];
                                const float gg = (pre4[e] <= thr) ? dS : 0.f;
                                gsum += gg;
                                dbacc = fmaf(dS, bm, dbacc);
                                const float z = PROD ? fmaf(zq4[e], ck, sv) : sv + fexp2(zq4[e] - rsb);
                                const float y = gg * frcp(z);
                                wblk += y;
                                yv[j] = FAST ? y : gg;
                                S[j] = P;
                                dP[j] = dS;
                            }
                        }
                        if constexpr (!FAST) {
                            // Exact R terms: 2^{c_t} / Z_ts = 1 / (2^{SUFL_s - c_t} + 2^{MIDL - c_t} + 2^{PREL_t - c_t})
                            // with the per-query reference c_t (every exponent is finite or -inf; rows past T
                            // have c_t = PREL_t = 0 and g = 0).
#pragma unroll
                            for (int jq = 0; jq < 4; ++jq) {
                                const int t4 = 32 * mt + 8 * jq + 4 * g;
                                const f32x4 pl4 = *reinterpret_cast<const f32x4 *>(&rPREL[t4]);
                                const f32x4 ct4 = *reinterpret_cast<const f32x4 *>(&rCT[t4]);
#pragma unroll
                                for (int e = 0; e < 4; ++e) {
                                    const float mterm = fexp2(midl - ct4[e]) + fexp2(pl4[e] - ct4[e]);
                                    yv[4 * jq + e] *= frcp(fexp2(sufl - ct4[e]) + mterm);
                                }
                            }
                        }
                    };
                    if (fast)
                        offdiag(std::true_type{}, std::true_type{});
                    else if (prod)
                        offdiag(std::false_type{}, std::true_type{});
                    else
                        offdiag(std::false_type{}, std::false_type{});
                } else {
                    float X[16];
                    diag_x_queries(X, r, phiblk, mt, sr, g);
#pragma unroll
                    for (int jq = 0; jq < 4; ++jq) {
                        const int t4 = 32 * mt + 8 * jq + 4 * g;
                        f32x4 g4;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int j = 4 * jq + e;
                            const int t = ib * BQ + t4 + e;
                            const bool valid = (t >= s) && s_valid;
                            const bool strict = valid && (t > s);
                            const float x = X[j] - psi_s;
                            const float bm = strict ? beff * fminf(x, 0.f) : 0.f;
                            const float P = valid ? fexp2(fmaf(S[j], p.sc2, bm)) : 0.f;
                            const float dS = P * dP[j];
                            const float gg = (strict && x <= 0.f) ? dS : 0.f;
                            gsum += gg;
                            dbacc = fmaf(dS, bm, dbacc);
                            g4[e] = gg;
                            S[j] = P;
                            dP[j] = dS;
                            yv[j] = 0.f;
                        }
                        if (s_valid) *reinterpret_cast<f32x4 *>(p.gd + ((brow + jb) * G + sr) * G + t4) = g4;
                    }
                }
                // fp16 P and dS: operands of dV and dK, and dS^T for the dQ pass.
                h8 ph[2], dh[2];
#pragma unroll
                for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        ph[hf][e] = (f16)S[8 * hf + e];
                        dh[hf][e] = (f16)dP[8 * hf + e];
                    }
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                    *reinterpret_cast<h4 *>(dsw + 32 * mt + 16 * hf + 4 * g) = h4{dh[hf][0], dh[hf][1], dh[hf][2], dh[hf][3]};
                    *reinterpret_cast<h4 *>(dsw + 32 * mt + 16 * hf + 8 + 4 * g) = h4{dh[hf][4], dh[hf][5], dh[hf][6], dh[hf][7]};
                }
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt) {
                    dvacc[dt] = mma_p2h_p3_pad<DT, true>(dvacc[dt], ph, Dt, 32 * mt, 32 * dt, lane);
                    dkacc[dt] = mma_p2h_p3_pad<DT, true>(dkacc[dt], dh, Qt, 32 * mt, 32 * dt, lane);
                }
                // Soft-min row sums of this 32-query tile: lane c holds query row acc_row(c >> 1, g).
                float rsum = 0.f;
                if (!diag) {
                    rsum = rowsum_scatter(yv, c);
                    if (fast) rsum *= fexp2(rCT[32 * mt + acc_row(c >> 1, g)] - rho);  // 2^{c_t - rho}
                }
                if ((c & 1) == 0) rsw[32 * mt + acc_row(c >> 1, g)] = rsum;
            }
            if (!diag) {  // close query block ib: key-block and middle-block soft-min sums
                const float ref = fast ? rho : rs;
                if (ref > ninf()) Wacc = fmaf(fexp2(Cs - ref), wblk, Wacc);
                if (ib > jb + 1) {
                    const float tp = wave_sum((ref > ninf()) ? fexp2(cmid - ref) * wblk : 0.f);
                    if (lane == 0) p.tbuf[((brow + ib) * p.NB + jb) * 2 + ((kw0 / 32) & 1)] = tp;
                }
            }
        } else {
            // Keys after the block (or past T): no pairs.  The dQ pass contracts over every key of
            // the tile, so this wave's rows of dS^T are zero, as are its row sums.
#pragma unroll
            for (int q4 = 0; q4 < 64; q4 += 8)
                *reinterpret_cast<h8 *>(dsw + q4) = h8{};
            rsw[lane] = 0.f;
        }
        if (wave_active && ib > jb) {  // block ib joins the middle of the blocks after it
            mid = fminf(mid, bm_here);
            midl = lse2_pair(midl, bl_cur);
            cmid = fmaxf(cmid, -bm_here * p.il2);
        }
        wait_loads();
        __syncthreads();
    }
    flush(it - 1, p.NB - 1);

    gsum = sum_halves(gsum);
    Wacc = sum_halves(Wacc);
    const float dbw = wave_sum(dbacc) / beff;
    if (!wave_active) return;
    if (lane == 0) p.dbp[(int64_t)bh * p.NK32 + kw0 / 32] = dbw;
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
                h4 kv4 = {(f16)(dkacc[dt][4 * jq + 0] * p.smscale), (f16)(dkacc[dt][4 * jq + 1] * p.smscale),
                          (f16)(dkacc[dt][4 * jq + 2] * p.smscale), (f16)(dkacc[dt][4 * jq + 3] * p.smscale)};
                h4 vv4 = {(f16)dvacc[dt][4 * jq + 0], (f16)dvacc[dt][4 * jq + 1], (f16)dvacc[dt][4 * jq + 2],
                          (f16)dvacc[dt][4 * jq + 3]};
                *reinterpret_cast<h4 *>(dKr + d0) = kv4;
                *reinterpret_cast<h4 *>(dVr + d0) = vv4;
            }
        }
}

}  // namespace fpa
