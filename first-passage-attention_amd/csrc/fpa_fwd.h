// fpa_fwd.h -- the forward pass of First Passage Attention, as a kernel template over the operand
// type and head dimension.  fpa_fwd.hip instantiates it for fp32 operands and fpa_fwd16.hip for
// fp16, so that build.py can compile each with the LLVM scheduling strategy that suits it.
//
// Reference behaviour: kernel.py:103-162 (_fwd) of yliu-fort/first-passage-attention.
// gfx950 design: a workgroup of FPA_NW waves owns 32 query rows per wave, streams 64-key tiles
// from the diagonal down to key 0 through double-buffered (single-buffered for fp32 at D = 128 and 256,
// where two stages of the workgroups that share a CU do not fit in LDS), padded LDS tiles filled by
// direct global->LDS loads (one
// barrier per tile), computes S^T = K Q^T and O^T += V^T P^T on the 32x32 MFMA (V^T read from the
// row-major tile with LDS transpose reads), and keeps each query's online-softmax state in its own
// lane.
#pragma once
#include "fpa_common.h"
#include "fpa_params.h"

// Tuning knobs (build-time): waves per SIMD of the D <= 64 forward kernel, fp16 and fp32 (fp32 at D <= 32
// runs three: fwd_wpe).  Three fp16 waves fit in 168 VGPRs each; with 3 workgroups per CU the cfg2 grid
// (768 workgroups) is resident at once.  The fp32 D = 64 kernel needs about 180 VGPRs.
#ifndef FPA_FWD_WPE
#define FPA_FWD_WPE 3
#endif
#ifndef FPA_FWD_WPE32
#define FPA_FWD_WPE32 2
#endif
// The scores of each 32-key half computed just before its softmax instead of both halves' MFMA chains
// interleaved up front: fp16 at D <= 64 (13 fewer live registers at D = 64, 1-4% faster at cfg2) and
// fp32 at D = 256 (see the kernel).
#ifndef FPA_FWD_SPLIT
#define FPA_FWD_SPLIT 1
#endif
// Balance the tiles of the workgroups that share a CU in the first round of dispatch
// (xcd_work_item); 0 keeps the heaviest-first order.
#ifndef FPA_FWD_SNAKE
#define FPA_FWD_SNAKE 1
#endif
// Split the key range of the heaviest half of the row tiles when the launch's workgroups fill at most
// this percentage of the slots (CUs x workgroups per CU); 0 never splits.  Measured on MI355X at
// T = 2048, D = 64 fp16: at half the slots (B2 H12) the split forward with its merge takes 40 against
// 47 us and at two thirds (B2 H16) 45.5 against 48.3; at three quarters (B3 H12) it is 6% slower, at
// one or two full rounds (B4, B8 H12; B2 H8 T4096 fp32) 8-16% slower.
#ifndef FPA_FWD_SPLIT_FILL
#define FPA_FWD_SPLIT_FILL 70
#endif

namespace fpa {

// ---------------------------------------------------------------------------
// Forward.
//
// Per lane: one query t (column c of the 32x32 accumulators) and, per 64-key tile,
// 32 of the keys.  Off the diagonal block the bias is built from three per-key values
// staged in LDS and one per-query value in a register:
//   b2 = med3(A_s, Y_t - P_s, E),  A_s = beta*log2e*min(SUF_s - psi_s, 0),
//   P_s = beta*log2e*psi_s, Y_t = beta*log2e*min(PRE_t, MID), E = -inf (beta >= 0) or +inf,
// which is beta*log2e*min(0, min(SUF_s, MID, PRE_t) - psi_s) for either sign of beta.  With fp32
// operands the staged values are SUF_s and psi_s instead, Y_t = min(PRE_t, MID), and the bias is
// beta*log2e*(min(Y_t, SUF_s, psi_s) - psi_s): the subtraction comes before the scaling.
// On the diagonal block X_ts = min phi(s, t] comes from a scan down the block.
// The running max is only moved when a row's tile max exceeds it by more than 8 (base 2):
// p <= 256 and the O rescale is skipped on most tiles.
// ---------------------------------------------------------------------------
constexpr float RESCALE_SLACK = 8.f;

template <typename T, int D, int WPE, int NW>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
fpa_fwd_kernel(FwdParams p) {
    constexpr int BM = 32 * NW, BN = 64;
    constexpr int DT = D < 32 ? 32 : D;
    constexpr int NDT = DT / 32;
    constexpr int TB = Pad<T, DT>::template bytes<BN>();  // one padded K or V tile
    // Two stages when WPE workgroups' worth of them (K, V and the per-key values) fit a CU's 160 KB.
    constexpr int NS = (WPE * (4 * TB + 2 * 4 * BN * 4) <= 160 * 1024) ? 2 : 1;
    __shared__ __attribute__((aligned(1024))) char Ks[NS][TB];
    __shared__ __attribute__((aligned(1024))) char Vs[NS][TB];
    // Per-key values of a tile: CA, CP (SUF, PSI for fp32), PHI and BST (the block's BMIN at [3][0]).
    __shared__ __attribute__((aligned(1024))) float cst[NS][4][BN];

    const int tid = thread_x(), lane = tid % 64, g = lane / 32, c = lane % 32;
    const int w = __builtin_amdgcn_readfirstlane(tid / 64);  // wave index, uniform across the wave
    const int nqt = (p.T + BM - 1) / BM;
    // Item k of a head (0 the heaviest): with ns split row tiles (rank r < ns, rank 0 the last rows),
    // items 3i and 3i + 1 are parts B and A of rank i and item 3i + 2 is the whole of rank ns + i; the
    // items after 3 ns are ranks 2 ns, 2 ns + 1, ... (nqt >= 2 ns).  part 0: every key of the rows.
    int k, bh;
    xcd_work_item(k, bh, p.BH, p.H, nqt + p.ns, FPA_FWD_SNAKE ? WPE : 1);
    int rank = k - p.ns, part = 0;
    if (k < 3 * p.ns) {
        const int i = k / 3, j = k - 3 * i;
        rank = (j == 2) ? p.ns + i : i;
        part = (j == 2) ? 0 : j + 1;
    }
    const int qt = nqt - 1 - rank;  // longest rows first
    const int b = bh / p.H, h = bh % p.H;
    const int q0 = qt * BM, qw0 = q0 + 32 * w, tq = qw0 + c;
    const int ib = qw0 / G;
    const bool wave_active = qw0 < p.T;
    const StateLayout L{p.BH, p.TP, p.NB};
    const int64_t rowbase = (int64_t)bh * p.TP;

    const T *Qb = static_cast<const T *>(p.q) + b * p.sq.b + h * p.sq.h;
    const T *Kb = static_cast<const T *>(p.k) + b * p.sk.b + h * p.sk.h;
    const T *Vb = static_cast<const T *>(p.v) + b * p.sv.b + h * p.sv.h;
    // Per-key values staged with one 64-lane load: lanes 0-15 CA, 16-31 CP, 32-47 PHI, 48-63 BST (byte
    // offsets from plane 0 of the head; the state planes hold TP >= every tile end rows).
    const float *st_head = p.state + L.at(0, bh, 0);
    constexpr bool XB = exact_bias<T>();
    const int cpl = (lane < 16) ? (XB ? PL_SUF : PL_CA) : (lane < 32) ? (XB ? PL_PSI : PL_CP) : (lane < 48) ? PL_PHI : PL_BST;
    const uint32_t cst_off = (uint32_t)((cpl * p.TP + 4 * (lane & 15)) * 4);

    // Tile jt of K, V and the per-key values into buffer `buf` (shared out over the waves; every wave
    // issues the per-key load, identical writes instead of a wave-dependent branch).  After tile 0
    // the prefetch repeats it into a buffer that is not read again.
    TileLoader<T, D, DT, BN, NW> kld, vld;
    kld.init(p.sk.t, w, lane);
    vld.init(p.sv.t, w, lane);
    const uint32_t aK = lds_addr(&Ks[0][0]), aV = lds_addr(&Vs[0][0]), aC = lds_addr(&cst[0][0][0]);
    auto issue = [&](int jt, int buf) {
        kld.issue(aK + buf * sizeof(Ks[0]), Kb, p.sk.t, jt * BN, p.T, w, lane);
        vld.issue(aV + buf * sizeof(Vs[0]), Vb, p.sv.t, jt * BN, p.T, w, lane);
        buf_lds16(buf_rsrc(st_head + jt * BN), cst_off, aC + buf * sizeof(cst[0]));
    };
    // Inside the loop every tile loaded is below the first one (jt - 1 < jtmax <= nkt - 1): all rows < T.
    auto issue_full = [&](int jt, int buf) {
        kld.issue_full(aK + buf * sizeof(Ks[0]), Kb, p.sk.t, jt * BN, w);
        vld.issue_full(aV + buf * sizeof(Vs[0]), Vb, p.sv.t, jt * BN, w);
        buf_lds16(buf_rsrc(st_head + jt * BN), cst_off, aC + buf * sizeof(cst[0]));
    };

    const int nkt = (p.T + BN - 1) / BN;
    const int jtmax = umin_i(nkt - 1, (q0 + BM - 1) / BN);
    // Key tiles of this item: part B takes jsplit .. jtmax (every diagonal block of the rows: jsplit
    // <= qt + 1 <= 2 qt for the split tiles, qt >= 1), part A the tiles below jsplit, all before q0.
    const int jsplit = (jtmax + 1) >> 1;
    const int jhi = (part == 2) ? jsplit - 1 : jtmax;
    const int jlo = (part == 1) ? jsplit : 0;
    issue(jhi, 0);

    OpRow<T, D> qreg;
    load_row_p1<T, D>(qreg, Qb + (int64_t)tq * p.sq.t, tq < p.T, g);

    const float beta = p.beta[h], betal = beta * LOG2E;
    const float E = (beta >= 0.f) ? ninf() : pinf();
    const float pre_t = (tq < p.TP) ? p.state[L.at(PL_PRE, bh, tq)] : pinf();

    float m_i = ninf(), l_i = 0.f;
    f32x16 oacc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) oacc[dt] = zero16();
    float mid = pinf();  // min phi over the blocks strictly between the key block and ib
    if (part == 2 && wave_active) {  // part A starts below block jsplit: mid covers blocks jsplit .. ib - 1
        const float *bmin = p.state + L.bplane(BP_MIN) + (int64_t)bh * p.NB;
        for (int j0 = jsplit; j0 < ib; j0 += 64) mid = fminf(mid, (j0 + lane < ib) ? bmin[j0 + lane] : pinf());
        mid = wave_min(mid);
    }

    wait_loads();
    __syncthreads();
    for (int jt = jhi, it = 0; jt >= jlo; --jt, ++it) {
        const int buf = (NS == 2) ? (it & 1) : 0;
        const int s0 = jt * BN;
        if constexpr (NS == 2) issue_full(jt > 0 ? jt - 1 : 0, buf ^ 1);
        if (wave_active && s0 <= qw0 + 31) {
            const char *Kt = Ks[buf];
            const float *cA = cst[buf][0], *cP = cst[buf][1], *cPHI = cst[buf][2];
            const int jb = jt;  // BN == G: the key tile is one statistics block
            const bool diag = (jb == ib);
            const float Y = XB ? fminf(pre_t, mid) : betal * fminf(pre_t, mid);
            const int tr = tq - s0;
            float r = pinf();  // running min of phi over [u, t] for the in-block scan
            // Both 32-key halves' scores first; then each half in turn (the second half's MFMAs
            // and the first half's P V run while the other half's VALU work goes on).
            f32x16 s[2];
            // Measured: fp16 at D <= 64 (3 waves per SIMD) and fp32 at D = 256 (20 fewer spilled registers,
            // 3% faster); level or slower for the other shapes.
            constexpr bool SPLIT = FPA_FWD_SPLIT && ((sizeof(T) == 2 && D <= 64) || (sizeof(T) == 4 && D == 256));
            if constexpr (!SPLIT) {
                s[0] = zero16();
                s[1] = zero16();
                mma_p1_pad_reg2<T, D, DT>(s[1], Kt, 32 + c, qreg, s[0], Kt, c, qreg, g);
            }
#pragma unroll
            for (int mt = 1; mt >= 0; --mt) {
                if constexpr (SPLIT) s[mt] = mma_p1_pad_reg<T, D, DT>(zero16(), Kt, 32 * mt + c, g, qreg);
                if (!diag) {
#pragma unroll
                    for (int jq = 0; jq < 4; ++jq) {
                        const int s4 = 32 * mt + 8 * jq + 4 * g;
                        const f32x4 a4 = *reinterpret_cast<const f32x4 *>(&cA[s4]);
                        const f32x4 p4 = *reinterpret_cast<const f32x4 *>(&cP[s4]);
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float b2 = XB ? betal * (fminf(fminf(Y, a4[e]), p4[e]) - p4[e])
                                                : __builtin_amdgcn_fmed3f(a4[e], Y - p4[e], E);
                            s[mt][4 * jq + e] = fmaf(s[mt][4 * jq + e], p.sc2, b2);
                        }
                    }
                } else {
                    // Diagonal block: X_ts = min phi(s, t] inside the block (scan from the top).
                    float X[16];
                    diag_x_keys(X, r, cPHI, mt, tr, g);
#pragma unroll
                    for (int jq = 0; jq < 4; ++jq) {
                        const int s4 = 32 * mt + 8 * jq + 4 * g;
                        const f32x4 p4 = *reinterpret_cast<const f32x4 *>(&cP[s4]);
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const int j = 4 * jq + e, sr = s4 + e;
                            const float bx = XB ? betal * fminf(X[j] - p4[e], 0.f)
                                                : __builtin_amdgcn_fmed3f(0.f, fmaf(betal, X[j], -p4[e]), E);
                            const float b2 = (sr < tr) ? bx : 0.f;  // b_tt = 0
                            const float z = fmaf(s[mt][j], p.sc2, b2);
                            s[mt][j] = (sr > tr || s0 + sr >= p.T) ? ninf() : z;
                        }
                    }
                }

                // Online softmax (base 2) over these 32 keys; lanes c and c + 32 hold the same query.
                float mx = s[mt][0];
#pragma unroll
                for (int j = 1; j < 16; ++j) mx = fmaxf(mx, s[mt][j]);
                mx = max_halves(mx);
                if (__any(mx > m_i + RESCALE_SLACK)) {
                    const float m_new = fmaxf(m_i, mx);
                    const float alpha = fexp2(m_i - m_new);  // 0 on the first update (m_i = -inf)
                    l_i *= alpha;
#pragma unroll
                    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                        for (int j = 0; j < 16; ++j) oacc[dt][j] *= alpha;
                    m_i = m_new;
                }
                // A half with no valid key yet (the upper half of the diagonal block for the lower
                // queries) leaves m_i = -inf: its scores are all -inf and exponentiate to 0.
                const float mref = (m_i > ninf()) ? m_i : 0.f;
                if constexpr (sizeof(T) == 2) {
                    // P in fp16 (the MFMA operand); the row sum adds the same rounded values.
                    h8 ph[2];
                    float rs = 0.f;
#pragma unroll
                    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
                        for (int e = 0; e < 8; e += 2) {
                            const h2 pp = {(f16)fexp2(s[mt][8 * hf + e] - mref), (f16)fexp2(s[mt][8 * hf + e + 1] - mref)};
                            ph[hf][e] = pp[0];
                            ph[hf][e + 1] = pp[1];
                            rs = __builtin_amdgcn_fdot2(pp, h2{(f16)1.f, (f16)1.f}, rs, false);
                        }
                    l_i += sum_halves(rs);
                    // O^T[d][t] += V^T[d][s] P^T[s][t]   (V read transposed from its natural layout)
#pragma unroll
                    for (int dt = 0; dt < NDT; ++dt)
                        oacc[dt] = mma_p2h_p3_pad<DT, true>(oacc[dt], ph, Vs[buf], 32 * mt, 32 * dt, lane);
                } else {
                    float rs = 0.f;
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        const float pv = fexp2(s[mt][j] - mref);
                        s[mt][j] = pv;
                        rs += pv;
                    }
                    l_i += sum_halves(rs);
#pragma unroll
                    for (int dt = 0; dt < NDT; ++dt)
                        oacc[dt] = mma_p2_p3_pad<T, DT, true>(oacc[dt], s[mt], Vs[buf], 32 * mt, 32 * dt, lane);
                }
            }

            if (jb < ib) mid = fminf(mid, cst[buf][3][0]);  // BMIN of block jb
        }
        if constexpr (NS == 1) {  // every wave is done with the tile: load the next one in its place
            __syncthreads();
            issue_full(jt > 0 ? jt - 1 : 0, 0);
        }
        wait_loads();
        __syncthreads();
    }

    if (!wave_active) return;
    const float inv = 1.f / l_i;
    // Split rows: the part's output normalised by its own sum (part B into o, part A into ows) and its
    // running maximum and sum (oml); the merge kernel writes the rows' o and lse.
    const int64_t srow = (int64_t)bh * (p.T - p.rs0) + (tq - p.rs0);
    if (tq < p.T) {
        T *Orow = (part == 2) ? static_cast<T *>(p.ows) + srow * D
                              : static_cast<T *>(p.o) + b * p.so.b + h * p.so.h + (int64_t)tq * p.so.t;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int jq = 0; jq < 4; ++jq) {
                const int d0 = 32 * dt + 8 * jq + 4 * g;
                if (d0 < D) {
                    if constexpr (sizeof(T) == 2) {
                        h4 v4 = {(f16)(oacc[dt][4 * jq + 0] * inv), (f16)(oacc[dt][4 * jq + 1] * inv),
                                 (f16)(oacc[dt][4 * jq + 2] * inv), (f16)(oacc[dt][4 * jq + 3] * inv)};
                        *reinterpret_cast<h4 *>(Orow + d0) = v4;
                    } else {
                        f32x4 v4 = {oacc[dt][4 * jq + 0] * inv, oacc[dt][4 * jq + 1] * inv,
                                    oacc[dt][4 * jq + 2] * inv, oacc[dt][4 * jq + 3] * inv};
                        *reinterpret_cast<f32x4 *>(Orow + d0) = v4;
                    }
                }
            }
    }
    if (part != 0) {  // rows past T (up to TP) get the whole-row values from part B
        if (tq < p.T) {
            if (g == 0) *reinterpret_cast<f32x2 *>(p.oml + 4 * srow + 2 * (part - 1)) = f32x2{m_i, l_i};
            return;
        }
        if (part == 2) return;
    }
    if (g == 0 && tq < p.TP) {
        if constexpr (XB) {  // fp32: the running maximum and log2 l, for the backward's P = 2^{(s - m) - log2 l}
            p.lse[rowbase + tq] = m_i;
            p.lse[(int64_t)p.BH * p.TP + rowbase + tq] = flog2(l_i);
        } else {
            p.lse[rowbase + tq] = m_i + flog2(l_i);
        }
    }
}

// Rows of a split row tile: o = (wB oB + wA oA) / (wB + wA) with w = l 2^{m - max(mA, mB)} from the two
// parts' normalised outputs, and the row's lse (fp32: the running maximum and log2 of the sum).  One
// thread per 16-byte chunk of a row.
template <typename T, int D>
__global__ void __launch_bounds__(256) fpa_fwd_merge_kernel(FwdParams p) {
    constexpr int CH = 16 / (int)sizeof(T), CPR = D / CH;  // elements per chunk, chunks per row
    const int64_t nsr = p.T - p.rs0;
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t row = gid / CPR;
    if (row >= (int64_t)p.BH * nsr) return;
    const int ch = (int)(gid - row * CPR);
    const int bh = (int)(row / nsr), t = p.rs0 + (int)(row - (int64_t)bh * nsr);
    const int b = bh / p.H, h = bh % p.H;
    const f32x4 ml = *reinterpret_cast<const f32x4 *>(p.oml + 4 * row);
    const float m = fmaxf(ml[0], ml[2]);
    const float wb = ml[1] * fexp2(ml[0] - m), wa = ml[3] * fexp2(ml[2] - m);
    const float l = wa + wb, inv = 1.f / l;
    T *orow = static_cast<T *>(p.o) + b * p.so.b + h * p.so.h + (int64_t)t * p.so.t + ch * CH;
    const T *arow = static_cast<const T *>(p.ows) + row * D + ch * CH;
    if constexpr (sizeof(T) == 2) {
        h8 ob = *reinterpret_cast<const h8 *>(orow), oa = *reinterpret_cast<const h8 *>(arow), out;
#pragma unroll
        for (int e = 0; e < 8; ++e) out[e] = (f16)(((float)ob[e] * wb + (float)oa[e] * wa) * inv);
        *reinterpret_cast<h8 *>(orow) = out;
    } else {
        f32x4 ob = *reinterpret_cast<const f32x4 *>(orow), oa = *reinterpret_cast<const f32x4 *>(arow), out;
#pragma unroll
        for (int e = 0; e < 4; ++e) out[e] = (ob[e] * wb + oa[e] * wa) * inv;
        *reinterpret_cast<f32x4 *>(orow) = out;
    }
    if (ch == 0) {
        const int64_t li = (int64_t)bh * p.TP + t;
        if constexpr (exact_bias<T>()) {
            p.lse[li] = m;
            p.lse[(int64_t)p.BH * p.TP + li] = flog2(l);
        } else {
            p.lse[li] = m + flog2(l);
        }
    }
}

// Waves per SIMD of the forward.  At D = 128 two fit: fp16 in 236 VGPRs with no spills and two LDS
// stages of K and V (70 KB per workgroup), fp32 in 256 with one register spilled outside the tile loop
// and one stage (67 KB).  Against one wave per SIMD, whose 512-register budget the compiler had filled
// (332 and 352 VGPRs): fp16 121 -> 85 us and fp32 531 -> 461 us at B4 H12 T2048, fp32 629 -> 593 us
// at B2 H8 T4096.  fp32 at D <= 32 fits three (141 and 152 VGPRs, no spills): 6-7% faster than two at
// B4 H12 T2048 and B2 H8 T4096.
template <typename T, int D>
constexpr int fwd_wpe() {
    return (D == 128) ? 2 : (D >= 128) ? 1 : (sizeof(T) == 2 ? FPA_FWD_WPE : (D <= 32 ? 3 : FPA_FWD_WPE32));
}

template <typename T, int D>
static hipError_t launch_fwd_t(const FwdParams &p, hipStream_t s) {
    constexpr int NW = FPA_NW, WPE = fwd_wpe<T, D>();
    const int nqt = (p.T + 32 * NW - 1) / (32 * NW);
    hipLaunchKernelGGL((fpa_fwd_kernel<T, D, WPE, NW>), head_grid(nqt + p.ns, p.H, p.BH), dim3(64 * NW), 0, s, p);
    return hipGetLastError();
}

template <typename T, int D>
static hipError_t launch_fwd_merge_t(const FwdParams &p, hipStream_t s) {
    const int64_t threads = (int64_t)p.BH * (p.T - p.rs0) * (D / (16 / (int)sizeof(T)));
    hipLaunchKernelGGL((fpa_fwd_merge_kernel<T, D>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, p);
    return hipGetLastError();
}

// fp16 instantiations (fpa_fwd16.hip).
hipError_t launch_fwd_f16(const FwdParams &p, int D, hipStream_t s);
hipError_t launch_fwd_merge_f16(const FwdParams &p, int D, hipStream_t s);

}  // namespace fpa
