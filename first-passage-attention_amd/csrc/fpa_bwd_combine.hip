// fpa_bwd_combine.hip -- the soft-min gradient of phi and the dbeta reduction.
//
// Reference behaviour: _bwd_dphi_diag (kernel.py:268-283), _bwd_dphi (kernel.py:343-370)
// and the dbeta sum of kernel.py:450 (yliu-fort/first-passage-attention).
//
// For position u in block U (base-2, a_u = -phi_u log2(e) / tau):
//   dphi_u = beta * ( sum_{s<u, s in U}  2^{a_u - C_s} W_s          key-block part
//                   + sum_{t>=u, t in U} 2^{a_u - c_t} R_t          query-block part
//                   + 2^{a_u - c_U} sum_{j<U<i} 2^{c_U - cmid(i,j)} TBUF[i][j]   middle blocks
//                   + sum_{s<u<=t, s,t in U} g_ts 2^{a_u} / Z_ts )  in-block pairs
// with C_s = max a over (s, end of U), c_t = max a over [start of U, t], c_U = max a over U,
// cmid(i, j) = max a over blocks j+1..i-1.
//
// In-block pairs, per column s: with m(u) = max a over (s, u] and
// Z(u) = sum_{s<v<=u} 2^{a_v - m(u)} (>= 1), the forward chain is
// Z(u) = Z(u-1) 2^{m(u-1) - m(u)} + 2^{a_u - m(u)}, and the reverse chain
// lam(u) = g_us + rho(u) lam(u+1) with rho(u) = Z(u) 2^{m(u) - m(u+1)} / Z(u+1) gives the
// contribution 2^{a_u - m(u)} lam(u) / Z(u) to u.  Only FMAs sit on the dependent chains,
// and the 64 steps are split over the four waves of the workgroup.  When a spans at most
// INBLOCK_SPREAD binades over the block, one reference (the block maximum c_U) serves every
// column instead: Z(u) 2^{-c_U} is a running sum of positive terms 2^{a_v - c_U}, and the
// contribution to u is 2^{a_u - c_U} sum_{t>=u} g_ts 2^{c_U} / Z(t) (one reciprocal per pair
// instead of the chains' exponentials), and the key-block and query-block parts become sums of
// per-position terms 2^{c_U - C_s} W_s and 2^{c_U - c_t} R_t times 2^{a_u - c_U}.
//
// The middle-block sum runs over every pair (i, j) around U (below MID_SCAN_NB blocks per head) or
// over the prefix sums that fpa_bwd_mid_kernel leaves per query block i (from MID_SCAN_NB on), already
// scaled to 2^{c_U}: then the combine holds no per-block array and any number of blocks fits.
//
// dbeta[h] is summed (fixed order) by the workgroup of block 0 of batch 0 of head h.
// All sums run in a fixed order: the result is bit-reproducible.
#include "fpa_common.h"
#include "fpa_params.h"

namespace fpa {

// Largest spread of a over a block (binades) for the single-reference in-block sums.
constexpr float INBLOCK_SPREAD = 100.f;

// Maximum over an array of n values held in LDS, scanned by one wave: out[i] = max of in[i..hi)
// (suffix) or of in(lo..i] (prefix), with elements outside [lo, hi) treated as -inf.  Each lane
// scans a contiguous chunk; chunk maxima are combined across lanes with shuffles.
__device__ __forceinline__ void wave_suffix_max(float *out, const float *in, int n, int hi, int lane) {
    const int k = (n + 63) / 64, i0 = lane * k;
    float run = ninf();
    for (int j = min(i0 + k, n) - 1; j >= i0; --j) {
        run = fmaxf(run, (j < hi) ? in[j] : ninf());
        out[j] = run;
    }
    // exclusive suffix maximum of the lanes' chunk maxima
    float x = run;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float y = __shfl_down(x, o, 64);
        if (lane + o < 64) x = fmaxf(x, y);
    }
    float excl = __shfl_down(x, 1, 64);
    if (lane == 63) excl = ninf();
    for (int j = i0; j < min(i0 + k, n); ++j) out[j] = fmaxf(out[j], excl);
}
__device__ __forceinline__ void wave_prefix_max(float *out, const float *in, int n, int lo, int lane) {
    const int k = (n + 63) / 64, i0 = lane * k;
    float run = ninf();
    for (int j = i0; j < min(i0 + k, n); ++j) {
        run = fmaxf(run, (j > lo) ? in[j] : ninf());
        out[j] = run;
    }
    float x = run;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float y = __shfl_up(x, o, 64);
        if (lane >= o) x = fmaxf(x, y);
    }
    float excl = __shfl_up(x, 1, 64);
    if (lane == 0) excl = ninf();
    for (int j = i0; j < min(i0 + k, n); ++j) out[j] = fmaxf(out[j], excl);
}

// Sum of x over the 256 threads in a fixed order (every call site is reached by all threads).
__device__ __forceinline__ float block_sum_256(float x, float *red, int w, int lane) {
    x = wave_sum(x);
    if (lane == 0) red[w] = x;
    __syncthreads();
    const float r = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return r;
}

// From this many blocks per head on, the middle-block sums run in O(NB^2) per head: the mid kernel
// below turns each row of TBUF into prefix sums first, and the combine reads one sum per query block.
// Below it the combine sums every (query block, key block) pair around each block, O(NB^3 / 6) per
// head, which costs less than a second launch (measured: the two break even between 128 and 192
// blocks at H12).
constexpr int MID_SCAN_NB = 160;

// Row i (query block) of a head's TBUF holds V(i, j) = 2^{cmid(i, j)} M(i, j) for key blocks j <= i - 2,
// M(i, j) the middle-block soft-min sum of the block pair and cmid(i, j) = max a over blocks j+1 .. i-1.
// The middle-block part of dphi in block U needs S_U = sum_{j < U < i} M(i, j).  With
// m_U = max a over blocks U .. i-1 (c_b = max a over block b), the row's prefix sums
//   Q_i(U) = 2^{m_U} sum_{j < U} M(i, j),   U = 1 .. i - 1,
// follow Q_i(U + 1) = 2^{m_{U+1} - m_U} Q_i(U) + V(i, U) from Q_i(0) = 0, every factor at most 1, and
// S_U 2^{c_U} = sum_{i > U} 2^{c_U - m_U} Q_i(U).  One wave per row: each lane takes a segment of U,
// composes the segment's affine map (going down, with m_U as a running maximum), the maps are scanned
// across the lanes, and each lane reruns its segment upward from the value entering it.
// 2^{c_U - m_U} Q_i(U) (a factor at most 1) goes to the upper triangle of the head's TBUF matrix (row U,
// column i > U), which the key side never writes; the m_U values are parked there between the two
// passes.  Up to MID_LDS_NB blocks the c_b of the head are staged in LDS, beyond that read from memory.
constexpr int MID_LDS_NB = 8192;

template <bool LDS>
__global__ void __launch_bounds__(NTHREADS) fpa_bwd_mid_kernel(BwdParams p) {
    __shared__ float cbs[LDS ? MID_LDS_NB : 1];  // c_b for the head's blocks
    const int bh = group_bh(p.H), tid = thread_x(), lane = tid % 64;
    const int w = __builtin_amdgcn_readfirstlane(tid / 64);
    const int NB = p.NB;
    const int64_t brow = (int64_t)bh * NB;
    const StateLayout L{p.BH, p.TP, p.NB};
    const float *bmin = p.state + L.bplane(BP_MIN) + brow;
    const int i = __builtin_amdgcn_readfirstlane(group_x() * (NTHREADS / 64) + w);  // this wave's row
    if constexpr (LDS) {
        for (int b = tid; b < NB; b += NTHREADS) cbs[b] = -bmin[b] * p.il2;
        __syncthreads();
    }
    auto cb = [&](int b) { return LDS ? cbs[b] : -bmin[b] * p.il2; };
    if (i < 2 || i >= NB) return;  // wave-uniform: rows 0 and 1 have no pair
    const float *V = p.tbuf + (brow + i) * NB;  // V(i, U) = V[U], U <= i - 2
    float *col = p.tbuf + brow * NB + i;        // Q_i(U) = col[U * NB]
    const int n = i - 1;                        // steps U = 0 .. n - 1
    const int k = (n + 63) / 64, lo = min(lane * k, n), hi = min(lo + k, n);
    // m_hi = max(c_hi .. c_{i-1}): the maxima of the later lanes' segments and c_{i-1}.
    float smax = ninf();
    for (int U = lo; U < hi; ++U) smax = fmaxf(smax, cb(U));
    float x = smax;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float y = __shfl_down(x, o, 64);
        if (lane + o < 64) x = fmaxf(x, y);
    }
    float mhi = __shfl_down(x, 1, 64);
    if (lane == 63) mhi = ninf();
    mhi = fmaxf(mhi, cb(i - 1));
    // Pass 1, down the segment: the composed map Q(hi) = A Q(lo) + B; m_U parked for lo < U < hi.
    float A = 1.f, B = 0.f, mnext = mhi;
    for (int U = hi - 1; U >= lo; --U) {
        const float m = fmaxf(cb(U), mnext);
        B = fmaf(V[U], A, B);
        A *= fexp2(mnext - m);
        if (U > lo) col[(int64_t)U * NB] = m;
        mnext = m;
    }
    const float mlo = mnext;
    // Inclusive scan of the maps over the lanes (lane 0 first), then the value entering each segment.
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float Ap = __shfl_up(A, o, 64), Bp = __shfl_up(B, o, 64);
        if (lane >= o) {
            B = fmaf(A, Bp, B);
            A *= Ap;
        }
    }
    float q = __shfl_up(B, 1, 64);
    if (lane == 0) q = 0.f;
    // Pass 2, up the segment: Q(U + 1) = 2^{m_{U+1} - m_U} Q(U) + V(i, U), stored times 2^{c_{U+1} - m_{U+1}}.
    float m = mlo;
    for (int U = lo; U < hi; ++U) {
        const float mn = (U + 1 < hi) ? col[(int64_t)(U + 1) * NB] : mhi;
        q = fmaf(fexp2(mn - m), q, V[U]);
        col[(int64_t)(U + 1) * NB] = fexp2(cb(U + 1) - mn) * q;
        m = mn;
    }
}

// Dynamic LDS: sBM, scanA, scanB, NB floats each, below MID_SCAN_NB blocks (none from there on).
__global__ void __launch_bounds__(NTHREADS) fpa_bwd_combine_kernel(BwdParams p) {
    extern __shared__ float dyn[];
    __shared__ float sA[G], sC[G], sc[G], sW[G], sR[G];
    __shared__ float segM[4][G], segZ[4][G], segM2[4][G], segZ2[4][G], segA[4][G], segB[4][G], pp[4][G];
    __shared__ float contrib[G][G + 1];      // [u][s]; before that, the block's gd tile as [s][t]
    __shared__ float sF[G], sH[G];           // single-reference key-block and query-block terms
    __shared__ float sE[G];                  // 2^{a_u - c_U} (0 past the block's last position)
    __shared__ float red[4];

    const int U = group_x(), bh = group_bh(p.H), b = bh / p.H, h = bh % p.H;
    const int tid = thread_x(), lane = tid % 64;
    const int w = __builtin_amdgcn_readfirstlane(tid / 64);
    const int sb = U * G, last = min(G - 1, p.T - 1 - sb);
    const StateLayout L{p.BH, p.TP, p.NB};
    const int64_t rowbase = (int64_t)bh * p.TP;
    const int64_t brow = (int64_t)bh * p.NB;
    const float il2 = p.il2;
    const int NB = p.NB;
    float *sBM = dyn, *scanA = dyn + NB, *scanB = dyn + 2 * NB;

    // The block's gated in-block dS tile (gd, [s][t], 16 KB), loaded first so that the latency overlaps
    // the setup below: 16-byte pieces in order (each wave instruction reads 1 KB of contiguous memory),
    // staged in `contrib` (pitch G + 1: the column reads below are free of bank conflicts) before the
    // first barrier.  A piece with no pair s < t (every t <= s) is never read and is not loaded.
    f32x4 gl[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = tid + NTHREADS * i, s = q >> 4, t0 = 4 * (q & 15);
        gl[i] = (t0 + 3 > s) ? reinterpret_cast<const f32x4 *>(p.gd + (brow + U) * G * G)[q] : f32x4{0.f, 0.f, 0.f, 0.f};
    }

    if (U == 0 && b == 0) {  // dbeta[h] = sum over batches and key-side partials
        const int n = p.NK32;
        float acc = 0.f;
        for (int bb = 0; bb < p.B; ++bb) {
            const float *src = p.dbp + (int64_t)(bb * p.H + h) * p.NK32;
            for (int i = tid; i < n; i += NTHREADS) acc += src[i];
        }
        const float tot = block_sum_256(acc, red, w, lane);
        if (tid == 0) p.dbeta[h] = tot;
    }

    if (tid < G) {
        const int64_t r = rowbase + sb + tid;
        const float ph = p.state[L.at(PL_PHI, bh, sb + tid)];
        const float suf = p.state[L.at(PL_SUF, bh, sb + tid)];
        const float pre = p.state[L.at(PL_PRE, bh, sb + tid)];
        sA[tid] = (ph < pinf()) ? -ph * il2 : ninf();
        sC[tid] = (suf < pinf()) ? -suf * il2 : ninf();
        sc[tid] = (pre < pinf()) ? -pre * il2 : ninf();
        sW[tid] = p.wsum[r];
        sR[tid] = p.rsum[r];
        {
            // c_U = max a over the block = -BMIN * log2(e) / tau (the value sBM[U] holds below).  No
            // FMA contraction here, so that the exponent is the one the LDS values give.
#pragma clang fp contract(off)
            const float cu = -p.state[L.bplane(BP_MIN) + brow + U] * il2;
            const float au = (ph < pinf()) ? -ph * il2 : ninf();
            sE[tid] = (tid <= last) ? fexp2(au - cu) : 0.f;
        }
    }
    const bool midscan = NB >= MID_SCAN_NB;  // uniform
    if (!midscan)
        for (int i = tid; i < NB; i += NTHREADS) sBM[i] = -p.state[L.bplane(BP_MIN) + brow + i] * il2;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int q = tid + NTHREADS * i, s = q >> 4, t0 = 4 * (q & 15);
#pragma unroll
        for (int e = 0; e < 4; ++e) contrib[s][t0 + e] = gl[i][e];
    }
    __syncthreads();
    // This lane's 16 values: column s = lane, rows u in [16w, 16w + 16).  Read before any wave writes
    // contrib again (after at least one more barrier).
    float gq[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) gq[k] = contrib[lane][16 * w + k];
    const float cU = -ld_uniform(p.state, L.bplane(BP_MIN) + brow + U) * il2;  // sBM[U]
    const int nI = NB - 1 - U;
    // (query block after U, key block before U) pairs: some exist when U > 0 and nI > 0; their count is
    // needed only by the pair loop below MID_SCAN_NB blocks, where it is small (at most (NB / 2)^2).
    const bool haspairs = U > 0 && nI > 0;
    const int npairs = midscan ? 0 : U * nI;
    float SU = 0.f;
    if (haspairs) {  // uniform: U is the workgroup's block
        // scanA[i] = max over [i, U), scanB[i] = max over (U, i]; waves 0 and 1 in parallel.
        if (!midscan) {
            if (w == 0) wave_suffix_max(scanA, sBM, NB, U, lane);
            if (w == 1) wave_prefix_max(scanB, sBM, NB, U, lane);
            __syncthreads();
        }
        // cmid(ib, jb) = max(A_jb, c_U, B_ib), A_jb = max over (jb, U) = scanA[jb + 1],
        // B_ib = max over (U, ib) = scanB[ib - 1].  Consecutive threads read consecutive jb.
        float acc = 0.f;
        if (midscan) {  // S_U 2^{c_U} = sum_{i > U} 2^{c_U - m_U(i)} Q_i(U), the terms as the mid pass left them
            const float *qrow = p.tbuf + (brow + U) * NB;  // at column i of row U
            for (int ib = U + 1 + tid; ib < NB; ib += NTHREADS) acc += qrow[ib];
        } else if (npairs <= NTHREADS) {  // uniform: one pair per thread at most
            if (tid < npairs) {
                const int ib = U + 1 + tid / U, jb = tid % U;
                const float cm = fmaxf(fmaxf(scanA[jb + 1], cU), scanB[ib - 1]);
                acc = fexp2(cU - cm) * p.tbuf[(brow + ib) * NB + jb];
            }
        } else {
            // Pair idx = (ib - U - 1) * U + jb, stepped by NTHREADS without a division per step; four
            // steps' loads are issued before their terms are added (in the order of idx).
            const int dq = NTHREADS / U, dr = NTHREADS - dq * U;
            int ib = U + 1 + tid / U, jb = tid % U;
            constexpr int UNR = 4;
            for (int idx = tid; idx < npairs; idx += UNR * NTHREADS) {
                float tv[UNR];
                int ibv[UNR], jbv[UNR];
#pragma unroll
                for (int r = 0; r < UNR; ++r) {
                    const bool ok = idx + r * NTHREADS < npairs;
                    ibv[r] = ok ? ib : U + 1;  // in range for the scans below; the term is 0
                    jbv[r] = ok ? jb : 0;
                    tv[r] = ok ? p.tbuf[(brow + ib) * NB + jb] : 0.f;
                    jb += dr;
                    ib += dq;
                    if (jb >= U) {
                        jb -= U;
                        ++ib;
                    }
                }
#pragma unroll
                for (int r = 0; r < UNR; ++r) {
                    const float cm = fmaxf(fmaxf(scanA[jbv[r] + 1], cU), scanB[ibv[r] - 1]);
                    acc += fexp2(cU - cm) * tv[r];
                }
            }
        }
        SU = block_sum_256(acc, red, w, lane);
    }

    // Spread of a over the block (cU is its maximum): a single reference for the in-block soft-min
    // sums when it is small.
    const float amin = wave_min((lane <= last) ? sA[lane] : pinf());
    const bool fast = cU - amin <= INBLOCK_SPREAD;  // uniform over the workgroup
    if (fast) {
        // Every term of Z relative to 2^{c_U}: e_v = 2^{a_v - c_U} >= 2^-INBLOCK_SPREAD, so the running
        // sums Z'(u) = sum_{s<v<=u} e_v are sums of positive terms that cannot underflow, and the
        // contribution to u of column s is e_u sum_{t>=u} g_ts / Z'(t).  Lane s owns column s,
        // wave w the steps u in [16w, 16w + 16); segment sums are joined through LDS.
        const int s = lane, u0 = 16 * w;
        if (w == 0) {  // key-block and query-block terms relative to c_U (C_s, c_t <= c_U)
            const bool vs = s <= last;
            sF[s] = (vs && sC[s] > ninf()) ? fexp2(cU - sC[s]) * sW[s] : 0.f;
            sH[s] = vs ? fexp2(cU - sc[s]) * sR[s] : 0.f;
        }
        float ev[16], Zs = 0.f;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int u = u0 + k;
            ev[k] = (u > s) ? sE[u] : 0.f;  // sE is 0 past the last position
            Zs += ev[k];
        }
        segZ[w][s] = Zs;
        __syncthreads();
        float Z = 0.f;
        for (int v = 0; v < w; ++v) Z += segZ[v][s];  // the sum entering this segment
        float qv[16], Qs = 0.f;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            Z += ev[k];
            qv[k] = (ev[k] > 0.f) ? gq[k] * frcp(Z) : 0.f;
            Qs += qv[k];
        }
        segA[w][s] = Qs;
        __syncthreads();
        float rev = 0.f;
        for (int v = 3; v > w; --v) rev += segA[v][s];  // sum of g / Z' beyond this segment
#pragma unroll
        for (int k = 15; k >= 0; --k) {
            rev += qv[k];
            contrib[u0 + k][s] = ev[k] * rev;
        }
    } else {
    // In-block pairs.  Lane s owns column s; wave w owns the steps u in [16w, 16w + 16).
    // Each wave runs its segment of both chains locally, the segments are joined through LDS
    // (forward states combine associatively, reverse affine maps compose), and each wave then
    // reruns its segment from the joined state.  Running maxima keep every term representable
    // whatever the spread of a.
        const int s = lane, u0 = 16 * w;
        float m = ninf(), Z = 0.f;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int u = u0 + k;
            if (u > s && u <= last) {
                const float mn = fmaxf(m, sA[u]);
                Z = fmaf(Z, fexp2(m - mn), fexp2(sA[u] - mn));
                m = mn;
            }
        }
        segM[w][s] = m;
        segZ[w][s] = Z;
        __syncthreads();
        m = ninf();
        Z = 0.f;
        for (int v = 0; v < w; ++v) {  // state entering this segment
            const float m2 = segM[v][s], z2 = segZ[v][s];
            if (m2 > ninf()) {
                const float mn = fmaxf(m, m2);
                Z = fmaf(Z, fexp2(m - mn), z2 * fexp2(m2 - mn));
                m = mn;
            }
        }
        float mv[16], zv[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const int u = u0 + k;
            if (u > s && u <= last) {
                const float mn = fmaxf(m, sA[u]);
                Z = fmaf(Z, fexp2(m - mn), fexp2(sA[u] - mn));
                m = mn;
            }
            mv[k] = m;
            zv[k] = Z;
        }
        segM2[w][s] = mv[0];
        segZ2[w][s] = zv[0];
        __syncthreads();
        const float mnext = (w < 3) ? segM2[w + 1][s] : 0.f;
        const float znext = (w < 3) ? segZ2[w + 1][s] : 1.f;
        float rho[16], gv[16];
        float lam = 0.f, Bc = 1.f;
#pragma unroll
        for (int k = 15; k >= 0; --k) {
            const int u = u0 + k;
            rho[k] = 0.f;
            gv[k] = 0.f;
            if (u > s && u <= last) {
                const float m1 = (k < 15) ? mv[k + 1] : mnext;
                const float z1 = (k < 15) ? zv[k + 1] : znext;
                rho[k] = (u < last) ? zv[k] * fexp2(mv[k] - m1) * frcp(z1) : 0.f;
                gv[k] = gq[k];
                lam = fmaf(rho[k], lam, gv[k]);
                Bc *= rho[k];
            }
        }
        segA[w][s] = lam;
        segB[w][s] = Bc;
        __syncthreads();
        lam = 0.f;
        for (int v = 3; v > w; --v) lam = fmaf(segB[v][s], lam, segA[v][s]);  // lambda entering from above
#pragma unroll
        for (int k = 15; k >= 0; --k) {
            const int u = u0 + k;
            float cval = 0.f;
            if (u > s && u <= last) {
                lam = fmaf(rho[k], lam, gv[k]);
                cval = fexp2(sA[u] - mv[k]) * frcp(zv[k]) * lam;
            }
            contrib[u][s] = cval;
        }
    }
    __syncthreads();  // contrib complete
    {
        // Key-block, query-block and in-block parts: lane u, wave w sums its 16 of the 64 terms
        // of each.
        const int u = lane, v0 = 16 * w;
        float part = 0.f, p4 = 0.f;
        if (u <= last) {
            const float au = sA[u];
            if (fast) {  // 2^{a_u - c_U} (sum_{v<u} sF[v] + sum_{v>=u} sH[v])
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    const int v = v0 + k;
                    if (v < u) {
                        part += sF[v];
                        p4 += contrib[u][v];
                    }
                    if (v >= u && v <= last) part += sH[v];
                }
                part *= sE[u];
            } else {
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    const int v = v0 + k;
                    if (v < u) {
                        part = fmaf(fexp2(au - sC[v]), sW[v], part);
                        p4 += contrib[u][v];
                    }
                    if (v >= u && v <= last) part = fmaf(fexp2(au - sc[v]), sR[v], part);
                }
            }
        }
        pp[w][u] = part + p4;
    }
    __syncthreads();
    if (w == 0) {
        const int u = lane;
        if (u <= last) {
            float tot = ((pp[0][u] + pp[1][u]) + (pp[2][u] + pp[3][u]));
            if (haspairs) tot += fexp2(sA[u] - cU) * SU;
            p.dphi[(int64_t)bh * p.T + sb + u] = p.beta[h] * tot;
        }
    }
}

hipError_t launch_bwd_combine(const BwdParams &p, hipStream_t s) {
    const size_t dyn = (p.NB < MID_SCAN_NB) ? 3 * (size_t)p.NB * sizeof(float) : 0;  // below 2 KB
    if (p.NB >= MID_SCAN_NB) {
        const dim3 grid = head_grid((p.NB + NTHREADS / 64 - 1) / (NTHREADS / 64), p.H, p.BH);
        if (p.NB <= MID_LDS_NB)
            hipLaunchKernelGGL(fpa_bwd_mid_kernel<true>, grid, dim3(NTHREADS), 0, s, p);
        else
            hipLaunchKernelGGL(fpa_bwd_mid_kernel<false>, grid, dim3(NTHREADS), 0, s, p);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(fpa_bwd_combine_kernel, head_grid(p.NB, p.H, p.BH), dim3(NTHREADS), dyn, s, p);
    return hipGetLastError();
}

}  // namespace fpa
