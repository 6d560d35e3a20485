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
// with C_s = max a over (s, end of U), c_t = max a over [start of U, t], c_U = max a
// over U, cmid(i, j) = max a over blocks j+1..i-1.  The in-block part runs, per
// column s, the recurrences lz(u) = log2 sum_{s<u'<=u} 2^{a_u'},
// lam(u) = g_us + 2^{lz(u) - lz(u+1)} lam(u+1), contribution 2^{a_u - lz(u)} lam(u).
// All sums run in a fixed order: the result is bit-reproducible.
#include "fpa_common.h"
#include "fpa_params.h"

namespace fpa {

constexpr int MAXNB = 2048;

__device__ __forceinline__ float block_sum_256(float x, float *red) {
    red[threadIdx.x] = x;
    __syncthreads();
#pragma unroll
    for (int o = 128; o >= 1; o >>= 1) {
        if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
        __syncthreads();
    }
    const float r = red[0];
    __syncthreads();
    return r;
}

__global__ void __launch_bounds__(NTHREADS) fpa_bwd_combine_kernel(BwdParams p) {
    __shared__ float sA[G], sC[G], sc[G], sW[G], sR[G], sP[G];
    __shared__ float lz[G][G + 1];
    __shared__ float contrib[G][G + 1];
    __shared__ float Amax[MAXNB], Bmax[MAXNB];
    __shared__ float red[NTHREADS];

    const int U = blockIdx.x, bh = blockIdx.y, h = bh % p.H;
    const int tid = threadIdx.x, lane = tid % 64, w = tid / 64;
    const int sb = U * G, last = min(G - 1, p.T - 1 - sb);
    const StateLayout L{p.BH, p.TP, p.NB};
    const int64_t rowbase = (int64_t)bh * p.TP;
    const int64_t brow = (int64_t)bh * p.NB;
    const float il2 = p.il2;

    if (tid < G) {
        const int64_t r = rowbase + sb + tid;
        const float ph = p.state[L.plane(PL_PHI) + r];
        const float suf = p.state[L.plane(PL_SUF) + r];
        const float pre = p.state[L.plane(PL_PRE) + r];
        sA[tid] = (ph < pinf()) ? -ph * il2 : ninf();
        sC[tid] = (suf < pinf()) ? -suf * il2 : ninf();
        sc[tid] = (pre < pinf()) ? -pre * il2 : ninf();
        sW[tid] = p.wsum[r];
        sR[tid] = p.rsum[r];
    }
    const float cU = -p.state[L.bplane(BP_MIN) + brow + U] * il2;
    const int nI = p.NB - 1 - U;
    const int npairs = U * nI;
    if (npairs > 0) {
        if (tid == 0) {
            float run = ninf();
            for (int jb = U - 1; jb >= 0; --jb) {
                Amax[jb] = run;
                run = fmaxf(run, -p.state[L.bplane(BP_MIN) + brow + jb] * il2);
            }
        } else if (tid == 64) {
            float run = ninf();
            for (int ib = U + 1; ib < p.NB; ++ib) {
                Bmax[ib] = run;
                run = fmaxf(run, -p.state[L.bplane(BP_MIN) + brow + ib] * il2);
            }
        }
    }
    __syncthreads();
    float acc = 0.f;
    for (int idx = tid; idx < npairs; idx += NTHREADS) {
        const int jb = idx / nI, ib = U + 1 + idx % nI;
        const float cm = fmaxf(fmaxf(Amax[jb], cU), Bmax[ib]);
        const float *tb = p.tbuf + ((brow + ib) * p.NB + jb) * 2;
        acc += fexp2(cU - cm) * (tb[0] + tb[1]);
    }
    const float SU = block_sum_256(acc, red);

    if (w == 0) {
        // In-block recurrences, one column s per lane.
        const int s = lane;
        const float *gcol = p.gd + ((brow + U) * G + s) * G;
        float run = ninf();
        for (int u = 0; u < G; ++u) {
            if (u > s && u <= last) run = lse2_pair(run, sA[u]);
            lz[s][u] = run;
        }
        float lam = 0.f;
        for (int u = G - 1; u >= 0; --u) {
            float cval = 0.f;
            if (u > s && u <= last) {
                const float rho = (u + 1 <= last) ? fexp2(lz[s][u] - lz[s][u + 1]) : 0.f;
                lam = gcol[u] + rho * lam;
                cval = fexp2(sA[u] - lz[s][u]) * lam;
            }
            contrib[u][s] = cval;
        }
    } else if (w == 1) {
        const int u = lane;
        float v = 0.f;
        if (u <= last) {
            const float au = sA[u];
            float p1 = 0.f, p2 = 0.f;
            for (int s = 0; s < u; ++s) p1 += fexp2(au - sC[s]) * sW[s];
            for (int t = u; t <= last; ++t) p2 += fexp2(au - sc[t]) * sR[t];
            v = p1 + p2 + ((npairs > 0) ? fexp2(au - cU) * SU : 0.f);
        }
        sP[u] = v;
    }
    __syncthreads();
    if (w == 0) {
        const int u = lane;
        if (u <= last) {
            float p4 = 0.f;
            for (int s = 0; s < u; ++s) p4 += contrib[u][s];
            p.dphi[(int64_t)bh * p.T + sb + u] = p.beta[h] * (sP[u] + p4);
        }
    }
}

// dbeta[h] = sum over batches and key-side partials, fixed order.
__global__ void __launch_bounds__(NTHREADS) fpa_bwd_dbeta_kernel(BwdParams p) {
    __shared__ float red[NTHREADS];
    const int h = blockIdx.x;
    const int n = p.NKV * 4;
    float acc = 0.f;
    for (int b = 0; b < p.B; ++b) {
        const float *src = p.dbp + ((int64_t)(b * p.H + h) * p.NKV) * 4;
        for (int i = threadIdx.x; i < n; i += NTHREADS) acc += src[i];
    }
    const float tot = block_sum_256(acc, red);
    if (threadIdx.x == 0) p.dbeta[h] = tot;
}

hipError_t launch_bwd_combine(const BwdParams &p, hipStream_t s) {
    hipLaunchKernelGGL(fpa_bwd_combine_kernel, dim3(p.NB, p.BH), dim3(NTHREADS), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_bwd_dbeta(const BwdParams &p, hipStream_t s) {
    hipLaunchKernelGGL(fpa_bwd_dbeta_kernel, dim3(p.H), dim3(NTHREADS), 0, s, p);
    return hipGetLastError();
}

}  // namespace fpa
