// fpa_field.hip -- the Field prologue of the FirstPassageAttention layer, forward and backward.
//
// Reference behaviour: Field.forward (kernel.py:502-509) of yliu-fort/first-passage-attention:
//   (delta, g, h) = x W^T + b in fp32 (W: 3H x C), W_t = cumsum_t delta_t,
//   phi = W + g, psi = W + h, per (batch, head);
// and the gradient torch's autograd takes through it (kernel.py relies on autograd).
//
// The projection has only 3H outputs per position (36 for H = 12), so it is a pass over x
// (HBM-bound) rather than a GEMM for the matrix cores.  A lane owns one position and the waves
// of a workgroup split the features; the weights, the same for every lane, are scalar loads
// used as SGPR operands, so no LDS traffic feeds the FMAs.  The projection is written per
// (batch, output) along t, so the cumulative sum over t reads contiguous rows.  Backward: a
// reverse cumulative sum gives d(delta); dx = d(lin) W is the same pass the other way round;
// dW = d(lin)^T x (and dbias, as a feature of ones) is summed in a fixed order (per-split
// partials, then one ordered reduction), so reruns are bit-identical.
#include <type_traits>

#include "fpa_common.h"
#include "fpa_params.h"

namespace fpa {

namespace {

constexpr int FT = 64;  // positions per workgroup (one per lane)

template <typename TX> __device__ __forceinline__ float to_f(TX v) { return (float)v; }
__device__ __forceinline__ int imin(int a, int b) { return a < b ? a : b; }  // per lane

// Inclusive scan of one value per thread over a 256-thread workgroup (fixed order).
__device__ __forceinline__ float block_scan256(float v, float *red) {
    const int tid = thread_x(), lane = tid % 64, w = tid / 64;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const float u = __shfl_up(v, o, 64);
        if (lane >= o) v += u;
    }
    if (lane == 63) red[w] = v;
    __syncthreads();
    float off = 0.f;
    for (int i = 0; i < w; ++i) off += red[i];
    __syncthreads();
    return v + off;
}

}  // namespace

// fp32 32x32x2 MFMA, A[m][k] x B[k][n] per wave: lane l gives A[l % 32][l / 32] and B[l / 32][l % 32];
// register j of the 32x32 accumulator holds row 8 (j / 4) + 4 (l / 32) + j % 4, column l % 32.
__device__ __forceinline__ f32x16 mma_f32(float a, float b, f32x16 c) { return MT<float>::mma(a, b, c); }

// A 64-position x 16-feature block of x passes through a wave-private LDS tile of pitch XP floats:
// global memory is read with lane = (feature l % 16, position l / 16 + 4 i), 64 contiguous bytes
// per position, and the MFMA operands are read from it with lane = position.
constexpr int XP = 20;

// lin[b][o][t] = sum_c x[b][t][c] W[o][c] + bias[o] on the MFMA.  Grid (ceil(T / 64), B), NWF waves:
// wave w owns features [w CS, (w + 1) CS) (CS a multiple of 16) for all 64 positions (two M tiles)
// and NT * 32 >= NO outputs (N tiles).  Per 16-feature block, k step ks contracts features
// c + ks (lanes 0-31) and c + 8 + ks (lanes 32-63): A from the staged x tile, B = W (vector loads,
// the next block's loaded during the current block's products, like x).  The NWF partial sums of
// a position meet in LDS and are added in wave order.
template <typename TX, int NT, int NWF>
__global__ void __launch_bounds__(64 * NWF) fpa_field_proj_kernel(FieldParams p) {
    constexpr int NOP = 32 * NT, RP = FT + 1;
    constexpr int RED = NWF * NOP * RP, STG = NWF * FT * XP;
    __shared__ __attribute__((aligned(16))) float lds[RED > STG ? RED : STG];
    const int tid = thread_x(), lane = tid % 64, g = lane / 32, c32 = lane % 32;
    const int w = __builtin_amdgcn_readfirstlane(tid / 64);
    const int b = group_y(), t0 = group_x() * FT, t = t0 + lane;
    const int CS = ((p.C + NWF - 1) / NWF + 15) / 16 * 16;
    const int ca = umin_i(w * CS, p.C), cb = umin_i(ca + CS, p.C);
    const TX *xb = static_cast<const TX *>(p.x) + (int64_t)b * p.sxb;
    float *xs = lds + w * FT * XP;
    const int lf = lane % 16, lr = lane / 16;
    f32x16 acc[2][NT];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = zero16();
    float xn[16], wn[NT][8];
    auto load = [&](int c) {  // x block and W block at features c .. c + 15 (zeros past cb or NO)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = lr + 4 * i, cc = c + lf;
            xn[i] = (t0 + r < p.T && cc < cb) ? to_f(xb[(int64_t)(t0 + r) * p.sxt + cc]) : 0.f;
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int o = 32 * nt + c32;
            const float *wr = p.w + (int64_t)(o < p.NO ? o : 0) * p.C;
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                const int cc = c + 8 * g + ks;
                wn[nt][ks] = (o < p.NO && cc < cb) ? wr[cc] : 0.f;
            }
        }
    };
    int c = ca;
    if (c < cb) load(c);
    for (; c < cb; c += 16) {
#pragma unroll
        for (int i = 0; i < 16; ++i) xs[(lr + 4 * i) * XP + lf] = xn[i];
        float wv[NT][8];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) wv[nt][ks] = wn[nt][ks];
        __builtin_amdgcn_wave_barrier();
        float xa[2][8];
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const f32x4 v = *reinterpret_cast<const f32x4 *>(&xs[(32 * mt + c32) * XP + 8 * g + 4 * q]);
#pragma unroll
                for (int e = 0; e < 4; ++e) xa[mt][4 * q + e] = v[e];
            }
        if (c + 16 < cb) load(c + 16);
#pragma unroll
        for (int ks = 0; ks < 8; ++ks)
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = mma_f32(xa[mt][ks], wv[nt][ks], acc[mt][nt]);
        __builtin_amdgcn_wave_barrier();
    }
    __syncthreads();  // staging tiles done; the same LDS now takes the partial sums, [w][o][position]
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int j = 0; j < 16; ++j)
                lds[(w * NOP + 32 * nt + c32) * RP + 32 * mt + 8 * (j / 4) + 4 * g + j % 4] = acc[mt][nt][j];
    __syncthreads();
    if (t >= p.T) return;
    for (int o = w; o < p.NO; o += NWF) {
        float v = 0.f;
#pragma unroll
        for (int k = 0; k < NWF; ++k) v += lds[(k * NOP + o) * RP + lane];
        p.lin[((int64_t)b * p.NO + o) * p.T + t] = v + p.bias[o];
    }
}

// phi = cumsum_t(delta) + g, psi = cumsum_t(delta) + h for one (b, h) per workgroup (256 threads,
// each a contiguous run of positions).
__global__ void __launch_bounds__(256) fpa_field_scan_kernel(FieldParams p) {
    __shared__ float red[4];
    const int bh = group_x(), b = bh / p.H, h = bh % p.H;
    const int tid = thread_x();
    const int per = (p.T + 255) / 256, ta = imin(tid * per, p.T), tb = imin(ta + per, p.T);
    const float *dl = p.lin + ((int64_t)b * p.NO + h) * p.T;
    const float *gl = p.lin + ((int64_t)b * p.NO + p.H + h) * p.T;
    const float *hl = p.lin + ((int64_t)b * p.NO + 2 * p.H + h) * p.T;
    float s = 0.f;
    for (int t = ta; t < tb; ++t) s += dl[t];
    float run = block_scan256(s, red) - s;  // sum of the runs before this thread's
    float *phi = p.phi + (int64_t)bh * p.T, *psi = p.psi + (int64_t)bh * p.T;
    for (int t = ta; t < tb; ++t) {
        run += dl[t];
        phi[t] = run + gl[t];
        psi[t] = run + hl[t];
    }
}

// Backward of the scan: d(delta)_t = sum_{u >= t} (dphi_u + dpsi_u), dg = dphi, dh = dpsi, written
// to lin position-major, d(lin)[b][t][o], so that a position's NO values are contiguous.
__global__ void __launch_bounds__(256) fpa_field_bwd_scan_kernel(FieldParams p) {
    __shared__ float red[4];
    const int bh = group_x(), b = bh / p.H, h = bh % p.H;
    const int tid = thread_x();
    // Thread tid takes the tid-th run counted from the end, so the scan runs from T down to 0.
    const int per = (p.T + 255) / 256;
    const int tb = p.T - imin(tid * per, p.T), ta = p.T - imin(tid * per + per, p.T);
    const float *dphi = p.dphi + (int64_t)bh * p.T, *dpsi = p.dpsi + (int64_t)bh * p.T;
    float s = 0.f;
    for (int t = tb - 1; t >= ta; --t) s += dphi[t] + dpsi[t];
    float run = block_scan256(s, red) - s;
    float *dl = p.lin + (int64_t)b * p.T * p.NO;  // d(lin) position-major: [b][t][o]
    for (int t = tb - 1; t >= ta; --t) {
        const float a = dphi[t], c = dpsi[t];
        run += a + c;
        dl[(int64_t)t * p.NO + h] = run;
        dl[(int64_t)t * p.NO + p.H + h] = a;
        dl[(int64_t)t * p.NO + 2 * p.H + h] = c;
    }
}

// dx[b][t][c] = sum_o d(lin)[b][t][o] W[o][c] on the MFMA.  Grid (ceil(T / 64), B), NWF waves: the
// workgroup's 64 positions' gradients (NO per position, KS = NO / 2 rounded up k steps) are staged in
// LDS once; wave w owns 32-feature N tiles [w CS, (w + 1) CS).  Per N tile and k step: A = d(lin)
// (positions x outputs 2 ks, 2 ks + 1) from LDS, B = W rows 2 ks, 2 ks + 1 at 32 consecutive
// features (one 128-byte load per lane group).  The accumulator rows are positions and its columns
// features, so dx is stored straight from it, 32 consecutive features per row.
template <typename TX, int KS, int NWF>
__global__ void __launch_bounds__(64 * NWF) fpa_field_dx_kernel(FieldParams p) {
    __shared__ float dls[FT][2 * KS + 1];
    const int tid = thread_x(), lane = tid % 64, g = lane / 32, c32 = lane % 32;
    const int w = __builtin_amdgcn_readfirstlane(tid / 64);
    const int b = group_y(), t0 = group_x() * FT;
    for (int i = tid; i < FT * 2 * KS; i += 64 * NWF) {
        const int r = i / (2 * KS), o = i % (2 * KS);
        dls[r][o] = (o < p.NO && t0 + r < p.T) ? p.lin[((int64_t)b * p.T + t0 + r) * p.NO + o] : 0.f;
    }
    __syncthreads();
    const int CS = ((p.C + NWF - 1) / NWF + 31) / 32 * 32;
    const int ca = umin_i(w * CS, p.C), cb = umin_i(ca + CS, p.C);
    TX *dxb = static_cast<TX *>(p.dx) + (int64_t)b * p.sdxb;
    for (int c = ca; c < cb; c += 32) {
        const int cc = c + c32;
        float wb[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int o = 2 * ks + g;
            wb[ks] = (o < p.NO && cc < cb) ? p.w[(int64_t)o * p.C + cc] : 0.f;
        }
        f32x16 acc[2] = {zero16(), zero16()};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)  // A: this lane's position 32 mt + c32, output 2 ks + g
                acc[mt] = mma_f32(dls[32 * mt + c32][2 * ks + g], wb[ks], acc[mt]);
        if (cc < cb) {
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int r = 32 * mt + 8 * (j / 4) + 4 * g + j % 4;
                    if (t0 + r < p.T) dxb[(int64_t)(t0 + r) * p.sdxt + cc] = (TX)acc[mt][j];
                }
        }
    }
}

// Partial dW and dbias over one split of the B*T positions on the MFMA: part[s][o][c] = sum_{n in
// split s} d(lin)[n][o] x[n][c] for c < C, and the same with x = 1 at c = C (the bias).  Grid
// (ceil((C + 1) / 64), S), 4 waves, each a quarter of the split's positions; per k step two
// positions (lanes 0-31: n, lanes 32-63: n + 1): A = d(lin)^T (outputs x positions, 128-byte rows
// of the position-major gradient), B = x (positions x 64 features, two N tiles).  The four
// quarters meet in LDS in wave order.
template <typename TX, int MT>
__global__ void __launch_bounds__(256) fpa_field_dw_kernel(FieldParams p) {
    constexpr int NOP = 32 * MT, RP = 64 + 1;
    __shared__ float red[4][NOP][RP];
    const int tid = thread_x(), lane = tid % 64, g = lane / 32, c32 = lane % 32;
    const int w = __builtin_amdgcn_readfirstlane(tid / 64);
    const int c0 = group_x() * 64, s = group_y();
    const int N = p.B * p.T;  // fpa_field_bwd checks B * T < 2^31
    const int per = (N + p.S - 1) / p.S, q = ((per + 3) / 4 + 1) / 2 * 2;  // even: whole k steps
    const int na = umin_i(s * per + w * q, N), lim = umin_i(s * per + per, N);
    const int nb = umin_i(na + q, lim);
    f32x16 acc[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt][0] = acc[mt][1] = zero16();
    if (na < nb) {
        // This lane's position n = n0 + g as (batch, t), advanced two positions per k step.
        int bl = (na + g) / p.T, tl = (na + g) % p.T;
        const TX *x = static_cast<const TX *>(p.x);
        constexpr int KU = 4;  // k steps whose loads are issued together
        for (int n0 = na; n0 < nb; n0 += 2 * KU) {
            float av[KU][MT], bv[KU][2];
#pragma unroll
            for (int u = 0; u < KU; ++u) {
                const int n = n0 + 2 * u + g;
                const bool nv = n < nb;
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const int o = 32 * mt + c32;
                    av[u][mt] = (nv && o < p.NO) ? p.lin[(int64_t)n * p.NO + o] : 0.f;
                }
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
                    const int cc = c0 + 32 * nt + c32;
                    float v = 0.f;
                    if (nv) v = (cc < p.C) ? to_f(x[(int64_t)bl * p.sxb + (int64_t)tl * p.sxt + cc]) : (cc == p.C ? 1.f : 0.f);
                    bv[u][nt] = v;
                }
                tl += 2;
                while (tl >= p.T) {  // at most twice (T >= 1)
                    tl -= p.T;
                    ++bl;
                }
            }
#pragma unroll
            for (int u = 0; u < KU; ++u)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) acc[mt][nt] = mma_f32(av[u][mt], bv[u][nt], acc[mt][nt]);
        }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
            for (int j = 0; j < 16; ++j) red[w][32 * mt + 8 * (j / 4) + 4 * g + j % 4][32 * nt + c32] = acc[mt][nt][j];
    __syncthreads();
    const int c = c0 + lane;
    if (c > p.C) return;
    for (int o = w; o < p.NO; o += 4)
        p.part[((int64_t)s * p.NO + o) * (p.C + 1) + c] = (red[0][o][lane] + red[1][o][lane]) + (red[2][o][lane] + red[3][o][lane]);
}

// dW[o][c] (c < C) and dbias[o] (c = C) = sum_s part[s][o][c] in a fixed order: 256 threads take 64
// entries, wave w the splits s = w mod 4, and the four wave sums are added in wave order.
__global__ void __launch_bounds__(256) fpa_field_reduce_kernel(FieldParams p) {
    __shared__ float red[4][64];
    const int tid = thread_x(), lane = tid % 64, w = tid / 64;
    const int64_t i = (int64_t)group_x() * 64 + lane;
    const int64_t C1 = p.C + 1, n = p.NO * C1;
    float a = 0.f;
    if (i < n)
        for (int s = w; s < p.S; s += 4) a += p.part[(int64_t)s * n + i];
    red[w][lane] = a;
    __syncthreads();
    if (w != 0 || i >= n) return;
    a = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
    const int o = (int)(i / C1), c = (int)(i % C1);
    if (c < p.C)
        p.dw[(int64_t)o * p.C + c] = a;
    else
        p.dbias[o] = a;
}

// ---------------------------------------------------------------------------------------------

template <typename TX>
static hipError_t field_fwd_t(const FieldParams &p, hipStream_t s) {
    const dim3 grid((p.T + FT - 1) / FT, p.B);
    if (p.NO <= 32) hipLaunchKernelGGL((fpa_field_proj_kernel<TX, 1, 8>), grid, dim3(512), 0, s, p);
    else if (p.NO <= 64) hipLaunchKernelGGL((fpa_field_proj_kernel<TX, 2, 8>), grid, dim3(512), 0, s, p);
    else hipLaunchKernelGGL((fpa_field_proj_kernel<TX, 3, 4>), grid, dim3(256), 0, s, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(fpa_field_scan_kernel, dim3(p.B * p.H), dim3(256), 0, s, p);
    return hipGetLastError();
}

template <typename TX>
static hipError_t field_bwd_t(const FieldParams &p, hipStream_t s) {
    hipLaunchKernelGGL(fpa_field_bwd_scan_kernel, dim3(p.B * p.H), dim3(256), 0, s, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (p.dx != nullptr) {
        const dim3 grid((p.T + FT - 1) / FT, p.B);
        if (p.NO <= 12) hipLaunchKernelGGL((fpa_field_dx_kernel<TX, 6, 8>), grid, dim3(512), 0, s, p);
        else if (p.NO <= 24) hipLaunchKernelGGL((fpa_field_dx_kernel<TX, 12, 8>), grid, dim3(512), 0, s, p);
        else if (p.NO <= 36) hipLaunchKernelGGL((fpa_field_dx_kernel<TX, 18, 8>), grid, dim3(512), 0, s, p);
        else if (p.NO <= 48) hipLaunchKernelGGL((fpa_field_dx_kernel<TX, 24, 8>), grid, dim3(512), 0, s, p);
        else hipLaunchKernelGGL((fpa_field_dx_kernel<TX, 48, 4>), grid, dim3(256), 0, s, p);  // registers
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    const dim3 gw((p.C + 1 + 63) / 64, p.S);
    if (p.NO <= 32) hipLaunchKernelGGL((fpa_field_dw_kernel<TX, 1>), gw, dim3(256), 0, s, p);
    else if (p.NO <= 64) hipLaunchKernelGGL((fpa_field_dw_kernel<TX, 2>), gw, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((fpa_field_dw_kernel<TX, 3>), gw, dim3(256), 0, s, p);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(fpa_field_reduce_kernel, dim3((p.NO * (p.C + 1) + 63) / 64), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_field_fwd(const FieldParams &p, int dtype, hipStream_t s) {
    return dtype == 0 ? field_fwd_t<f16>(p, s) : field_fwd_t<float>(p, s);
}

hipError_t launch_field_bwd(const FieldParams &p, int dtype, hipStream_t s) {
    return dtype == 0 ? field_bwd_t<f16>(p, s) : field_bwd_t<float>(p, s);
}

}  // namespace fpa
