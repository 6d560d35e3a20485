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

// A 64-position x 16-feature block of x (or of dx) passes through a wave-private LDS tile of
// pitch XP floats: global memory is read (written) with lane = (feature l % 16, position l / 16 +
// 4 i), 64 contiguous bytes per position, and the FMAs read (write) it with lane = position.
constexpr int XP = 20;
constexpr int DWG = 8;  // positions per step of the dW kernel

// W[o][c .. c + 15] as 16 scalar loads (one s_load_dwordx16), or, in the last block of a row,
// clamped to column C - 1 (those weights multiply zeros).
template <bool TAIL>
__device__ __forceinline__ float wv16(const float *w, int C, int row, int c, int j) {
    if constexpr (TAIL)
        return ld_uniform(w, (int64_t)row * C + (c + j < C ? c + j : C - 1));
    else
        return ld_uniform(w + (int64_t)row * C + c, j);
}

// lin[b][o][t] = sum_c x[b][t][c] W[o][c] + bias[o].  Grid (ceil(T / 64), B), NWF waves of 64
// lanes: lane = position, wave w = features [w CS, (w + 1) CS) (CS a multiple of 16).  W is read
// with scalar loads, so each weight is an SGPR operand of 64 lanes' FMAs; the NWF partial sums of a
// position meet in LDS and are added in wave order.  NOP >= NO outputs (a compile-time bound).
template <typename TX, int NOP, int NWF>
__global__ void __launch_bounds__(64 * NWF) fpa_field_proj_kernel(FieldParams p) {
    constexpr int RED = NWF * NOP * FT, STG = NWF * FT * XP;
    __shared__ __attribute__((aligned(16))) float lds[RED > STG ? RED : STG];
    const int tid = thread_x(), lane = tid % 64;
    const int w = __builtin_amdgcn_readfirstlane(tid / 64);
    const int b = group_y(), t0 = group_x() * FT, t = t0 + lane;
    const int CS = ((p.C + NWF - 1) / NWF + 15) / 16 * 16;
    const int ca = umin_i(w * CS, p.C), cb = umin_i(ca + CS, p.C);
    const TX *xb = static_cast<const TX *>(p.x) + (int64_t)b * p.sxb;
    float *xs = lds + w * FT * XP;
    const int lf = lane % 16, lr = lane / 16;
    float acc[NOP];
#pragma unroll
    for (int o = 0; o < NOP; ++o) acc[o] = 0.f;
    // The next block's x is loaded into registers while the current block's FMAs run.
    float xn[16];
    auto load = [&](int c) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = lr + 4 * i, cc = c + lf;
            xn[i] = (t0 + r < p.T && cc < cb) ? to_f(xb[(int64_t)(t0 + r) * p.sxt + cc]) : 0.f;
        }
    };
    auto block = [&](auto tail_c, int c) {
        constexpr bool TAIL = decltype(tail_c)::value;
#pragma unroll
        for (int i = 0; i < 16; ++i) xs[(lr + 4 * i) * XP + lf] = xn[i];
        __builtin_amdgcn_wave_barrier();
        float xv[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const f32x4 v = *reinterpret_cast<const f32x4 *>(&xs[lane * XP + 4 * q]);
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[4 * q + e] = v[e];
        }
        if (c + 16 < cb) load(c + 16);
#pragma unroll
        for (int o = 0; o < NOP; ++o) {
            const int row = umin_i(o, p.NO - 1);  // rows past NO: discarded
#pragma unroll
            for (int j = 0; j < 16; ++j) acc[o] = fmaf(xv[j], wv16<TAIL>(p.w, p.C, row, c, j), acc[o]);
        }
        __builtin_amdgcn_wave_barrier();
    };
    int c = ca;
    if (c < cb) load(c);
    for (; c + 16 <= cb; c += 16) block(std::false_type{}, c);
    if (c < cb) block(std::true_type{}, c);
    __syncthreads();  // staging tiles done; the same LDS now takes the partial sums
#pragma unroll
    for (int o = 0; o < NOP; ++o) lds[(w * NOP + o) * FT + lane] = acc[o];
    __syncthreads();
    if (t >= p.T) return;
    for (int o = w; o < p.NO; o += NWF) {
        float v = 0.f;
#pragma unroll
        for (int k = 0; k < NWF; ++k) v += lds[(k * NOP + o) * FT + lane];
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

// dx[b][t][c] = sum_o d(lin)[b][t][o] W[o][c].  Grid (ceil(T / 64), B), NWF waves: lane =
// position (its NO gradients staged in LDS, then in registers), wave w = features [w CS, (w + 1)
// CS); W rows by scalar loads, 16 features at a time; dx leaves through the staging tile.
template <typename TX, int NOP, int NWF>
__global__ void __launch_bounds__(64 * NWF) fpa_field_dx_kernel(FieldParams p) {
    __shared__ float dls[FT][NOP + 1];
    __shared__ __attribute__((aligned(16))) float stg[NWF * FT * XP];
    const int tid = thread_x(), lane = tid % 64;
    const int w = __builtin_amdgcn_readfirstlane(tid / 64);
    const int b = group_y(), t0 = group_x() * FT;
    for (int i = tid; i < FT * NOP; i += 64 * NWF) {
        const int r = i / NOP, o = i % NOP;
        dls[r][o] = (o < p.NO && t0 + r < p.T) ? p.lin[((int64_t)b * p.T + t0 + r) * p.NO + o] : 0.f;
    }
    __syncthreads();
    float dl[NOP];
#pragma unroll
    for (int o = 0; o < NOP; ++o) dl[o] = dls[lane][o];
    const int CS = ((p.C + NWF - 1) / NWF + 15) / 16 * 16;
    const int ca = umin_i(w * CS, p.C), cb = umin_i(ca + CS, p.C);
    TX *dxb = static_cast<TX *>(p.dx) + (int64_t)b * p.sdxb;
    float *xs = stg + w * FT * XP;
    const int lf = lane % 16, lr = lane / 16;
    auto block = [&](auto tail_c, int c) {
        constexpr bool TAIL = decltype(tail_c)::value;
        float acc[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[j] = 0.f;
#pragma unroll
        for (int o = 0; o < NOP; ++o) {
            const int row = umin_i(o, p.NO - 1);  // dl[o] = 0 past NO
#pragma unroll
            for (int j = 0; j < 16; ++j) acc[j] = fmaf(dl[o], wv16<TAIL>(p.w, p.C, row, c, j), acc[j]);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
            *reinterpret_cast<f32x4 *>(&xs[lane * XP + 4 * q]) = f32x4{acc[4 * q], acc[4 * q + 1], acc[4 * q + 2], acc[4 * q + 3]};
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int r = lr + 4 * i, cc = c + lf;
            const float v = xs[r * XP + lf];
            if (t0 + r < p.T && cc < cb) dxb[(int64_t)(t0 + r) * p.sdxt + cc] = (TX)v;
        }
        __builtin_amdgcn_wave_barrier();
    };
    int c = ca;
    for (; c + 16 <= cb; c += 16) block(std::false_type{}, c);
    if (c < cb) block(std::true_type{}, c);
}

// Partial dW and dbias over one split of the B*T positions: part[s][o][c] = sum_{n in split s}
// d(lin)[n][o] x[n][c] for c < C, and the same with x = 1 at c = C (the bias).  Grid
// (ceil((C + 1) / 64), S), 4 waves: lane = feature, wave w = a quarter of the split's positions,
// DWG positions at a time (their x loads in flight together); a position's NO gradients are
// scalar loads.  The four quarters meet in LDS in wave order.
template <typename TX, int NOP>
__global__ void __launch_bounds__(256) fpa_field_dw_kernel(FieldParams p) {
    __shared__ float red[4][NOP][64];
    const int tid = thread_x(), lane = tid % 64;
    const int w = __builtin_amdgcn_readfirstlane(tid / 64);
    const int c = group_x() * 64 + lane, s = group_y();
    const int N = p.B * p.T;  // fpa_field_bwd checks B * T < 2^31
    const int per = (N + p.S - 1) / p.S, q = (per + 3) / 4;
    const int na = umin_i(s * per + w * q, N), lim = umin_i(s * per + per, N);
    const int nb = umin_i(na + q, lim);
    float acc[NOP];
#pragma unroll
    for (int o = 0; o < NOP; ++o) acc[o] = 0.f;
    if (na < nb) {
        int b = __builtin_amdgcn_readfirstlane(na / p.T), t = __builtin_amdgcn_readfirstlane(na % p.T);
        const TX *x = static_cast<const TX *>(p.x);
        float xn[DWG];  // the next step's x, loaded while the current step's FMAs run
        auto load = [&](int n0) {
#pragma unroll
            for (int j = 0; j < DWG; ++j) {
                float v = 0.f;
                if (n0 + j < nb) v = (c < p.C) ? to_f(x[(int64_t)b * p.sxb + (int64_t)t * p.sxt + c]) : (c == p.C ? 1.f : 0.f);
                xn[j] = v;
                if (++t == p.T) {  // next position
                    t = 0;
                    ++b;
                }
            }
        };
        load(na);
        for (int n0 = na; n0 < nb; n0 += DWG) {
            float xv[DWG];
#pragma unroll
            for (int j = 0; j < DWG; ++j) xv[j] = xn[j];
            if (n0 + DWG < nb) load(n0 + DWG);
#pragma unroll
            for (int j = 0; j < DWG; ++j) {
                // Positions past the split have x = 0; outputs o >= NO read the next position's
                // values (the region is padded) and are discarded.
                const float *dlr = p.lin + (int64_t)umin_i(n0 + j, nb - 1) * p.NO;
#pragma unroll
                for (int o = 0; o < NOP; ++o) acc[o] = fmaf(ld_uniform(dlr, o), xv[j], acc[o]);
            }
        }
    }
#pragma unroll
    for (int o = 0; o < NOP; ++o) red[w][o][lane] = acc[o];
    __syncthreads();
    if (c > p.C) return;
    for (int o = w; o < p.NO; o += 4)
        p.part[((int64_t)s * p.NO + o) * (p.C + 1) + c] = (red[0][o][lane] + red[1][o][lane]) + (red[2][o][lane] + red[3][o][lane]);
}

// dW[o][c] (c < C) and dbias[o] (c = C) = sum_s part[s][o][c], in split order.
__global__ void __launch_bounds__(256) fpa_field_reduce_kernel(FieldParams p) {
    const int64_t i = (int64_t)group_x() * 256 + thread_x();
    const int64_t C1 = p.C + 1;
    if (i >= p.NO * C1) return;
    float a = 0.f;
    for (int s = 0; s < p.S; ++s) a += p.part[(int64_t)s * p.NO * C1 + i];
    const int o = (int)(i / C1), c = (int)(i % C1);
    if (c < p.C)
        p.dw[(int64_t)o * p.C + c] = a;
    else
        p.dbias[o] = a;
}

// ---------------------------------------------------------------------------------------------

// Outputs rounded up to a compile-time bound (NO = 3H <= 96).
#define FIELD_NO_DISPATCH(CALL)            \
    do {                                   \
        if (p.NO <= 12) CALL(12);          \
        else if (p.NO <= 24) CALL(24);     \
        else if (p.NO <= 36) CALL(36);     \
        else if (p.NO <= 48) CALL(48);     \
        else CALL(96);                     \
    } while (0)

template <typename TX>
static hipError_t field_fwd_t(const FieldParams &p, hipStream_t s) {
    const dim3 grid((p.T + FT - 1) / FT, p.B);
#define PROJ(NOP)                                                                                         \
    hipLaunchKernelGGL((fpa_field_proj_kernel<TX, NOP, (NOP > 48 ? 4 : 8)>), grid, dim3(64 * (NOP > 48 ? 4 : 8)), \
                       0, s, p)
    FIELD_NO_DISPATCH(PROJ);
#undef PROJ
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
#define DX(NOP) hipLaunchKernelGGL((fpa_field_dx_kernel<TX, NOP, 8>), grid, dim3(512), 0, s, p)
        FIELD_NO_DISPATCH(DX);
#undef DX
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    const dim3 gw((p.C + 1 + 63) / 64, p.S);
#define DW(NOP) hipLaunchKernelGGL((fpa_field_dw_kernel<TX, NOP>), gw, dim3(256), 0, s, p)
    FIELD_NO_DISPATCH(DW);
#undef DW
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(fpa_field_reduce_kernel, dim3((p.NO * (p.C + 1) + 255) / 256), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_field_fwd(const FieldParams &p, int dtype, hipStream_t s) {
    return dtype == 0 ? field_fwd_t<f16>(p, s) : field_fwd_t<float>(p, s);
}

hipError_t launch_field_bwd(const FieldParams &p, int dtype, hipStream_t s) {
    return dtype == 0 ? field_bwd_t<f16>(p, s) : field_bwd_t<float>(p, s);
}

}  // namespace fpa
