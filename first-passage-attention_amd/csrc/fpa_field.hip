// fpa_field.hip -- the Field prologue of the FirstPassageAttention layer, forward and backward.
//
// Reference behaviour: Field.forward (kernel.py:502-509) of yliu-fort/first-passage-attention:
//   (delta, g, h) = x W^T + b in fp32 (W: 3H x C), W_t = cumsum_t delta_t,
//   phi = W + g, psi = W + h, per (batch, head);
// and the gradient torch's autograd takes through it (kernel.py relies on autograd).
//
// The projection has only 3H outputs per position (36 for H = 12), so it is a pass over x
// (HBM-bound) with little arithmetic, done on the fp32 MFMA (the reference computes it in fp32).
// With x aligned to four features (the usual case) the 16x16x4 kernels read x, W and d(lin) as
// 16-byte vectors into MFMA operands (the projection, up to 48 outputs, through an LDS tile staged
// from contiguous row pieces), using the freedom to order the contraction so that one four-feature
// operand feeds four MFMAs; other layouts take the 32x32x2 kernels, which read one element per lane.  The projection is stored per (batch, output) along t, in rows of TL = T
// rounded up to 16, so the cumulative sum over t reads contiguous rows.  Backward: a reverse
// cumulative sum gives d(delta) (the gradient is stored in the same layout, zero past T); dx =
// d(lin) W is the same pass the other way round; dW = d(lin)^T x (and dbias) is summed in a fixed
// order (per-split partials, then one ordered reduction), so reruns are bit-identical.
#include <type_traits>

#include "fpa_common.h"
#include "fpa_params.h"

namespace fpa {

namespace {

constexpr int FT = 64;  // positions per workgroup (one per lane)

template <typename TX> __device__ __forceinline__ float to_f(TX v) { return (float)v; }
__device__ __forceinline__ int imin(int a, int b) { return a < b ? a : b; }  // per lane

// Inclusive scan of one value per thread over a 256-thread workgroup (fixed order); total gets the
// sum of all 256 values.
__device__ __forceinline__ float block_scan256(float v, float *red, float &total) {
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
    total = ((red[0] + red[1]) + red[2]) + red[3];
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
        p.lin[((int64_t)b * p.NO + o) * p.TL + t] = v + p.bias[o];
    }
}

// fp32 16x16x4 MFMA, A[m][k] x B[k][n] per wave: lane l gives A[l % 16][l / 16] and B[l / 16][l % 16];
// register r of the 16x16 accumulator holds row 4 (l / 16) + r, column l % 16.
__device__ __forceinline__ f32x4 mma16_f32(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Four consecutive features of x as one load (16 bytes in fp32, 8 in fp16), widened to fp32.
template <typename TX> __device__ __forceinline__ f32x4 load4(const TX *a);
template <> __device__ __forceinline__ f32x4 load4<float>(const float *a) { return *reinterpret_cast<const f32x4 *>(a); }
template <> __device__ __forceinline__ f32x4 load4<f16>(const f16 *a) {
    return __builtin_convertvector(*reinterpret_cast<const h4 *>(a), f32x4);
}

// lin on the 16x16x4 MFMA, x loaded straight into A operands (the path for more than 48 outputs;
// fewer take the staged kernel below): needs C, x's strides and the x and W pointers aligned to four
// features.  Grid (ceil(T / (16 MT)), B), NWF waves; wave w owns features [w CS, (w + 1) CS) for the
// workgroup's 16 MT positions (MT M tiles) and 16 NT >= NO outputs (N tiles).  Per 16-feature step,
// lane (k group j = l / 16, row r = l % 16) loads features c + 4j .. c + 4j + 3 of each of its MT
// positions and of each of its W rows, and k step s of the four contracts feature c + 4j + s: one
// 4-feature load feeds four MFMAs, x is read once, and the operands do not pass through LDS.  Loads
// run PD steps ahead in a ring of registers; nothing is done to the loaded values before their
// MFMAs (rows past T or NO read an in-bounds row, and only give sums that are never stored), so
// the waits for a step's loads fall just before its products.  A last step of 4, 8 or 12 features
// (C not a multiple of 16) zeroes the W values past the wave's features.  The NWF partial sums of
// a position meet in LDS and are added in wave order.
template <typename TX, int NT, int NWF, int PD, int MT>
__global__ void __launch_bounds__(64 * NWF) fpa_field_proj16_kernel(FieldParams p) {
    constexpr int NOP = 16 * NT, FM = 16 * MT, RP = FM + 1;
    __shared__ float red[NWF * NOP * RP];
    const int tid = thread_x(), lane = tid % 64, j = lane / 16, r16 = lane % 16;
    const int w = __builtin_amdgcn_readfirstlane(tid / 64);
    const int b = group_y(), t0 = group_x() * FM;
    const int CS = ((p.C + NWF - 1) / NWF + 15) / 16 * 16;
    const int ca = umin_i(w * CS, p.C), cb = umin_i(ca + CS, p.C);
    const TX *xb = static_cast<const TX *>(p.x) + (int64_t)b * p.sxb;
    const TX *xrow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int t = t0 + 16 * mt + r16;
        xrow[mt] = xb + (int64_t)(t < p.T ? t : p.T - 1) * p.sxt + 4 * j;
    }
    const float *wrow[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const int o = 16 * nt + r16;
        wrow[nt] = p.w + (int64_t)(o < p.NO ? o : 0) * p.C + 4 * j;
    }
    const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
    f32x4 xr[PD][MT], wr[PD][NT], acc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = z4;
    auto load = [&](f32x4 (&xv)[MT], f32x4 (&wv)[NT], int c) {  // features c + 4j .. c + 4j + 3 (< C)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) xv[mt] = load4<TX>(xrow[mt] + c);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) wv[nt] = *reinterpret_cast<const f32x4 *>(wrow[nt] + c);
        __builtin_amdgcn_sched_barrier(0);  // steps' loads stay in step order
    };
    auto step = [&](const f32x4 (&xv)[MT], const f32x4 (&wv)[NT]) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = mma16_f32(xv[mt][ks], wv[nt][ks], acc[mt][nt]);
        __builtin_amdgcn_sched_barrier(0);
    };
    const int nfull = (cb - ca) / 16;  // whole 16-feature steps
    if (nfull > 0) {
        // Loads are issued unconditionally, so the waits count them exactly; those past the last whole
        // step repeat its addresses (cache hits) and are not used.
        const int clast = ca + 16 * (nfull - 1);
#pragma unroll
        for (int u = 0; u < PD; ++u) load(xr[u], wr[u], umin_i(ca + 16 * u, clast));
        for (int s0 = 0; s0 < nfull; s0 += PD) {
#pragma unroll
            for (int u = 0; u < PD; ++u) {
                if (s0 + u < nfull) step(xr[u], wr[u]);
                load(xr[u], wr[u], umin_i(ca + 16 * (s0 + u + PD), clast));
            }
        }
    }
    if (ca + 16 * nfull < cb) {  // the last 4, 8 or 12 features of x
        const int c = ca + 16 * nfull;
        load(xr[0], wr[0], c + 4 * j < cb ? c : c - 4 * j);  // lanes past cb read features c .. c + 3
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) wr[0][nt] = c + 4 * j < cb ? wr[0][nt] : z4;
        step(xr[0], wr[0]);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[(w * NOP + 16 * nt + r16) * RP + 16 * mt + 4 * j + r] = acc[mt][nt][r];
    __syncthreads();
    for (int i = tid; i < p.NO * FM; i += 64 * NWF) {
        const int o = i / FM, r = i % FM, t = t0 + r;
        if (t >= p.T) continue;
        float v = 0.f;
#pragma unroll
        for (int k = 0; k < NWF; ++k) v += red[(k * NOP + o) * RP + r];
        p.lin[((int64_t)b * p.NO + o) * p.TL + t] = v + p.bias[o];
    }
}

constexpr int SCK = 8;  // 256-position chunks whose loads a scan issues together

// lin with the operand layout of fpa_field_proj16_kernel, x staged through LDS (up to 48 outputs):
// 8 waves, 64 positions; the workgroup loads 128-feature chunks of its 64 rows
// with 512 contiguous bytes per row (fp32; 256 in fp16) into a double-buffered LDS tile, the loads
// two chunks ahead, and wave w takes features 16w .. 16w + 15 of each chunk (A operands as 16-byte
// LDS reads, W as 16-byte loads, one chunk ahead).  One barrier per chunk; past C the tile and W
// hold zeros.  Each wave's partial sums (its slices of every chunk, in chunk order) are added in
// wave order, so reruns are bit-identical.
template <typename TX, int NT>
__global__ void __launch_bounds__(512) fpa_field_proj_staged_kernel(FieldParams p) {
    constexpr int NWF = 8, KC = 16 * NWF, XPS = KC + 4, NOP = 16 * NT, RP = FT + 1;
    constexpr int STG = 2 * FT * XPS, RED = NWF * NOP * RP;
    __shared__ __attribute__((aligned(16))) float lds[STG > RED ? STG : RED];
    const int tid = thread_x(), lane = tid % 64, j = lane / 16, r16 = lane % 16;
    const int w = __builtin_amdgcn_readfirstlane(tid / 64);
    const int b = group_y(), t0 = group_x() * FT;
    const TX *xb = static_cast<const TX *>(p.x) + (int64_t)b * p.sxb;
    const int NCH = (p.C + KC - 1) / KC;
    const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
    // Staging: thread tid moves rows lr + 16q (q < 4), features 4 lc .. 4 lc + 3 of a chunk; rows
    // past T read row T - 1 (their sums are not stored).
    const int lr = tid / 32, lc = tid % 32;
    const TX *srow[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int t = t0 + lr + 16 * q;
        srow[q] = xb + (int64_t)(t < p.T ? t : p.T - 1) * p.sxt;
    }
    f32x4 sa[4], sb[4];  // chunks ch + 1 and ch + 2 in flight, alternately in sa and sb
    auto gload = [&](int ch, f32x4 (&sv)[4]) {
        const int c = ch * KC + 4 * lc;
        const int cl = c < p.C ? c : p.C - 4;
#pragma unroll
        for (int q = 0; q < 4; ++q) sv[q] = load4<TX>(srow[q] + cl);
    };
    auto lstore = [&](int ch, int buf, const f32x4 (&sv)[4]) {
        const bool ok = ch * KC + 4 * lc < p.C;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            *reinterpret_cast<f32x4 *>(&lds[(buf * FT + lr + 16 * q) * XPS + 4 * lc]) = ok ? sv[q] : z4;
    };
    const float *wrow[NT];  // rows past NO read row 0 (their sums are not stored)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) wrow[nt] = p.w + (int64_t)(16 * nt + r16 < p.NO ? 16 * nt + r16 : 0) * p.C;
    f32x4 wv[NT], wn[NT], acc[4][NT];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = z4;
    auto wload = [&](int ch) {
        const int c = ch * KC + 16 * w + 4 * j;
        const int cl = c < p.C ? c : p.C - 4;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) wn[nt] = *reinterpret_cast<const f32x4 *>(wrow[nt] + cl);
    };
    // Chunk ch: compute from LDS buffer ch % 2, then stage chunk ch + 1 (loaded two chunks earlier,
    // in sb for even ch, in sa for odd) into the other buffer and load chunk ch + 3 in its place.
    auto chunk = [&](int ch, f32x4 (&sv)[4]) {
        const int buf = ch & 1;
        const bool wok = ch * KC + 16 * w + 4 * j < p.C;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) wv[nt] = wok ? wn[nt] : z4;
        if (ch + 1 < NCH) wload(ch + 1);
        __syncthreads();  // chunk ch is in buffer buf; buffer buf ^ 1 is no longer read
        f32x4 xa[4];
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
            xa[mt] = *reinterpret_cast<const f32x4 *>(&lds[(buf * FT + 16 * mt + r16) * XPS + 16 * w + 4 * j]);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = mma16_f32(xa[mt][ks], wv[nt][ks], acc[mt][nt]);
        if (ch + 1 < NCH) {
            lstore(ch + 1, buf ^ 1, sv);
            if (ch + 3 < NCH) gload(ch + 3, sv);
        }
    };
    gload(0, sa);
    wload(0);
    lstore(0, 0, sa);
    if (NCH > 1) gload(1, sb);
    if (NCH > 2) gload(2, sa);
    for (int ch = 0; ch < NCH; ch += 2) {
        chunk(ch, sb);
        if (ch + 1 < NCH) chunk(ch + 1, sa);
    }
    __syncthreads();  // staging done; the same LDS takes the partial sums, [w][o][position]
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int r = 0; r < 4; ++r) lds[(w * NOP + 16 * nt + r16) * RP + 16 * mt + 4 * j + r] = acc[mt][nt][r];
    __syncthreads();
    const int t = t0 + lane;
    if (t >= p.T) return;
    for (int o = w; o < p.NO; o += NWF) {
        float v = 0.f;
#pragma unroll
        for (int k = 0; k < NWF; ++k) v += lds[(k * NOP + o) * RP + lane];
        p.lin[((int64_t)b * p.NO + o) * p.TL + t] = v + p.bias[o];
    }
}

// phi = cumsum_t(delta) + g, psi = cumsum_t(delta) + h for one (b, h) per workgroup (256 threads):
// 256 consecutive positions at a time, one per thread (coalesced rows), scanned across the
// workgroup and added to the running total of the positions before them; the loads of SCK chunks
// are issued before their scans.
__global__ void __launch_bounds__(256) fpa_field_scan_kernel(FieldParams p) {
    __shared__ float red[4];
    const int bh = group_x(), b = bh / p.H, h = bh % p.H;
    const int tid = thread_x();
    const float *dl = p.lin + ((int64_t)b * p.NO + h) * p.TL;
    const float *gl = dl + (int64_t)p.H * p.TL, *hl = gl + (int64_t)p.H * p.TL;
    float *phi = p.phi + (int64_t)bh * p.T, *psi = p.psi + (int64_t)bh * p.T;
    float carry = 0.f;
    // 64-bit positions: T may come within a chunk of 2^31 (check_field bounds B * TL below 2^31).
    for (int64_t c0 = 0; c0 < p.T; c0 += 256 * SCK) {
        float d[SCK], g[SCK], e[SCK];
#pragma unroll
        for (int k = 0; k < SCK; ++k) {
            const int64_t t = c0 + 256 * k + tid;
            const bool ok = t < p.T;
            d[k] = ok ? dl[t] : 0.f;
            g[k] = ok ? gl[t] : 0.f;
            e[k] = ok ? hl[t] : 0.f;
        }
#pragma unroll
        for (int k = 0; k < SCK; ++k) {
            const int64_t t = c0 + 256 * k + tid;
            float total;
            const float run = carry + block_scan256(d[k], red, total);
            if (t < p.T) {
                phi[t] = run + g[k];
                psi[t] = run + e[k];
            }
            carry += total;
        }
    }
}

// Backward of the scan: d(delta)_t = sum_{u >= t} (dphi_u + dpsi_u), dg = dphi, dh = dpsi, written
// to lin as (B, NO, TL) rows, zero past T.  Positions are taken 256 at a time from the end (thread
// i has position c - i), so the workgroup scan runs from T down to 0; the loads of SCK chunks are
// issued before their scans.
__global__ void __launch_bounds__(256) fpa_field_bwd_scan_kernel(FieldParams p) {
    __shared__ float red[4];
    const int bh = group_x(), b = bh / p.H, h = bh % p.H;
    const int tid = thread_x();
    const float *dphi = p.dphi + (int64_t)bh * p.T, *dpsi = p.dpsi + (int64_t)bh * p.T;
    float *dd = p.lin + ((int64_t)b * p.NO + h) * p.TL;
    float *dg = dd + (int64_t)p.H * p.TL, *dh = dg + (int64_t)p.H * p.TL;
    float carry = 0.f;
    for (int64_t c0 = 0; c0 < p.T; c0 += 256 * SCK) {
        float a[SCK], c[SCK];
#pragma unroll
        for (int k = 0; k < SCK; ++k) {
            const int64_t t = p.T - 1 - c0 - 256 * k - tid;
            a[k] = t >= 0 ? dphi[t] : 0.f;
            c[k] = t >= 0 ? dpsi[t] : 0.f;
        }
#pragma unroll
        for (int k = 0; k < SCK; ++k) {
            const int64_t t = p.T - 1 - c0 - 256 * k - tid;
            float total;
            const float run = carry + block_scan256(a[k] + c[k], red, total);
            if (t >= 0) {
                dd[t] = run;
                dg[t] = a[k];
                dh[t] = c[k];
            }
            carry += total;
        }
    }
    const int64_t tz = (int64_t)p.T + tid;
    if (tz < p.TL) dd[tz] = dg[tz] = dh[tz] = 0.f;
}

// dx[b][t][c] = sum_o d(lin)[b][o][t] W[o][c] on the MFMA.  Grid (ceil(T / 64), B), NWF waves: the
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
        const int o = i / FT, r = i % FT;
        dls[r][o] = (o < p.NO && t0 + r < p.T) ? p.lin[((int64_t)b * p.NO + o) * p.TL + t0 + r] : 0.f;
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

// Four fp32 values stored as four consecutive features of dx (16 bytes in fp32, 8 in fp16).
template <typename TX> __device__ __forceinline__ void store4(TX *a, f32x4 v);
template <> __device__ __forceinline__ void store4<float>(float *a, f32x4 v) { *reinterpret_cast<f32x4 *>(a) = v; }
template <> __device__ __forceinline__ void store4<f16>(f16 *a, f32x4 v) {
    *reinterpret_cast<h4 *>(a) = __builtin_convertvector(v, h4);
}

// dx = d(lin) W on the 16x16x4 MFMA with 16-byte W loads and dx stores: needs x and dx aligned to
// four features.  Grid (ceil(T / (16 MTD)), B), 4 waves: the workgroup's 16 MTD positions' gradients
// (4 KS4 >= NO outputs, zero past NO and T) are staged in LDS once, [o][position]; wave w takes the
// 64-feature N blocks w, w + 4, ...  In an N block at c0, k step m contracts outputs 4m + j over the
// lane groups j: lane (j, r) gives A = d(lin)[4m + j][its position r] from LDS and B = W[4m + j][c0 +
// 4r .. c0 + 4r + 3] (one 16-byte load for the four N tiles; N tile nt holds feature c0 + 4r + nt),
// so each lane ends with four consecutive features of four positions and stores each position's as
// one vector.  The next N block's W is loaded during the current block's products.
// Workgroup (gx, gy) = (position tile, batch); dls is LDS of 4 KS4 rows.
template <typename TX, int KS4, int MTD>
__device__ __forceinline__ void field_dx16(const FieldParams &p, int gx, int gy, float (*dls)[16 * MTD + 1]) {
    constexpr int FM = 16 * MTD;
    const int tid = thread_x(), lane = tid % 64, j = lane / 16, r16 = lane % 16;
    const int w = __builtin_amdgcn_readfirstlane(tid / 64);
    const int b = gy, t0 = gx * FM;
    for (int i = tid; i < 4 * KS4 * FM; i += 256) {
        const int o = i / FM, r = i % FM;
        dls[o][r] = (o < p.NO && t0 + r < p.T) ? p.lin[((int64_t)b * p.NO + o) * p.TL + t0 + r] : 0.f;
    }
    TX *dxb = static_cast<TX *>(p.dx) + (int64_t)b * p.sdxb;
    const int NBK = (p.C + 63) / 64;
    const float *wrow[KS4];  // W rows 4m + j (rows past NO read row 0; their A values are zero)
#pragma unroll
    for (int m = 0; m < KS4; ++m) wrow[m] = p.w + (int64_t)(4 * m + j < p.NO ? 4 * m + j : 0) * p.C;
    auto col = [&](int nb) { const int c = nb * 64 + 4 * r16; return c < p.C ? c : p.C - 4; };
    f32x4 wv[KS4], wn[KS4];
    if (w < NBK) {
        const int cl = col(w);
#pragma unroll
        for (int m = 0; m < KS4; ++m) wn[m] = *reinterpret_cast<const f32x4 *>(wrow[m] + cl);
    }
    __syncthreads();
    for (int nb = w; nb < NBK; nb += 4) {
#pragma unroll
        for (int m = 0; m < KS4; ++m) wv[m] = wn[m];
        if (nb + 4 < NBK) {
            const int cl = col(nb + 4);
#pragma unroll
            for (int m = 0; m < KS4; ++m) wn[m] = *reinterpret_cast<const f32x4 *>(wrow[m] + cl);
        }
        const int c = nb * 64 + 4 * r16;
#pragma unroll
        for (int mt = 0; mt < MTD; ++mt) {
            const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
            f32x4 acc[4] = {z4, z4, z4, z4};
#pragma unroll
            for (int m = 0; m < KS4; ++m) {
                const float a = dls[4 * m + j][16 * mt + r16];
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) acc[nt] = mma16_f32(a, wv[m][nt], acc[nt]);
            }
            if (c < p.C) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = t0 + 16 * mt + 4 * j + r;
                    if (t < p.T) store4<TX>(dxb + (int64_t)t * p.sdxt + c, f32x4{acc[0][r], acc[1][r], acc[2][r], acc[3][r]});
                }
            }
        }
    }
}

// Partial dW and dbias over one split of the B*T positions on the MFMA: part[s][o][c] = sum_{n in
// split s} d(lin)[n][o] x[n][c] for c < C, and the same with x = 1 at c = C (the bias).  Grid
// (ceil((C + 1) / 64), S), 4 waves, each a quarter of the split's positions; per k step two
// positions (lanes 0-31: n, lanes 32-63: n + 1): A = d(lin)^T (outputs x positions), B = x
// (positions x 64 features, two N tiles), one element per lane and operand.  The four quarters meet
// in LDS in wave order.  (Any x layout; fpa_field_dw16_kernel takes four-feature-aligned x.)
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
                    av[u][mt] = (nv && o < p.NO) ? p.lin[((int64_t)bl * p.NO + o) * p.TL + tl] : 0.f;
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

// Partial dW and dbias over one split of the positions on the 16x16x4 MFMA, both operands loaded
// straight from memory: needs x aligned to four features (as the 16x16 projection).  The positions
// are taken in groups of 16 inside one batch (a batch's TL-long rows of d(lin) are zero past T, and x
// rows past T read row T - 1); split s takes groups [s GS, (s + 1) GS) of the B TL / 16 and wave w a
// quarter of them.  Grid (ceil(C / 64), S), 4 waves; M = outputs (NT tiles), N = the workgroup's 64
// features.  In a group at t0, k step j of the MFMA contracts positions t0 + 4j + s over the four
// sub-steps s, and lane (j, r) loads d(lin)[o][t0 + 4j .. t0 + 4j + 3] for each of its outputs
// o = 16 mt + r (A, one value per sub-step) and x[t0 + 4j + s][c0 + 4r .. c0 + 4r + 3] for each s
// (B: feature c0 + 4r + nt in N tile nt): every load is 16 contiguous bytes and feeds four MFMAs.
// Loads run PD groups ahead, unconditionally (as in the projection), so the waits count them
// exactly.  dbias adds up the A values on the VALU.  The four waves meet in LDS in wave order, and
// part[s][o][c] has the layout of fpa_field_dw_kernel's (the bias at c = C, from workgroup 0).
// Workgroup (gx, gy) = (feature block, split); red and bred are LDS ([4][16 NT][65] and, for dbias,
// [wave][k group][output]).
template <typename TX, int NT, int PD>
__device__ __forceinline__ void field_dw16(const FieldParams &p, int gx, int gy, float (*red)[16 * NT][65],
                                           float (*bred)[4][16 * NT]) {
    constexpr int NOP = 16 * NT;
    const int tid = thread_x(), lane = tid % 64, j = lane / 16, r16 = lane % 16;
    const int w = __builtin_amdgcn_readfirstlane(tid / 64);
    const int c0 = gx * 64, s = gy;
    const int GB = p.TL / 16, G = p.B * GB;  // groups per batch, in all
    const int per = (G + p.S - 1) / p.S, q = (per + 3) / 4;
    const int lim = umin_i(s * per + per, G);
    const int ga = umin_i(s * per + w * q, lim), gb = umin_i(ga + q, lim);
    const int cx = c0 + 4 * r16 < p.C ? c0 + 4 * r16 : p.C - 4;  // columns past C are not stored
    const TX *xcol = static_cast<const TX *>(p.x) + cx;
    int orow[NT];  // d(lin) row offsets within a batch; rows past NO read row 0 and are not stored
#pragma unroll
    for (int mt = 0; mt < NT; ++mt) orow[mt] = (16 * mt + r16 < p.NO ? 16 * mt + r16 : 0) * p.TL + 4 * j;
    const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
    f32x4 xv[PD][4], dv[PD][NT], acc[NT][4], bacc[NT];
#pragma unroll
    for (int mt = 0; mt < NT; ++mt) {
        bacc[mt] = z4;
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = z4;
    }
    auto load = [&](f32x4 (&xg)[4], f32x4 (&dg)[NT], int g) {
        const int b = g / GB, t0 = (g % GB) * 16;
        const TX *xb = xcol + (int64_t)b * p.sxb;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int t = t0 + 4 * j + e;
            xg[e] = load4<TX>(xb + (int64_t)(t < p.T ? t : p.T - 1) * p.sxt);
        }
        const float *db = p.lin + (int64_t)b * p.NO * p.TL + t0;
#pragma unroll
        for (int mt = 0; mt < NT; ++mt) dg[mt] = *reinterpret_cast<const f32x4 *>(db + orow[mt]);
        __builtin_amdgcn_sched_barrier(0);
    };
    auto step = [&](const f32x4 (&xg)[4], const f32x4 (&dg)[NT]) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int mt = 0; mt < NT; ++mt)
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = mma16_f32(dg[mt][e], xg[e][nt], acc[mt][nt]);
#pragma unroll
        for (int mt = 0; mt < NT; ++mt) bacc[mt] += dg[mt];
        __builtin_amdgcn_sched_barrier(0);
    };
    const int n = gb - ga;
    if (n > 0) {
        const int glast = gb - 1;
#pragma unroll
        for (int u = 0; u < PD; ++u) load(xv[u], dv[u], umin_i(ga + u, glast));
        for (int s0 = 0; s0 < n; s0 += PD) {
#pragma unroll
            for (int u = 0; u < PD; ++u) {
                if (s0 + u < n) step(xv[u], dv[u]);
                load(xv[u], dv[u], umin_i(ga + s0 + u + PD, glast));
            }
        }
    }
#pragma unroll
    for (int mt = 0; mt < NT; ++mt) {
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[w][16 * mt + 4 * j + r][4 * r16 + nt] = acc[mt][nt][r];
        bred[w][j][16 * mt + r16] = (bacc[mt][0] + bacc[mt][1]) + (bacc[mt][2] + bacc[mt][3]);
    }
    __syncthreads();
    for (int i = tid; i < p.NO * 64; i += 256) {
        const int o = i / 64, cc = i % 64, c = c0 + cc;
        if (c < p.C)
            p.part[((int64_t)s * p.NO + o) * (p.C + 1) + c] = (red[0][o][cc] + red[1][o][cc]) + (red[2][o][cc] + red[3][o][cc]);
    }
    if (gx == 0 && tid < p.NO) {
        float v = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) v += (bred[k][0][tid] + bred[k][1][tid]) + (bred[k][2][tid] + bred[k][3][tid]);
        p.part[((int64_t)s * p.NO + tid) * (p.C + 1) + p.C] = v;
    }
}

template <typename TX, int NT, int PD>
__global__ void __launch_bounds__(256) fpa_field_dw16_kernel(FieldParams p) {
    __shared__ float red[4][16 * NT][65];
    __shared__ float bred[4][4][16 * NT];
    field_dw16<TX, NT, PD>(p, group_x(), group_y(), red, bred);
}

// dx and the dW partials in one launch, so that the two passes share the chip (dx has one wave per
// SIMD alone): a 1-D grid of the dx workgroups first (the longer ones), then the dW workgroups, over
// one LDS area that either kind uses as its own.
template <typename TX, int KS4, int NT>
__global__ void __launch_bounds__(256) fpa_field_dxdw_kernel(FieldParams p) {
    constexpr int MTD = 4, FM = 16 * MTD;
    constexpr int DXF = 4 * KS4 * (FM + 1), DWF = 4 * 16 * NT * 65 + 4 * 4 * 16 * NT;
    __shared__ __attribute__((aligned(16))) float lds[DXF > DWF ? DXF : DWF];
    const int ntb = (p.T + FM - 1) / FM, ndx = ntb * p.B, id = group_x();
    if (id < ndx) {
        field_dx16<TX, KS4, MTD>(p, id % ntb, id / ntb, reinterpret_cast<float (*)[FM + 1]>(lds));
    } else {
        const int k = id - ndx, nbx = (p.C + 63) / 64;
        field_dw16<TX, NT, 2>(p, k % nbx, k / nbx, reinterpret_cast<float (*)[16 * NT][65]>(lds),
                              reinterpret_cast<float (*)[4][16 * NT]>(lds + 4 * 16 * NT * 65));
    }
}

// dW[o][c] (c < C) and dbias[o] (c = C) = sum_s part[s][o][c] in a fixed order: 256 threads take 64
// entries, wave w the splits s = w mod 4, and the four wave sums are added in wave order.
__global__ void __launch_bounds__(256) fpa_field_reduce_kernel(FieldParams p) {
    __shared__ float red[4][64];
    const int tid = thread_x(), lane = tid % 64, w = tid / 64;
    const int64_t i = (int64_t)group_x() * 64 + lane;
    const int64_t C1 = p.C + 1, n = p.NO * C1;
    float a = 0.f;
    if (i < n) {
        // Eight splits' loads at a time, then added in split order.
        for (int s0 = w; s0 < p.S; s0 += 32) {
            float v[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = s0 + 4 * k < p.S ? p.part[(int64_t)(s0 + 4 * k) * n + i] : 0.f;
#pragma unroll
            for (int k = 0; k < 8; ++k) a += v[k];
        }
    }
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

// x and W in four-feature units: the unit-stride loads of the 16x16 projection are aligned.
template <typename TX>
static bool four_feature_aligned(const FieldParams &p) {
    const uintptr_t ax = reinterpret_cast<uintptr_t>(p.x), aw = reinterpret_cast<uintptr_t>(p.w);
    return p.C % 4 == 0 && p.sxt % 4 == 0 && p.sxb % 4 == 0 && ax % (4 * sizeof(TX)) == 0 && aw % 16 == 0;
}

// The same for dx (the backward's 16x16 kernels read x and write dx in four-feature vectors).
template <typename TX>
static bool dx_four_feature_aligned(const FieldParams &p) {
    const uintptr_t ad = reinterpret_cast<uintptr_t>(p.dx);
    return four_feature_aligned<TX>(p) && p.sdxt % 4 == 0 && p.sdxb % 4 == 0 && ad % (4 * sizeof(TX)) == 0;
}

template <typename TX>
static hipError_t field_fwd_t(const FieldParams &p, hipStream_t s) {
    const dim3 grid((p.T + FT - 1) / FT, p.B);
    if (four_feature_aligned<TX>(p)) {
        constexpr int MT = 4, PD = 3;
        const dim3 g16((p.T + 16 * MT - 1) / (16 * MT), p.B);
        if (p.NO <= 16) hipLaunchKernelGGL((fpa_field_proj_staged_kernel<TX, 1>), grid, dim3(512), 0, s, p);
        else if (p.NO <= 32) hipLaunchKernelGGL((fpa_field_proj_staged_kernel<TX, 2>), grid, dim3(512), 0, s, p);
        else if (p.NO <= 48) hipLaunchKernelGGL((fpa_field_proj_staged_kernel<TX, 3>), grid, dim3(512), 0, s, p);
        else if (p.NO <= 64) hipLaunchKernelGGL((fpa_field_proj16_kernel<TX, 4, 4, PD, MT>), g16, dim3(256), 0, s, p);
        else hipLaunchKernelGGL((fpa_field_proj16_kernel<TX, 6, 4, PD, MT>), g16, dim3(256), 0, s, p);
    } else if (p.NO <= 32) hipLaunchKernelGGL((fpa_field_proj_kernel<TX, 1, 8>), grid, dim3(512), 0, s, p);
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
    if (p.dx != nullptr && dx_four_feature_aligned<TX>(p)) {  // dx and dW partials in one launch
        const dim3 grid(((p.T + 63) / 64) * p.B + ((p.C + 63) / 64) * p.S);
        if (p.NO <= 12) hipLaunchKernelGGL((fpa_field_dxdw_kernel<TX, 3, 1>), grid, dim3(256), 0, s, p);
        else if (p.NO <= 16) hipLaunchKernelGGL((fpa_field_dxdw_kernel<TX, 6, 1>), grid, dim3(256), 0, s, p);
        else if (p.NO <= 24) hipLaunchKernelGGL((fpa_field_dxdw_kernel<TX, 6, 2>), grid, dim3(256), 0, s, p);
        else if (p.NO <= 32) hipLaunchKernelGGL((fpa_field_dxdw_kernel<TX, 9, 2>), grid, dim3(256), 0, s, p);
        else if (p.NO <= 36) hipLaunchKernelGGL((fpa_field_dxdw_kernel<TX, 9, 3>), grid, dim3(256), 0, s, p);
        else if (p.NO <= 48) hipLaunchKernelGGL((fpa_field_dxdw_kernel<TX, 12, 3>), grid, dim3(256), 0, s, p);
        else if (p.NO <= 64) hipLaunchKernelGGL((fpa_field_dxdw_kernel<TX, 24, 4>), grid, dim3(256), 0, s, p);
        else hipLaunchKernelGGL((fpa_field_dxdw_kernel<TX, 24, 6>), grid, dim3(256), 0, s, p);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        hipLaunchKernelGGL(fpa_field_reduce_kernel, dim3((p.NO * (p.C + 1) + 63) / 64), dim3(256), 0, s, p);
        return hipGetLastError();
    }
    if (p.dx != nullptr) {
        const dim3 grid((p.T + FT - 1) / FT, p.B);
        if (p.NO <= 12) hipLaunchKernelGGL((fpa_field_dx_kernel<TX, 6, 8>), grid, dim3(512), 0, s, p);
        else if (p.NO <= 24) hipLaunchKernelGGL((fpa_field_dx_kernel<TX, 12, 8>), grid, dim3(512), 0, s, p);
        else if (p.NO <= 36) hipLaunchKernelGGL((fpa_field_dx_kernel<TX, 18, 8>), grid, dim3(512), 0, s, p);
        else if (p.NO <= 48) hipLaunchKernelGGL((fpa_field_dx_kernel<TX, 24, 8>), grid, dim3(512), 0, s, p);
        else hipLaunchKernelGGL((fpa_field_dx_kernel<TX, 48, 4>), grid, dim3(256), 0, s, p);  // registers
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    if (four_feature_aligned<TX>(p)) {
        constexpr int PD = 2;
        const dim3 gw((p.C + 63) / 64, p.S);
        if (p.NO <= 16) hipLaunchKernelGGL((fpa_field_dw16_kernel<TX, 1, PD>), gw, dim3(256), 0, s, p);
        else if (p.NO <= 32) hipLaunchKernelGGL((fpa_field_dw16_kernel<TX, 2, PD>), gw, dim3(256), 0, s, p);
        else if (p.NO <= 48) hipLaunchKernelGGL((fpa_field_dw16_kernel<TX, 3, PD>), gw, dim3(256), 0, s, p);
        else if (p.NO <= 64) hipLaunchKernelGGL((fpa_field_dw16_kernel<TX, 4, PD>), gw, dim3(256), 0, s, p);
        else hipLaunchKernelGGL((fpa_field_dw16_kernel<TX, 6, PD>), gw, dim3(256), 0, s, p);
    } else {
        const dim3 gw((p.C + 1 + 63) / 64, p.S);
        if (p.NO <= 32) hipLaunchKernelGGL((fpa_field_dw_kernel<TX, 1>), gw, dim3(256), 0, s, p);
        else if (p.NO <= 64) hipLaunchKernelGGL((fpa_field_dw_kernel<TX, 2>), gw, dim3(256), 0, s, p);
        else hipLaunchKernelGGL((fpa_field_dw_kernel<TX, 3>), gw, dim3(256), 0, s, p);
    }
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
