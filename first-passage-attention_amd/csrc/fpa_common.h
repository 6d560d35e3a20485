// fpa_common.h -- shared device code for the gfx950 First Passage Attention kernels.
//
// Conventions used by every kernel in this directory.
//
// * One head = one (b, h) pair, flattened to bh = b * H + h.  Positions are cut
//   into blocks of G = 64; TP = T rounded up to G, NB = TP / G.
// * Logits are kept in base 2: logit2 = (q.k / sqrt(D) + bias) * log2(e), so the
//   softmax uses exp2 and the saved row statistic lse2 is a base-2 log-sum-exp.
// * Matrix products run on the 32x32 MFMA of gfx950:
//     fp16: v_mfma_f32_32x32x16_f16  (one K step contracts 16 indices)
//     fp32: v_mfma_f32_32x32x2_f32   (one K step contracts 2 indices)
//   Lane l = 32 * g + c (g = l / 32, c = l % 32).  A operand: lane holds row c;
//   B operand: lane holds column c; lane group g holds its half of the K step.
//   The 32x32 accumulator: register j of lane l is C[8*(j/4) + 4*g + j%4][c].
// * A contraction index may be permuted freely as long as both operands use the
//   same permutation.  Three operand access patterns are used:
//     P1  row-major source X[row][k], k contiguous (LDS or registers):
//         fp16 step ks: X[row][16*ks + 8*g .. +8];
//         fp32 step st: X[row][g*K/2 + st].
//     P2  the accumulator of a previous product, its rows becoming the K index:
//         fp16 step ks of tile mt = ks/2: registers 8*(ks%2) .. +8, i.e. rows
//              32*mt + 16*(ks%2) + 8*(e/4) + 4*g + e%4 for element e;
//         fp32 step (mt, j): register j, i.e. row 32*mt + 8*(j/4) + 4*g + j%4.
//     P3  the partner of P2, read from a transposed source XT[n][krow]:
//         fp16: XT[n][R .. R+3] and XT[n][R+8 .. R+11], R = 32*mt + 16*(ks%2) + 4*g;
//         fp32: XT[n][32*mt + 8*(j/4) + 4*g + j%4] (4 steps per 16-byte read).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fpa {

typedef _Float16 f16;
typedef f16 h8 __attribute__((ext_vector_type(8)));
typedef f16 h4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float LOG2E = 1.4426950408889634f;
constexpr int G = 64;        // statistics block
constexpr int NTHREADS = 256;

__device__ __forceinline__ float pinf() { return __builtin_inff(); }
__device__ __forceinline__ float ninf() { return -__builtin_inff(); }
__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float frcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float flog2(float x) { return __builtin_amdgcn_logf(x); }

// log2(2^a + 2^b) with -inf handled (both -inf -> -inf).
__device__ __forceinline__ float lse2_pair(float a, float b) {
    float m = fmaxf(a, b);
    if (m == ninf()) return m;
    float d = fminf(a, b) - m;
    return m + flog2(1.0f + fexp2(d));
}

// Element (row, column) of accumulator register j for lane group g (column = lane % 32).
__device__ __forceinline__ constexpr int acc_row(int j, int g) { return 8 * (j / 4) + 4 * g + (j % 4); }

__device__ __forceinline__ float uniform_f(float x) {  // value of the first active lane
    return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
}

// A tile of soft-min terms whose exponents span less than this many binades uses one shared
// reference (products of per-key and per-query factors); wider tiles use per-element references.
constexpr float FAST_SPREAD = 96.f;

__device__ __forceinline__ f32x16 zero16() {
    f32x16 z;
#pragma unroll
    for (int i = 0; i < 16; ++i) z[i] = 0.f;
    return z;
}

// ---------------------------------------------------------------------------
// MFMA traits
// ---------------------------------------------------------------------------
template <typename T> struct MT;

template <> struct MT<f16> {
    typedef h8 op_t;
    static constexpr int KSTEP = 16;
    static constexpr int CHUNK = 8;  // elements per 16-byte global/LDS chunk
    __device__ static __forceinline__ f32x16 mma(op_t a, op_t b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

template <> struct MT<float> {
    typedef float op_t;
    static constexpr int KSTEP = 2;
    static constexpr int CHUNK = 4;
    __device__ static __forceinline__ f32x16 mma(op_t a, op_t b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    }
};

// Number of P1 operands that cover a contraction of length K (K = D here).
template <typename T, int K> struct P1Count {
    static constexpr int N = (sizeof(T) == 2) ? K / 16 : K / 2;
};
// Register array of the P1 operands of one row.
template <typename T, int K> using OpRow = typename MT<T>::op_t[P1Count<T, K>::N];

// All P1 operands of one row, read with 16-byte loads (row must be 16-byte aligned).
template <typename T, int K>
__device__ __forceinline__ void p1_load_row(OpRow<T, K> &dst, const T *row, int g) {
    if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int i = 0; i < K / 16; ++i) dst[i] = *reinterpret_cast<const h8 *>(row + 16 * i + 8 * g);
    } else {
#pragma unroll
        for (int i = 0; i < K / 8; ++i) {
            f32x4 v = *reinterpret_cast<const f32x4 *>(row + g * (K / 2) + 4 * i);
            dst[4 * i + 0] = v[0];
            dst[4 * i + 1] = v[1];
            dst[4 * i + 2] = v[2];
            dst[4 * i + 3] = v[3];
        }
    }
}

template <typename T, int K>
__device__ __forceinline__ void p1_zero(OpRow<T, K> &dst) {
#pragma unroll
    for (int i = 0; i < P1Count<T, K>::N; ++i) {
        if constexpr (sizeof(T) == 2) {
            h8 z;
#pragma unroll
            for (int e = 0; e < 8; ++e) z[e] = (f16)0.f;
            dst[i] = z;
        } else {
            dst[i] = 0.f;
        }
    }
}

// acc += A * B over a contraction of length K, both operands P1 (A from an LDS row, B in registers).
template <typename T, int K>
__device__ __forceinline__ f32x16 mma_p1_lds_reg(f32x16 acc, const T *arow, int g, const OpRow<T, K> &breg) {
    if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int i = 0; i < K / 16; ++i)
            acc = MT<T>::mma(*reinterpret_cast<const h8 *>(arow + 16 * i + 8 * g), breg[i], acc);
    } else {
#pragma unroll
        for (int i = 0; i < K / 8; ++i) {
            f32x4 a = *reinterpret_cast<const f32x4 *>(arow + g * (K / 2) + 4 * i);
            acc = MT<T>::mma(a[0], breg[4 * i + 0], acc);
            acc = MT<T>::mma(a[1], breg[4 * i + 1], acc);
            acc = MT<T>::mma(a[2], breg[4 * i + 2], acc);
            acc = MT<T>::mma(a[3], breg[4 * i + 3], acc);
        }
    }
    return acc;
}

// acc += A * B over a contraction of length K, both operands P1 rows in LDS.
template <typename T, int K>
__device__ __forceinline__ f32x16 mma_p1_lds_lds(f32x16 acc, const T *arow, const T *brow, int g) {
    if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int i = 0; i < K / 16; ++i)
            acc = MT<T>::mma(*reinterpret_cast<const h8 *>(arow + 16 * i + 8 * g),
                             *reinterpret_cast<const h8 *>(brow + 16 * i + 8 * g), acc);
    } else {
#pragma unroll
        for (int i = 0; i < K / 8; ++i) {
            const f32x4 a = *reinterpret_cast<const f32x4 *>(arow + g * (K / 2) + 4 * i);
            const f32x4 b = *reinterpret_cast<const f32x4 *>(brow + g * (K / 2) + 4 * i);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc = MT<T>::mma(a[e], b[e], acc);
        }
    }
    return acc;
}

// ---------------------------------------------------------------------------
// P3 operands read from a natural-layout LDS tile X[krow][n] (pitch in elements).
//
// fp16: ds_read_b64_tr_b16.  Within each group of 16 lanes, input lane j supplies the
// four 16-bit elements a_j[0..3] at its address and output lane i receives
// b_i[k] = a_{4k + i/4}[i % 4].  Pointing input lane j at X[R + j/4][n0 + 4*(j%4)]
// therefore hands output lane i the column n0 + i of rows R..R+3.
// ---------------------------------------------------------------------------
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

__device__ __forceinline__ h4 ds_read_tr16(const f16 *p) {
    const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(p));
    return __builtin_bit_cast(h4, v);
}

// fp16 P3 operand of contraction rows rbase + 4g + {0..3, 8..11} at column ncol0 + c.
__device__ __forceinline__ h8 p3_tr(const f16 *X, int pitch, int rbase, int ncol0, int lane) {
    const int j = lane & 15, q = lane >> 4;
    const int row = rbase + 4 * (q >> 1) + (j >> 2);
    const int col = ncol0 + 16 * (q & 1) + 4 * (j & 3);
    const f16 *p0 = X + row * pitch + col;
    const h4 lo = ds_read_tr16(p0);
    const h4 hi = ds_read_tr16(p0 + 8 * pitch);
    return h8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// acc += A * B where one operand comes from accumulator tiles c[0..NT) (P2, their rows being
// the contraction index) and the other from the natural-layout LDS tile X[krow][n] at
// column n = ncol0 + lane % 32 (P3).  A_IS_P3: the P3 value is the A operand.
template <typename T, int NT, bool A_IS_P3>
__device__ __forceinline__ f32x16 mma_p2_p3(f32x16 acc, const f32x16 (&c)[NT], const T *X, int pitch, int ncol0,
                                            int lane) {
    const int g = lane >> 5;
    if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int mt = 0; mt < NT; ++mt) {
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                h8 p2;
#pragma unroll
                for (int e = 0; e < 8; ++e) p2[e] = (f16)c[mt][8 * hf + e];
                const h8 p3 = p3_tr(X, pitch, 32 * mt + 16 * hf, ncol0, lane);
                acc = A_IS_P3 ? MT<T>::mma(p3, p2, acc) : MT<T>::mma(p2, p3, acc);
            }
        }
    } else {
        const int n = ncol0 + (lane & 31);
#pragma unroll
        for (int mt = 0; mt < NT; ++mt) {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const float p3 = X[(32 * mt + acc_row(j, g)) * pitch + n];
                acc = A_IS_P3 ? MT<T>::mma(p3, c[mt][j], acc) : MT<T>::mma(c[mt][j], p3, acc);
            }
        }
    }
    return acc;
}

// ---------------------------------------------------------------------------
// In-block range minimum X = min phi(s, t] for the accumulator registers of one 32-row
// tile of a diagonal 64-block (phi = the block's 64 values, +inf past T).  Branch-free:
// the running minimum is kept for every step and each register selects its step by
// lane group.  Entries whose range is empty hold garbage and must be masked by the caller.
// ---------------------------------------------------------------------------

// Lane = query tr (0..63 in the block); registers = keys 32*mt + acc_row(j, g).  Descending
// scan; `r` carries min phi[32*mt + 33 .. tr] in and min phi[32*mt + 1 .. tr] out.  `phi` is
// the block's 64 values in LDS (16-byte aligned): every read is unconditional (the same
// address in all lanes) and positions past tr are masked by a select, so the scan has no
// branches.
__device__ __forceinline__ void diag_x_keys(float (&X)[16], float &r, const float *phi, int mt, int tr, int g) {
    float pv[33];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const f32x4 v = *reinterpret_cast<const f32x4 *>(phi + 32 * mt + 4 * i);
        pv[4 * i] = v[0]; pv[4 * i + 1] = v[1]; pv[4 * i + 2] = v[2]; pv[4 * i + 3] = v[3];
    }
    pv[32] = (mt == 0) ? phi[32] : pinf();
    float rr[33];
#pragma unroll
    for (int k = 32; k >= 1; --k) {
        const int u = 32 * mt + k;
        r = fminf(r, (u <= tr) ? pv[k] : pinf());
        rr[k] = r;  // min phi[u .. tr]: the value for key u - 1
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int k0 = 8 * (j / 4) + (j % 4);
        X[j] = g ? rr[k0 + 5] : rr[k0 + 1];
    }
}

// Lane = key sr (0..63 in the block); registers = queries 32*mt + acc_row(j, g).  Ascending
// scan; `r` carries min phi[sr+1 .. 32*mt - 1] in and min phi[sr+1 .. 32*mt + 31] out.
// Branch-free like diag_x_keys.
__device__ __forceinline__ void diag_x_queries(float (&X)[16], float &r, const float *phi, int mt, int sr, int g) {
    float pv[32];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const f32x4 v = *reinterpret_cast<const f32x4 *>(phi + 32 * mt + 4 * i);
        pv[4 * i] = v[0]; pv[4 * i + 1] = v[1]; pv[4 * i + 2] = v[2]; pv[4 * i + 3] = v[3];
    }
    float rr[32];
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        const int u = 32 * mt + k;
        r = fminf(r, (u > sr) ? pv[k] : pinf());
        rr[k] = r;  // min phi[sr+1 .. u]: the value for query u
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int k0 = 8 * (j / 4) + (j % 4);
        X[j] = g ? rr[k0 + 4] : rr[k0];
    }
}

// x[l] + x[l ^ 32] and max(x[l], x[l ^ 32]) with the gfx950 half-wave swap (no LDS round trip).
__device__ __forceinline__ float sum_halves(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_halves(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// ---------------------------------------------------------------------------
// Swizzled LDS tiles filled by direct global -> LDS loads.
//
// A tile of NR rows x D elements is stored unpadded (D * sizeof(T) bytes per row) in
// 16-byte chunks; logical chunk lc of row r sits at physical chunk lc ^ (r & SW), which
// spreads a column of chunks over the LDS banks.  global_load_lds_dwordx4 writes the 16
// bytes of lane l of a wave to (LDS base + 16 * l): each wave instruction fills 64
// consecutive slots, and each lane picks the global row/chunk that belongs in its slot.
// Rows at or past T are loaded from row T - 1 (finite values that callers mask).
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void gbl_void_t;

template <typename T, int D> struct Sw {
    static constexpr int CE = 16 / sizeof(T);           // elements per chunk
    static constexpr int CPR = D / CE;                   // chunks per row
    static constexpr int SW = (CPR < 8 ? CPR : 8) - 1;   // swizzle mask
    static constexpr int ROWB = D * sizeof(T);           // bytes per row
    // byte offset of element e (a multiple of 4 elements for fp16) of row r
    __device__ static __forceinline__ int off(int r, int e) {
        return r * ROWB + (((e / CE) ^ (r & SW)) << 4) + (e % CE) * (int)sizeof(T);
    }
    template <int NR> static constexpr int bytes() { return NR * ROWB; }
};

__device__ __forceinline__ void gl_lds16(const void *src, void *lds_dst) {
    __builtin_amdgcn_global_load_lds((gbl_void_t *)(src), (lds_void_t *)(lds_dst), 16, 0, 0);
}

// Issue the loads of rows [row0, row0 + NR) of a (B, H, T, D)-strided tensor into the swizzled
// tile at `tile` (all waves of the workgroup take part; completes at the next vmcnt(0) wait).
template <typename T, int D, int NR>
__device__ __forceinline__ void tile_issue(char *tile, const T *base, int64_t st, int row0, int T_, int wave, int lane) {
    using S = Sw<T, D>;
    constexpr int NI = NR * S::CPR / 64;  // wave instructions per tile
    static_assert(NR * S::CPR % 64 == 0, "tile must fill whole wave instructions");
    for (int i = wave; i < NI; i += NTHREADS / 64) {
        const int k = 64 * i + lane;
        const int r = k / S::CPR, pc = k % S::CPR, lc = pc ^ (r & S::SW);
        const int row = min(row0 + r, T_ - 1);
        gl_lds16(base + (int64_t)row * st + lc * S::CE, tile + 1024 * i);
    }
}

// Load n consecutive floats (n <= 256, multiple of 4) from global into LDS with one wave.
__device__ __forceinline__ void vec_issue(float *lds, const float *src, int n, int lane) {
    if (4 * lane < n) gl_lds16(src + 4 * lane, lds);
}

__device__ __forceinline__ void wait_loads() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// P1 operands from a swizzled tile row.
template <typename T, int K>
__device__ __forceinline__ f32x16 mma_p1_sw_reg(f32x16 acc, const char *tile, int row, int g, const OpRow<T, K> &breg) {
    using S = Sw<T, K>;
    if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int i = 0; i < K / 16; ++i)
            acc = MT<T>::mma(*reinterpret_cast<const h8 *>(tile + S::off(row, 16 * i + 8 * g)), breg[i], acc);
    } else {
#pragma unroll
        for (int i = 0; i < K / 8; ++i) {
            const f32x4 a = *reinterpret_cast<const f32x4 *>(tile + S::off(row, g * (K / 2) + 4 * i));
#pragma unroll
            for (int e = 0; e < 4; ++e) acc = MT<T>::mma(a[e], breg[4 * i + e], acc);
        }
    }
    return acc;
}

// acc += A * B with the P3 operand from a swizzled tile (rows = contraction, column n = ncol0 + c)
// and the P2 operand from the accumulator tile c0 (rows 32*mt0 .. of the tile are its rows).
template <typename T, int D, bool A_IS_P3>
__device__ __forceinline__ f32x16 mma_p2_p3_sw(f32x16 acc, const f32x16 &c0, const char *tile, int row0, int ncol0,
                                               int lane) {
    using S = Sw<T, D>;
    const int g = lane >> 5;
    if constexpr (sizeof(T) == 2) {
        const int j = lane & 15, q = lane >> 4;
        const int col = ncol0 + 16 * (q & 1) + 4 * (j & 3);
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            h8 p2;
#pragma unroll
            for (int e = 0; e < 8; ++e) p2[e] = (f16)c0[8 * hf + e];
            const int row = row0 + 16 * hf + 4 * (q >> 1) + (j >> 2);
            const h4 lo = ds_read_tr16(reinterpret_cast<const f16 *>(tile + S::off(row, col)));
            const h4 hi = ds_read_tr16(reinterpret_cast<const f16 *>(tile + S::off(row + 8, col)));
            const h8 p3 = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            acc = A_IS_P3 ? MT<T>::mma(p3, p2, acc) : MT<T>::mma(p2, p3, acc);
        }
    } else {
        const int n = ncol0 + (lane & 31);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const float p3 = *reinterpret_cast<const float *>(tile + S::off(row0 + acc_row(j, g), n));
            acc = A_IS_P3 ? MT<T>::mma(p3, c0[j], acc) : MT<T>::mma(c0[j], p3, acc);
        }
    }
    return acc;
}

// ---------------------------------------------------------------------------
// Register prefetch of an NR x D tile of a (B, H, T, D)-strided tensor (rows row0 + r,
// zero past T), stored afterwards into a natural-layout LDS tile of the given pitch.
// ---------------------------------------------------------------------------
template <typename T, int D, int NR> struct TileRegs {
    static constexpr int CE = MT<T>::CHUNK;
    static constexpr int CPR = D / CE;
    static constexpr int NCH = NR * CPR;
    static constexpr int PER = (NCH + NTHREADS - 1) / NTHREADS;
    f32x4 r[PER];
    __device__ __forceinline__ void load(const T *base, int64_t st, int row0, int T_) {
        if (row0 + NR <= T_ && NCH % NTHREADS == 0) {  // full tile: no per-row guard
#pragma unroll
            for (int i = 0; i < PER; ++i) {
                const int idx = threadIdx.x + i * NTHREADS;
                const int row = idx / CPR, cc = idx % CPR;
                r[i] = *reinterpret_cast<const f32x4 *>(base + (int64_t)(row0 + row) * st + cc * CE);
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = threadIdx.x + i * NTHREADS;
            const int row = idx / CPR, cc = idx % CPR;
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (idx < NCH && row0 + row < T_)
                v = *reinterpret_cast<const f32x4 *>(base + (int64_t)(row0 + row) * st + cc * CE);
            r[i] = v;
        }
    }
    __device__ __forceinline__ void store(T *dst, int pitch) const {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
            const int idx = threadIdx.x + i * NTHREADS;
            const int row = idx / CPR, cc = idx % CPR;
            if (idx < NCH) *reinterpret_cast<f32x4 *>(dst + row * pitch + cc * CE) = r[i];
        }
    }
};

// Register P1 operands of one global row (zeros when the row is past T).
template <typename T, int D>
__device__ __forceinline__ void load_row_p1(OpRow<T, D> &dst, const T *rowp, bool valid, int g) {
    if (valid)
        p1_load_row<T, D>(dst, rowp, g);
    else
        p1_zero<T, D>(dst);
}

// Work item of this workgroup in a grid of (ntiles, BH): rank 0 is the heaviest tile.
// Workgroups are dispatched in linear order, round-robin over the 8 XCDs of the chip; when
// BH is a multiple of 8 every head is pinned to one XCD (its K/V stay in that XCD's L2)
// and each XCD takes its heads' tiles heaviest first.
__device__ __forceinline__ void xcd_work_item(int &rank, int &bh, int BH) {
    const int L = blockIdx.x + gridDim.x * blockIdx.y;
    if ((BH & 7) == 0) {
        const int xcd = L & 7, k = L >> 3, hpx = BH >> 3;
        rank = k / hpx;
        bh = (k % hpx) * 8 + xcd;
    } else {
        rank = blockIdx.x;
        bh = blockIdx.y;
    }
}

// Sum over the 64 lanes of a wave, fixed order (butterfly).
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}


// State planes (float offsets), each plane is BH * TP floats except the two block planes.
struct StateLayout {
    int64_t BH, TP, NB;
    __host__ __device__ int64_t plane(int k) const { return (int64_t)k * BH * TP; }  // 0..7
    __host__ __device__ int64_t bplane(int k) const { return 8 * BH * TP + (int64_t)k * BH * NB; }  // 0..1
    __host__ __device__ int64_t total() const { return 8 * BH * TP + 2 * BH * NB; }
};
// PL_CA = beta*log2e*min(SUF - psi, 0) and PL_CP = beta*log2e*psi: the forward's per-key bias terms.
enum { PL_PHI = 0, PL_PSI = 1, PL_PRE = 2, PL_PREL = 3, PL_SUF = 4, PL_SUFL = 5, PL_CA = 6, PL_CP = 7 };
enum { BP_MIN = 0, BP_LSE = 1 };

}  // namespace fpa
