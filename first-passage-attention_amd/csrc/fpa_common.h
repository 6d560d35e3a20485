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
typedef f16 h2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr float LOG2E = 1.4426950408889634f;
constexpr int G = 64;        // statistics block
constexpr int NTHREADS = 256;
// Waves per workgroup of the three main kernels: each wave owns 32 queries (forward, query side)
// or 32 keys (key side), so a workgroup covers 32 * FPA_NW rows and its LDS tiles are shared by
// FPA_NW waves.
#ifndef FPA_NW
#define FPA_NW 4
#endif

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

// Minimum of two wave-uniform ints, kept in SGPRs (loop bounds stay scalar).
__device__ __forceinline__ int umin_i(int a, int b) { return __builtin_amdgcn_readfirstlane(a < b ? a : b); }

__device__ __forceinline__ float uniform_f(float x) {  // value of the first active lane
    return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
}

// A tile of soft-min terms whose exponents span less than this many binades uses one shared
// reference (products of per-key and per-query factors); wider tiles use per-element references.
constexpr float FAST_SPREAD = 96.f;
constexpr float PROD_SPREAD = 100.f;  // max PREL spread of a query block for the product form of Z

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
// branches.  ALL_BEFORE: every key of the half is before every query of the wave (tr >= 32 * mt +
// 32), no mask.  The values are read four at a time as the scan reaches them and each register
// takes its value when the scan passes its key (the key of register j is 32*mt + k - 1 with
// k = 8*(j/4) + 4*g + j%4 + 1: lane group 1 takes it at step k, lane group 0 four steps later), so
// few registers are live at once.
template <bool ALL_BEFORE = false>
__device__ __forceinline__ void diag_x_keys(float (&X)[16], float &r, const float *phi, int mt, int tr, int g) {
    const bool g1 = g != 0;
    const float top = (mt == 0) ? phi[32] : pinf();
    // steps k = 32 .. 1 visit u = 32*mt + k; the value of step 32 is `top`
    {
        const int u = 32 * mt + 32;
        r = fminf(r, (ALL_BEFORE || u <= tr) ? top : pinf());
    }
#pragma unroll
    for (int i = 7; i >= 0; --i) {
        const f32x4 v = *reinterpret_cast<const f32x4 *>(phi + 32 * mt + 4 * i);
#pragma unroll
        for (int e = 3; e >= 0; --e) {
            const int k = 4 * i + e;  // steps 31 .. 0 (step k + 1 was the previous one)
            // after step k + 1 the running minimum is min phi[32*mt + k + 1 .. tr]: the value of the
            // key 32*mt + k, i.e. of the register with 8*(j/4) + 4*g + j%4 = k
            const int jj = 4 * (k / 8) + (k % 4);
            if ((k % 8) >= 4)
                X[jj] = r;  // lane group 1 (k = 8*(j/4) + 4 + j%4); group 0 overwrites it below
            else
                X[jj] = g1 ? X[jj] : r;  // lane group 0 (k = 8*(j/4) + j%4)
            if (k >= 1) {
                const int u = 32 * mt + k;
                r = fminf(r, (ALL_BEFORE || u <= tr) ? v[e] : pinf());
            }
        }
    }
}

// Lane = key sr (0..63 in the block); registers = queries 32*mt + acc_row(j, g).  Ascending
// scan; `r` carries min phi[sr+1 .. 32*mt - 1] in and min phi[sr+1 .. 32*mt + 31] out.
// Branch-free like diag_x_keys, with the values read four at a time as the scan reaches them.
// ALL_AFTER: every query of the half is after every key of the wave (sr < 32 * mt), no mask.
template <bool ALL_AFTER = false>
__device__ __forceinline__ void diag_x_queries(float (&X)[16], float &r, const float *phi, int mt, int sr, int g) {
    const bool g1 = g != 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const f32x4 v = *reinterpret_cast<const f32x4 *>(phi + 32 * mt + 4 * i);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int k = 4 * i + e;
            const int u = 32 * mt + k;
            r = fminf(r, (ALL_AFTER || u > sr) ? v[e] : pinf());  // min phi[sr+1 .. u]: the value for query u
            const int jj = 4 * (k / 8) + (k % 4);
            if ((k % 8) < 4)
                X[jj] = r;  // lane group 0 (query 8*(j/4) + j%4)
            else
                X[jj] = g1 ? r : X[jj];  // lane group 1 (query 8*(j/4) + 4 + j%4)
        }
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
// LDS tiles filled by direct global -> LDS loads.
//
// A tile holds NR rows of DT elements (DT = D rounded up to 32) at a pitch of DT + one
// 16-byte chunk: row r starts at byte r * ROWB, so every LDS read of a lane is a per-lane
// base plus an immediate offset, and a 16-lane group reading one chunk column touches 16
// distinct bank groups (ROWB / 16 is odd).  An LDS-direct buffer load writes the 16 bytes of
// lane l of a wave to (LDS base + 16 * l): each wave instruction fills 64 consecutive
// chunk slots of the tile, and each lane fetches the global chunk that belongs in its
// slot.  Pad slots and the chunks of columns D..DT-1 fetch a real chunk of the same row
// (finite values whose products are discarded), and rows at or past T fetch row T - 1
// (finite values that the callers mask).
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void_t;

template <typename T, int DT> struct Pad {
    static constexpr int CE = 16 / sizeof(T);  // elements per chunk
    static constexpr int CPR = DT / CE;        // chunks of a row
    static constexpr int CPRP = CPR + 1;       // with the pad chunk
    static constexpr int PITCH = DT + CE;      // elements
    static constexpr int ROWB = PITCH * sizeof(T);
    template <int NR> static constexpr int bytes() { return NR * ROWB; }
};

// LDS stages of a pair of padded tiles streamed through a block loop: two (the next block's loads
// are issued before this block's work) when two pairs and `extra` bytes fit in the 160 KB of a
// CU, else one (the loads of the next block follow this block's work).
template <int TB> constexpr int tile_stages(int extra) { return (4 * TB + extra <= 160 * 1024) ? 2 : 1; }

// Raw buffer resource (four SGPRs) over bytes [base, base + 2^31) of a wave-uniform pointer:
// base address (48 bits, stride 0), number of records, and the format word.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x4 buf_rsrc(const void *base) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
    return u32x4{lo, hi & 0xffffu, 0x7fffffffu, 0x00020000u};
}

// 16 bytes per lane from the buffer at byte offset voff straight into LDS at lds_dst + 16 * lane
// (lds_dst a wave-uniform LDS byte address; the kernels take lds_addr of each staging array once
// and add constant offsets, since every conversion of a generic pointer to an LDS address costs a
// null check on the scalar unit).  Counted by vmcnt like a global load.  Issued as inline assembly so that
// the compiler does not track the LDS write: tracked, it makes every later LDS read it cannot
// prove disjoint (the transposed reads among them) wait for all loads in flight, the next tile's
// included.  The callers order these writes themselves: wait_loads() and a barrier before any
// read of the tile.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void_t *)p);
}
__device__ __forceinline__ void buf_lds16(u32x4 r, uint32_t voff, uint32_t lds_dst) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds_dst), "v"(voff), "s"(r)
                 : "m0");
}

// 4 bytes per lane (lds_dst + 4 * lane).
__device__ __forceinline__ void buf_lds4(u32x4 r, uint32_t voff, uint32_t lds_dst) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
                 :
                 : "s"(lds_dst), "v"(voff), "s"(r)
                 : "m0");
}

// Wave-uniform element of memory that the running kernel does not write, read through the scalar
// cache (counted by lgkmcnt, so it never waits on the vector loads in flight).
template <typename X> __device__ __forceinline__ X ld_uniform(const X *ptr, int64_t i) {
    return ((const __attribute__((address_space(4))) X *)ptr)[i];
}

__device__ __forceinline__ void wait_loads() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Loads NR-row tiles of one (B, H, T, D)-strided tensor (d stride 1, rows 16-byte aligned,
// 64 * row stride < 2^31 bytes) into padded LDS tiles.  The NI wave instructions of a tile
// are shared out over the NW waves of the workgroup (when NW does not divide NI, the waves past
// the last instruction issue it again: identical writes instead of a wave-dependent branch); each
// wave keeps the byte offsets of its lanes' source chunks relative to the tile's first row, so a
// full tile costs no VALU work.
template <typename T, int D, int DT, int NR, int NW> struct TileLoader {
    using P = Pad<T, DT>;
    static constexpr int CPRD = D / P::CE;                // chunks of data in a row
    static constexpr int NI = NR * P::CPRP / 64;          // wave instructions per tile
    static constexpr int PER = (NI + NW - 1) / NW;        // per wave
    static_assert(NR * P::CPRP % 64 == 0, "a tile fills whole wave instructions");
    uint32_t off[PER];
    __device__ static __forceinline__ void slot(int i, int lane, int &r, int &lc) {
        const int k = 64 * i + lane;
        r = k / P::CPRP;
        const int pc = k % P::CPRP;
        lc = (pc < CPRD) ? pc : pc % CPRD;
    }
    __device__ __forceinline__ void init(int64_t st, int wave, int lane) {
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            int r, lc;
            slot(min(wave + NW * j, NI - 1), lane, r, lc);
            off[j] = (uint32_t)((r * st + lc * P::CE) * (int64_t)sizeof(T));
        }
    }
    // issue() for a tile whose rows are all below T: no per-lane clamping, so a loop that only loads
    // such tiles keeps no clamped offsets live.
    __device__ __forceinline__ void issue_full(uint32_t tile, const T *base, int64_t st, int row0, int wave) const {
        const u32x4 rs = buf_rsrc(base + (int64_t)row0 * st);
#pragma unroll
        for (int j = 0; j < PER; ++j) buf_lds16(rs, off[j], tile + 1024 * min(wave + NW * j, NI - 1));
    }
    // Rows row0 .. row0 + NR - 1 (wave-uniform row0 < T_) of the tensor whose row 0 is `base` into
    // `tile`, through a buffer resource based at row row0 (the offsets stay 32-bit).
    __device__ __forceinline__ void issue(uint32_t tile, const T *base, int64_t st, int row0, int T_, int wave,
                                          int lane) const {
        const u32x4 rs = buf_rsrc(base + (int64_t)row0 * st);
        if (row0 + NR <= T_) {
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                const int i = min(wave + NW * j, NI - 1);  // waves past the last instruction repeat it
                buf_lds16(rs, off[j], tile + 1024 * i);
            }
        } else {
            const int rmax = T_ - 1 - row0;  // rows past T read row T - 1
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                const int i = min(wave + NW * j, NI - 1);
                int r, lc;
                slot(i, lane, r, lc);
                buf_lds16(rs, (uint32_t)((min(r, rmax) * st + lc * P::CE) * (int64_t)sizeof(T)), tile + 1024 * i);
            }
        }
    }
};

// acc += A * B over a contraction of length K: A = P1 operands of row `row` of a padded tile
// of width DT, B = P1 operands in registers.
template <typename T, int K, int DT>
__device__ __forceinline__ f32x16 mma_p1_pad_reg(f32x16 acc, const char *tile, int row, int g, const OpRow<T, K> &breg) {
    return mma_p1_lds_reg<T, K>(acc, reinterpret_cast<const T *>(tile) + row * Pad<T, DT>::PITCH, g, breg);
}

// Two independent mma_p1_pad_reg chains with their steps alternated, so that each MFMA's
// accumulator dependency is covered by the other chain's MFMA instead of a stall.
template <typename T, int K, int DT>
__device__ __forceinline__ void mma_p1_pad_reg2(f32x16 &accA, const char *tileA, int rowA, const OpRow<T, K> &bA,
                                                f32x16 &accB, const char *tileB, int rowB, const OpRow<T, K> &bB,
                                                int g) {
    const T *ra = reinterpret_cast<const T *>(tileA) + rowA * Pad<T, DT>::PITCH;
    const T *rb = reinterpret_cast<const T *>(tileB) + rowB * Pad<T, DT>::PITCH;
    if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int i = 0; i < K / 16; ++i) {
            accA = MT<T>::mma(*reinterpret_cast<const h8 *>(ra + 16 * i + 8 * g), bA[i], accA);
            accB = MT<T>::mma(*reinterpret_cast<const h8 *>(rb + 16 * i + 8 * g), bB[i], accB);
        }
    } else {
#pragma unroll
        for (int i = 0; i < K / 8; ++i) {
            const f32x4 a = *reinterpret_cast<const f32x4 *>(ra + g * (K / 2) + 4 * i);
            const f32x4 b = *reinterpret_cast<const f32x4 *>(rb + g * (K / 2) + 4 * i);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                accA = MT<T>::mma(a[e], bA[4 * i + e], accA);
                accB = MT<T>::mma(b[e], bB[4 * i + e], accB);
            }
        }
    }
}

// fp16 form of mma_p2_p3_pad with the P2 operand already converted: p2[hf] holds registers
// 8 * hf .. 8 * hf + 7 of the accumulator tile.
template <int DT, bool A_IS_P3>
__device__ __forceinline__ f32x16 mma_p2h_p3_pad(f32x16 acc, const h8 (&p2)[2], const char *tile, int row0, int ncol0,
                                                 int lane) {
    constexpr int PITCH = Pad<f16, DT>::PITCH;
    const f16 *X = reinterpret_cast<const f16 *>(tile) + row0 * PITCH;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
        const h8 p3 = p3_tr(X, PITCH, 16 * hf, ncol0, lane);
        acc = A_IS_P3 ? MT<f16>::mma(p3, p2[hf], acc) : MT<f16>::mma(p2[hf], p3, acc);
    }
    return acc;
}

// acc += A * B with the P3 operand from a padded tile (contraction over its rows row0 .. row0 + 31,
// column n = ncol0 + lane % 32) and the P2 operand from the accumulator tile c0 (its rows are the
// contraction index).  A_IS_P3: the P3 value is A.
template <typename T, int DT, bool A_IS_P3>
__device__ __forceinline__ f32x16 mma_p2_p3_pad(f32x16 acc, const f32x16 &c0, const char *tile, int row0, int ncol0,
                                                int lane) {
    const f32x16 c[1] = {c0};
    return mma_p2_p3<T, 1, A_IS_P3>(acc, c, reinterpret_cast<const T *>(tile) + row0 * Pad<T, DT>::PITCH,
                                    Pad<T, DT>::PITCH, ncol0, lane);
}

// Register P1 operands of one global row (zeros when the row is past T).
template <typename T, int D>
__device__ __forceinline__ void load_row_p1(OpRow<T, D> &dst, const T *rowp, bool valid, int g) {
    if (valid)
        p1_load_row<T, D>(dst, rowp, g);
    else
        p1_zero<T, D>(dst);
}

// Work-item and workgroup ids read from the hardware registers.  (Built with IEEE mode off,
// the kernels cannot inline the device library's accessors behind threadIdx / blockIdx /
// gridDim, which then become function calls.)
__device__ __forceinline__ int thread_x() { return __builtin_amdgcn_workitem_id_x(); }
__device__ __forceinline__ int group_x() { return __builtin_amdgcn_workgroup_id_x(); }
__device__ __forceinline__ int group_y() { return __builtin_amdgcn_workgroup_id_y(); }
__device__ __forceinline__ int group_z() { return __builtin_amdgcn_workgroup_id_z(); }

// Per-head grids are (n, H, B), as many workgroups per head as the kernel needs times H times
// B (each at most 65535, the grid's y and z limits); the flattened head index is b * H + h.
__device__ __forceinline__ int group_bh(int H) { return group_z() * H + group_y(); }
inline dim3 head_grid(int n, int H, int BH) { return dim3(n, H, BH / H); }

// Work item of this workgroup in a per-head grid of ntiles workgroups per head: rank 0 is the
// heaviest tile.  Workgroups are dispatched in linear order (x fastest, then the head), round-
// robin over the 8 XCDs of the chip; when BH is a multiple of 8 every head is pinned to one XCD
// (its K/V stay in that XCD's L2) and each XCD takes its heads' tiles heaviest first.  Otherwise
// the dispatch order is rank-major over all heads (every head's heaviest tile first), so that the
// longest tiles never wait for a free slot behind the short tiles of earlier heads.  The entry
// points keep ntiles * BH below 2^31.
//
// slots > 1 (the workgroups one CU holds at once): the first round of dispatch places workgroup
// k of an XCD's ncu CUs (k counting that XCD's workgroups) on CU k % ncu, so a CU
// starts with the workgroups k, k + ncu, k + 2 ncu, ...; when every workgroup is resident at once
// (the launch is one round), the CU with the heaviest first-slot tile would otherwise also get the
// heaviest tiles of the later slots and set the launch time.  Odd slots of the first round take
// their tiles in reverse order instead (heavy + light + medium on every CU).
__device__ __forceinline__ int snake_index(int k, int n, int ncu, int slots) {
    const int s = k / ncu, c = k - s * ncu;
    return ((s & 1) && s < slots && (s + 1) * ncu <= n) ? s * ncu + (ncu - 1 - c) : k;
}
constexpr int XCD_CUS = 32;  // CUs per XCD of MI355X (8 XCDs, 256 CUs)

__device__ __forceinline__ void xcd_work_item(int &rank, int &bh, int BH, int H, int ntiles, int slots = 1) {
    int L = group_x() + ntiles * group_bh(H);
    if ((BH & 7) == 0) {
        const int xcd = L & 7, hpx = BH >> 3;
        const int k = slots > 1 ? snake_index(L >> 3, ntiles * hpx, XCD_CUS, slots) : (L >> 3);
        rank = k / hpx;
        bh = (k % hpx) * 8 + xcd;
    } else {
        // Reversed within each XCD (L & 7 kept), so that an item stays on the XCD of the plain
        // order and each XCD's L2 keeps seeing the same heads.
        if (slots > 1) L = (snake_index(L >> 3, (ntiles * BH) >> 3, XCD_CUS, slots) << 3) | (L & 7);
        rank = L / BH;
        bh = L % BH;
    }
    rank = __builtin_amdgcn_readfirstlane(rank);  // uniform: loop bounds and addresses stay scalar
    bh = __builtin_amdgcn_readfirstlane(bh);
}

// Lane exchange within rows of 16 lanes by a DPP pattern (every source lane is inside the row).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
// Reduction over the 64 lanes of a wave in a fixed order, result in every lane: lanes ^1 and ^2
// (quad_perm), the quads and halves of each 16-lane row (row_half_mirror, row_mirror), then rows
// 0+1 / 2+3 (permlane16 swap) and the two 32-lane halves (permlane32 swap).  VALU only, no LDS.
template <typename Op>
__device__ __forceinline__ float wave_reduce(float x, Op op) {
    x = op(x, dpp_f<0xB1>(x));   // quad_perm [1,0,3,2]
    x = op(x, dpp_f<0x4E>(x));   // quad_perm [2,3,0,1]
    x = op(x, dpp_f<0x141>(x));  // row_half_mirror
    x = op(x, dpp_f<0x140>(x));  // row_mirror
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = op(__uint_as_float(r[0]), __uint_as_float(r[1]));
    const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return op(__uint_as_float(q[0]), __uint_as_float(q[1]));
}
__device__ __forceinline__ float wave_sum(float x) {
    return wave_reduce(x, [](float a, float b) { return a + b; });
}
__device__ __forceinline__ float wave_min(float x) {
    return wave_reduce(x, [](float a, float b) { return fminf(a, b); });
}
__device__ __forceinline__ float wave_max(float x) {
    return wave_reduce(x, [](float a, float b) { return fmaxf(a, b); });
}


// State planes (float offsets): NPL per-position planes of TP floats per head, then two block planes.
constexpr int NPL = 10;  // per-position planes
struct StateLayout {
    int64_t BH, TP, NB;
    // Element t of per-position plane k (0 .. NPL-1) of head bh: a head's planes are contiguous
    // ([bh][k][TP]), so a block's values of several planes sit within 32-bit offsets of each other.
    __host__ __device__ int64_t at(int k, int64_t bh, int64_t t) const { return (bh * NPL + k) * TP + t; }
    __host__ __device__ int64_t bplane(int k) const { return NPL * BH * TP + (int64_t)k * BH * NB; }  // 0..1
    __host__ __device__ int64_t total() const { return NPL * BH * TP + 2 * BH * NB; }
};
// Per-key bias terms, betal = beta * log2(e): PL_CA = betal * min(SUF - psi, 0), PL_CP = betal * psi,
// PL_BSUF = betal * SUF (an infinite SUF keeps the sign of beta, and gives 0 when beta = 0).
// PL_BST holds, at positions 0, 1, 2 of each block, the block's BMIN, BLSE and SUF of its first
// position (0 elsewhere): staged with a tile, the kernels read them from LDS, never from memory
// inside their loops.
// How the kernels form the bias beta * min(0, x), x = m - psi_s (m a minimum of PRE, SUF and MID
// values).  For fp32 operands they subtract first and scale after: x is exact when m and psi_s are
// close, as the float32 evaluation of the formula is.  Scaling first, betal * m - betal * psi_s,
// rounds betal * psi_s on its own: phi is a walk whose values reach hundreds at long T, and at
// |betal * psi_s| = 300 that rounding moves every bias of key s by up to 1.5e-5 (base 2), an
// error per key that the sums of dS over queries in dbeta do not cancel.  The fp16 path scales
// first (one VALU operation less per element): its error there is far below what fp16 resolves.
template <typename T>
constexpr bool exact_bias() { return sizeof(T) == 4; }

enum { PL_PHI = 0, PL_PSI = 1, PL_PRE = 2, PL_PREL = 3, PL_SUF = 4, PL_SUFL = 5, PL_CA = 6, PL_CP = 7, PL_BSUF = 8,
       PL_BST = 9 };
enum { BP_MIN = 0, BP_LSE = 1 };

}  // namespace fpa
