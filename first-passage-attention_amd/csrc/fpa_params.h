// fpa_params.h -- kernel parameter blocks and launcher entry points (host <-> device).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fpa {

// Element strides (b, h, t) of a (B, H, T, D) tensor whose d stride is 1.
struct S3 {
    int64_t b, h, t;
};

struct StatsParams {
    const float *phi; S3 sphi;
    const float *psi; S3 spsi;
    const float *beta;
    float *state;
    int H, T, TP, NB, BH;
    float il2;  // log2(e) / tau
};

struct FwdParams {
    const void *q; S3 sq;
    const void *k; S3 sk;
    const void *v; S3 sv;
    void *o; S3 so;
    const float *beta;
    float *lse;          // BH * TP
    const float *state;  // block statistics
    int H, T, TP, NB, BH;
    float sc2;           // log2(e) / sqrt(D)
    // Split rows: the ns heaviest row tiles of each head (rows rs0 .. T-1) run as two items, the keys
    // from the middle tile up to the diagonal (part B: its normalised output goes to o) and the keys
    // below (part A: to ows); fpa_fwd_merge_kernel combines them.  ns = 0: no split.
    void *ows;           // BH * (T - rs0) * D elements of q's type: part A's normalised output
    float *oml;          // BH * (T - rs0) * 4: running maximum and sum of part B, then of part A
    int ns, rs0;
};

struct BwdParams {
    const void *q; S3 sq;
    const void *k; S3 sk;
    const void *v; S3 sv;
    const void *o; S3 so;
    const void *dout; S3 sdo;
    void *dq; S3 sdq;
    void *dk; S3 sdk;
    void *dv; S3 sdv;
    const float *beta;
    const float *lse;
    const float *state;
    float *dphi;   // (B, H, T) contiguous
    float *dpsi;   // (B, H, T) contiguous
    float *dbeta;  // (H,)
    // workspace regions
    float *qinfo;  // BH * NB * QI_PLANES * 64: per-query values of the backward (QI_*)
    float *wsum;   // BH * TP   key-block soft-min sums W_s
    float *rsum;   // BH * TP   query-block soft-min sums R_t
    float *gd;     // BH * NB * G * G   gated dS of in-block pairs, [s][t]
    float *tbuf;   // BH * NB * NB      middle-block sums
    float *dbp;    // 2 * BH * NK32     dbeta partials, one per 32-key group (the second half: far parts)
    // Split tiles (small fused launches): the nks heaviest key tiles (keys < KS = 128 nks) and the nqs
    // heaviest query tiles (queries >= QS) run as two items each over halves of their block range
    // (near: the diagonal side), writing partial results that the combine adds.  KS = 0 and QS = T: none.
    float *pkv;    // 2 * BH * KS * 2D  dK and dV accumulators per part and key
    float *pks;    // 2 * BH * KS * 2   W and the gated dS sum per part and key
    float *pq;     // 2 * BH * (T - QS) * D  dQ accumulators per part and query
    float *pqr;    // 2 * BH * (T - QS)      R per part and query
    int KS, QS;
    int B, H, T, TP, NB, BH, NK32;
    float sc2;     // log2(e) / sqrt(D)
    float smscale; // 1 / sqrt(D)
    float il2;     // log2(e) / tau
};

// The Field prologue (projection of x to (delta, g, h), cumulative sum over t) and its gradient.
struct FieldParams {
    const void *x; int64_t sxb, sxt;    // (B, T, C), unit feature stride
    void *dx; int64_t sdxb, sdxt;       // backward: x's dtype and layout rules (NULL: not computed)
    const float *w;                     // (NO, C) row-major
    const float *bias;                  // (NO,)
    float *lin;                         // the projection, or in the backward its gradient: (B, NO, TL)
    float *phi, *psi;                   // (B, H, T) contiguous
    const float *dphi, *dpsi;           // (B, H, T) contiguous
    float *dw, *dbias;                  // (NO, C), (NO,)
    float *part;                        // (S, NO, C + 1): dW and dbias partials over S splits of the B*T positions
    int B, T, C, H, NO, S;              // NO = 3H
    int TL;                             // lin's row length: T rounded up to 16 (the gradient is zero past T)
};

// BwdParams::qinfo holds, per 64-query block of a head, QI_PLANES planes of 64 floats
// ([bh][block][plane][64]), so the key side stages a block's first four planes with one 1 KB load.
// QI_BST holds the block's BMIN and BLSE at positions 0 and 1; QI_LL (fp32 only) each row's log2 l;
// planes 6-7 are unused.
enum { QI_LQ = 0, QI_DL = 1, QI_PRE = 2, QI_ZQ = 3, QI_BST = 4, QI_LL = 5, QI_PLANES = 8 };
__host__ __device__ inline int64_t qi_at(int64_t bh, int NB, int row, int plane) {
    return ((bh * NB + row / 64) * QI_PLANES + plane) * 64 + row % 64;
}

// Launchers (defined next to their kernels); return hipSuccess or the launch error.
hipError_t launch_stats(const StatsParams &p, hipStream_t s);
hipError_t launch_fwd(const FwdParams &p, int dtype, int D, hipStream_t s);
hipError_t launch_fwd_merge(const FwdParams &p, int dtype, int D, hipStream_t s);
// Row tiles per head that the forward splits (0: none) for a (BH, T) problem.
int fwd_split_tiles(int64_t BH, int64_t T, int dtype, int D);
hipError_t launch_bwd_prep(const BwdParams &p, int dtype, int D, hipStream_t s);
hipError_t launch_bwd_kv(const BwdParams &p, int dtype, int D, hipStream_t s);
hipError_t launch_bwd_q(const BwdParams &p, int dtype, int D, hipStream_t s);
hipError_t launch_bwd_kvq(const BwdParams &p, int dtype, int D, hipStream_t s);  // both sides, one launch
hipError_t launch_bwd_combine(const BwdParams &p, hipStream_t s);
// Adds the two parts of the split tiles (before the combine): dk, dv, dpsi, W, dq, R, dbeta partials.
hipError_t launch_bwd_merge(const BwdParams &p, int dtype, int D, hipStream_t s);
// Key and query tiles per head that the fused backward splits (0, 0: none) for a (BH, T) problem.
void bwd_split_tiles(int64_t BH, int64_t T, int dtype, int D, int &nks, int &nqs);
hipError_t launch_field_fwd(const FieldParams &p, int dtype, hipStream_t s);
hipError_t launch_field_bwd(const FieldParams &p, int dtype, hipStream_t s);

// Head dimensions with built kernels.
inline bool supported_d(int dtype, int D) {
    (void)dtype;
    return D == 16 || D == 32 || D == 64 || D == 128 || D == 256;
}

// Most 64-blocks of T: T <= 8388608.  The backward workspace holds 4 bytes per block pair (TBUF), 64 GiB
// per head at this cap; every index into it is 64-bit, and the 32-bit values derived from the block count
// stay below 2^31 (positions, workgroup ids, 32-bit offsets of at most ten planes of TP floats).
constexpr int MAX_NB = 131072;

}  // namespace fpa
