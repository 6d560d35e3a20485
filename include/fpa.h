/*
 * fpa.h -- C ABI of the MI355X (gfx950) First Passage Attention library, libfpa.so.
 *
 * Plain C: device pointers, element strides and sizes; no torch or HIP types in
 * the signatures (the stream is passed as the opaque hipStream_t pointer value,
 * NULL = the default stream).  Every buffer is owned by the caller: the library
 * never allocates device memory.  Calls only enqueue work on `stream` and never
 * synchronise the host; they are re-entrant (no global mutable state besides the
 * thread-local error message).
 *
 * Reference interfaces replaced (yliu-fort/first-passage-attention, kernel.py):
 *   fpa_fwd  <- _forward (kernel.py:398-412) with _block_stats (387-395) and the
 *               _stats / _fwd Triton kernels (83-100, 103-162);
 *   fpa_bwd  <- _FirstPassageAttention.backward (kernel.py:424-451) with the
 *               _bwd_delta/_bwd_kv/_bwd_dphi_diag/_bwd_q/_bwd_dphi kernels
 *               (165-370) and the dbeta sum at kernel.py:450 (four kernels here:
 *               delta, key side, query side, phi/beta combine);
 *   fpa_state_floats / fpa_bwd_workspace_bytes <- the scratch allocations of
 *               kernel.py:390-392, 406-407, 430-436, sized so the caller owns them;
 *   fpa_fwd_workspace_bytes: no counterpart in the reference (the scratch of this
 *               forward's split row tiles, see FpaFwdArgs.workspace);
 *   fpa_field_fwd <- Field.forward (kernel.py:502-509): the fp32 projection of x
 *               to (delta, g, h), W = cumsum_t delta, phi = W + g, psi = W + h;
 *   fpa_field_bwd <- the autograd backward of those operations (dx, dW, dbias
 *               from dphi, dpsi), which the reference leaves to torch.
 * Error behaviour mirrors the validation of first_passage_attention
 * (kernel.py:467-486): invalid shapes or dtypes return FPA_ERR_INVALID with the
 * reference's message available from fpa_last_error().
 */
#ifndef FPA_H
#define FPA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype of q, k, v, o, do, dq, dk, dv */
#define FPA_F16 0
#define FPA_F32 1

/* phase bits (FpaFwdArgs.phases / FpaBwdArgs.phases) */
#define FPA_FWD_STATS 1    /* block statistics of phi                      */
#define FPA_FWD_MAIN 2     /* the forward kernel (o, lse)                  */
#define FPA_FWD_MERGE 4    /* o and lse of the split row tiles             */
#define FPA_BWD_DELTA 1    /* Delta_t = sum_d dO o                         */
#define FPA_BWD_KEYS 2     /* key side: dk, dv, dpsi, dbeta partials, ...  */
#define FPA_BWD_QUERIES 4  /* query side: dq, query-block soft-min sums;
                              KEYS | QUERIES runs both sides as one kernel */
#define FPA_BWD_PHI 8      /* dphi and dbeta (one kernel)                  */
#define FPA_BWD_BETA 16    /* same kernel as FPA_BWD_PHI                   */

/* status codes */
#define FPA_OK 0
#define FPA_ERR_INVALID 1     /* invalid argument (shape, dtype, tau, stride)        */
#define FPA_ERR_UNSUPPORTED 2 /* valid for the reference but not built (e.g. D > 256, T > 8388608) */
#define FPA_ERR_HIP 3         /* a HIP runtime call failed                            */

/* Forward arguments.  Tensors are (B, H, T, D) for q/k/v/o and (B, H, T) for
 * phi/psi, addressed with element strides s*[0..3] = (b, h, t, d); the d stride
 * must be 1.  phi, psi, beta are float32; beta is (H,) contiguous.  lse and
 * state are contiguous float32 buffers the forward fills and the backward reads:
 * lse holds 2*B*H*TP floats (TP = T rounded up to 64): for fp16 the base-2
 * log-sum-exp of each query row in the first B*H*TP; for fp32 the row's running
 * maximum there and log2 of its sum in the second half.  state holds
 * fpa_state_floats(B, H, T) floats (block statistics).  */
typedef struct {
    int64_t B, H, T, D;
    int32_t dtype;
    float tau;
    const void *q;  int64_t sq[4];
    const void *k;  int64_t sk[4];
    const void *v;  int64_t sv[4];
    const float *phi; int64_t sphi[3];
    const float *psi; int64_t spsi[3];
    const float *beta;
    void *o;        int64_t so[4];
    float *lse;
    float *state;
    int32_t phases;  /* 0: everything.  Otherwise a bitmask of the kernels to enqueue
                        (FPA_FWD_STATS | FPA_FWD_MAIN | FPA_FWD_MERGE), for per-kernel
                        timing only. */
    void *workspace; /* fpa_fwd_workspace_bytes(...) bytes of device memory, 256-byte
                        aligned, contents on entry irrelevant; or NULL.  When the launch
                        would be short of workgroups, the heaviest row tiles are split in
                        two halves of their key range that run side by side, and a merge
                        kernel combines them through this scratch; with NULL (or a shape
                        that needs none) every row tile runs whole.  Same results up to
                        rounding either way.  Needed only until the call's work ends.  */
} FpaFwdArgs;

/* Backward arguments: the forward's inputs, o, lse and state, the incoming
 * gradient do (strided like q), and the outputs.  dq, dk, dv have the dtype of
 * q and strides sdq/sdk/sdv; dphi, dpsi are float32 (B, H, T) contiguous; dbeta is
 * float32 (H,).  workspace is fpa_bwd_workspace_bytes(...) bytes of device memory,
 * 256-byte aligned; its contents on entry do not matter.                        */
typedef struct {
    int64_t B, H, T, D;
    int32_t dtype;
    float tau;
    const void *q;  int64_t sq[4];
    const void *k;  int64_t sk[4];
    const void *v;  int64_t sv[4];
    const float *beta;
    const void *o;  int64_t so[4];
    const void *dout; int64_t sdo[4];
    const float *lse;
    const float *state;
    void *dq;       int64_t sdq[4];
    void *dk;       int64_t sdk[4];
    void *dv;       int64_t sdv[4];
    float *dphi;
    float *dpsi;
    float *dbeta;
    void *workspace;
    int32_t phases;  /* 0: everything.  Otherwise a bitmask of FPA_BWD_* kernels to enqueue,
                        for per-kernel timing only: a partial run reads the workspace
                        left by an earlier full run and leaves skipped outputs unwritten. */
} FpaBwdArgs;

/* Field prologue of the layer (kernel.py:492-509).  x is (B, T, C) with a unit feature stride,
 * fp16 or fp32; the projection (3H outputs, H <= 32) is computed in fp32. */
typedef struct {
    int64_t B, T, C, H;
    int32_t dtype;          /* of x: FPA_F16 or FPA_F32 */
    const void *x;
    int64_t sx[2];          /* element strides of b and t */
    const float *weight;    /* (3H, C) row-major: Field.proj.weight */
    const float *bias;      /* (3H,): Field.proj.bias */
    float *phi;             /* (B, H, T) contiguous */
    float *psi;             /* (B, H, T) contiguous */
    void *workspace;        /* fpa_field_workspace_bytes(), 256-byte aligned */
} FpaFieldFwdArgs;

typedef struct {
    int64_t B, T, C, H;
    int32_t dtype;          /* of x and dx */
    const void *x;
    int64_t sx[2];
    const float *weight;    /* (3H, C) */
    const float *dphi;      /* (B, H, T) contiguous */
    const float *dpsi;      /* (B, H, T) contiguous */
    void *dx;               /* (B, T, C) like x, or NULL to skip it */
    int64_t sdx[2];
    float *dweight;         /* (3H, C) */
    float *dbias;           /* (3H,) */
    void *workspace;        /* fpa_field_workspace_bytes(), 256-byte aligned */
} FpaFieldBwdArgs;

/* Bytes of scratch of fpa_field_fwd and fpa_field_bwd (the larger of the two). */
int64_t fpa_field_workspace_bytes(int64_t B, int64_t T, int64_t C, int64_t H);

/* Enqueue the Field forward (phi, psi) on `stream`. */
int fpa_field_fwd(const FpaFieldFwdArgs *args, void *stream);

/* Enqueue the Field backward (dx, dweight, dbias) on `stream`.  Deterministic. */
int fpa_field_bwd(const FpaFieldBwdArgs *args, void *stream);

/* Floats of the forward state (block statistics) for a (B, H, T) problem. */
int64_t fpa_state_floats(int64_t B, int64_t H, int64_t T);

/* Floats of lse for a (B, H, T) problem (2 * B * H * TP). */
int64_t fpa_lse_floats(int64_t B, int64_t H, int64_t T);

/* Bytes of forward scratch for a (B, H, T, D) problem: 0 when its forward splits no
 * row tile (see FpaFwdArgs.workspace). */
int64_t fpa_fwd_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D, int32_t dtype);

/* Bytes of backward scratch for a (B, H, T, D) problem. */
int64_t fpa_bwd_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D, int32_t dtype);

/* Enqueue the forward on `stream` (a hipStream_t, NULL for the default stream). */
int fpa_fwd(const FpaFwdArgs *args, void *stream);

/* Enqueue the backward on `stream`. */
int fpa_bwd(const FpaBwdArgs *args, void *stream);

/* The backward without a caller workspace, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart
 * in the reference.  Same arguments and results as fpa_bwd (args->workspace is ignored; should the
 * partial sums of a small launch's split tiles not fit, every tile runs whole, the same results to
 * rounding); the scratch is a static device array of FPA_NOALLOC_SCRATCH_BYTES per GPU, held until
 * the process ends.  Problems whose fpa_bwd_workspace_bytes exceed it return FPA_ERR_UNSUPPORTED before any
 * launch.  Calls that overlap on one GPU (two streams, two threads) share that array and race:
 * serialise them.  Allocates nothing (no hipMalloc or allocating library routine).            */
#define FPA_NOALLOC_SCRATCH_BYTES (64ll << 20)
int fpa_bwd_noalloc(const FpaBwdArgs *args, void *stream);

/* Message of the last failed call on this host thread ("" if none). */
const char *fpa_last_error(void);

/* ABI version (bumped whenever the structs above or the buffer sizes change). */
int fpa_abi_version(void);

/* Hash of the sources the library was built from (16 hex digits; "unknown" when the build did
 * not set it).  The Python loader compares it with the sources next to it and refuses a stale
 * library.  No counterpart in the reference, which compiles its kernels at first call.  */
const char *fpa_source_hash(void);

#ifdef __cplusplus
}
#endif

#endif /* FPA_H */
