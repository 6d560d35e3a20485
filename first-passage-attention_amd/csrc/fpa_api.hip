// fpa_api.hip -- the extern "C" entry points of libfpa.so (declared in include/fpa.h).
//
// Validation mirrors first_passage_attention (kernel.py:467-486 of
// yliu-fort/first-passage-attention); scratch sizing replaces the torch allocations of
// kernel.py:390-392, 406-407 and 430-436 so that the caller owns every buffer.
#include <stdint.h>

#include <mutex>
#include <string>

#include "fpa.h"
#include "fpa_common.h"
#include "fpa_params.h"

using namespace fpa;

namespace {

thread_local std::string g_err;

int fail(int code, const std::string &msg) {
    g_err = msg;
    return code;
}

int64_t tp_of(int64_t T) { return ((T + G - 1) / G) * G; }
int64_t align64(int64_t n) { return (n + 63) / 64 * 64; }  // floats -> 256-byte multiple

struct WsLayout {
    int64_t qinfo, wsum, rsum, gd, tbuf, dbp, pkv, pks, pq, pqr, total;  // float offsets
    int64_t KS, QS;  // split keys < KS and queries >= QS (KS = 0, QS = T: no split)
};

// The split-tile regions are sized for the launch that runs both backward sides as one (the fused
// launch splits its heaviest tiles when it fills few of the GPU's slots).
WsLayout ws_layout(int64_t B, int64_t H, int64_t T, int64_t D, int32_t dtype, bool split_ok = true) {
    const int64_t BH = B * H, TP = tp_of(T), NB = TP / G, NK32 = (T + 31) / 32;
    WsLayout w;
    int64_t off = 0;
    w.qinfo = off; off += align64((int64_t)QI_PLANES * BH * TP);
    w.wsum = off;  off += align64(BH * TP);
    w.rsum = off;  off += align64(BH * TP);
    w.gd = off;    off += align64(BH * NB * G * G);
    w.tbuf = off;  off += align64(BH * NB * NB);
    w.dbp = off;   off += align64(2 * BH * NK32);
    int nks = 0, nqs = 0;
    if (split_ok && (dtype == FPA_F16 || dtype == FPA_F32) && supported_d(dtype, (int)D))
        bwd_split_tiles(BH, T, dtype, (int)D, nks, nqs);
    const int64_t BT = 32 * FPA_NW, nt = (T + BT - 1) / BT;
    w.KS = nks * BT;
    w.QS = nqs ? (nt - nqs) * BT : T;
    w.pkv = off;   off += align64(2 * BH * w.KS * 2 * D);
    w.pks = off;   off += align64(2 * BH * w.KS * 2);
    w.pq = off;    off += align64(2 * BH * (T - w.QS) * D);
    w.pqr = off;   off += align64(2 * BH * (T - w.QS));
    w.total = off;
    return w;
}

S3 s3(const int64_t *s) { return S3{s[0], s[1], s[2]}; }

// Field scratch: the projection (or its gradient) as B * 3H rows of TL = T rounded up to 16 floats,
// then the dW / dbias partials.
struct FieldLayout {
    int64_t lin, part, total;  // float offsets
    int S;
};
int64_t field_tl(int64_t T) { return (T + 15) / 16 * 16; }
FieldLayout field_layout(int64_t B, int64_t T, int64_t C, int64_t H) {
    FieldLayout f;
    const int64_t N = B * T;
    f.S = (int)((N + 255) / 256 < 64 ? (N + 255) / 256 : 64);
    f.lin = 0;
    f.part = align64(B * 3 * H * field_tl(T));
    f.total = f.part + align64((int64_t)f.S * 3 * H * (C + 1));  // the bias is feature C
    return f;
}

int check_field(int64_t B, int64_t T, int64_t C, int64_t H, int32_t dtype, const void *x, const int64_t *sx,
                const float *weight, const void *ws) {
    if (B < 1 || T < 1 || C < 1 || H < 1) return fail(FPA_ERR_INVALID, "x must be (B, T, C) with B, T, C >= 1 and n_heads >= 1");
    if (dtype != FPA_F16 && dtype != FPA_F32) return fail(FPA_ERR_INVALID, "x must be fp16 or fp32");
    if (H > 32) return fail(FPA_ERR_UNSUPPORTED, "the Field kernels take at most 32 heads");
    if (B > 65535 || B * field_tl(T) >= (int64_t(1) << 31) || C > (int64_t(1) << 24))
        return fail(FPA_ERR_UNSUPPORTED, "x is too large for the Field kernels");
    if (!x || !weight || !ws) return fail(FPA_ERR_INVALID, "x, weight and workspace must be non-NULL");
    if (sx[0] < 0 || sx[1] < 0) return fail(FPA_ERR_INVALID, "x strides must be non-negative");
    if ((reinterpret_cast<uintptr_t>(ws) & 255) != 0) return fail(FPA_ERR_INVALID, "workspace must be 256-byte aligned");
    return FPA_OK;
}

// Shared checks of the forward and backward arguments.
int check_common(int64_t B, int64_t H, int64_t T, int64_t D, int32_t dtype, float tau) {
    if (B < 1 || H < 1 || T < 1) return fail(FPA_ERR_INVALID, "q, k and v must have the same shape (B, H, T, D)");
    if (dtype != FPA_F16 && dtype != FPA_F32) return fail(FPA_ERR_INVALID, "q, k and v must all be fp16 or all fp32");
    if (D < 16 || (D & (D - 1)) != 0)
        return fail(FPA_ERR_INVALID, "the head dimension and the block must be powers of two >= 16");
    if (!(tau > 0.f)) return fail(FPA_ERR_INVALID, "tau must be positive");
    if (!supported_d(dtype, (int)D))
        return fail(FPA_ERR_UNSUPPORTED, "head dimension " + std::to_string(D) + " is not built (16, 32, 64, 128, 256)");
    if (B > 65535 || H > 65535) return fail(FPA_ERR_UNSUPPORTED, "B and H must each be at most 65535");
    // The backward workspace grows as the square of the block count; workgroup counts stay below 2^31.
    if (tp_of(T) / G > MAX_NB) return fail(FPA_ERR_UNSUPPORTED, "T must be at most " + std::to_string(MAX_NB * G));
    if (B * H * (tp_of(T) / G + 1) >= (int64_t(1) << 31)) return fail(FPA_ERR_UNSUPPORTED, "B * H * T is too large");
    return FPA_OK;
}

// 16-byte row alignment of a (B, H, T, D) tensor with unit d stride.
int check_rows(const void *ptr, const int64_t *st, int32_t dtype, const char *name) {
    if (ptr == nullptr) return fail(FPA_ERR_INVALID, std::string(name) + " is NULL");
    const int64_t ce = (dtype == FPA_F16) ? 8 : 4;
    if ((reinterpret_cast<uintptr_t>(ptr) & 15) != 0 || st[0] % ce || st[1] % ce || st[2] % ce)
        return fail(FPA_ERR_INVALID, std::string(name) +
                                         " rows must be 16-byte aligned (contiguous head dimension, aligned strides)");
    // Tile loads address 64 rows with 32-bit byte offsets from the first row.
    if (st[2] < 0 || st[2] * 64 * (ce == 8 ? 2 : 4) >= (int64_t(1) << 31))
        return fail(FPA_ERR_INVALID, std::string(name) + " row stride is out of range (at most 2^25 bytes)");
    return FPA_OK;
}

int hip_fail(hipError_t e, const char *where) {
    return fail(FPA_ERR_HIP, std::string(where) + ": " + hipGetErrorString(e));
}

// Forward scratch: part A's normalised output of the split rows (q's type), then four floats per
// split row (running maximum and sum of parts B and A).  ns = 0: no split, no scratch.
struct FwdWs {
    int ns = 0;
    int64_t rs0 = 0, obytes = 0, total = 0;  // bytes
};

FwdWs fwd_ws(int64_t B, int64_t H, int64_t T, int64_t D, int32_t dtype) {
    FwdWs f;
    if (B < 1 || H < 1 || T < 1 || (dtype != FPA_F16 && dtype != FPA_F32) || !supported_d(dtype, (int)D)) return f;
    f.ns = fwd_split_tiles(B * H, T, dtype, (int)D);
    if (f.ns == 0) return f;
    const int64_t BM = 32 * FPA_NW, nqt = (T + BM - 1) / BM;
    f.rs0 = (nqt - f.ns) * BM;
    const int64_t rows = B * H * (T - f.rs0);
    f.obytes = (rows * D * (dtype == FPA_F16 ? 2 : 4) + 255) / 256 * 256;
    f.total = f.obytes + rows * 16;
    return f;
}

}  // namespace

#ifndef FPA_SOURCE_HASH
#define FPA_SOURCE_HASH "unknown"
#endif

extern "C" {

int fpa_abi_version(void) { return 5; }

const char *fpa_source_hash(void) { return FPA_SOURCE_HASH; }

const char *fpa_last_error(void) { return g_err.c_str(); }

int64_t fpa_state_floats(int64_t B, int64_t H, int64_t T) {
    const int64_t TP = tp_of(T);
    return StateLayout{B * H, TP, TP / G}.total();
}

int64_t fpa_lse_floats(int64_t B, int64_t H, int64_t T) { return 2 * B * H * tp_of(T); }

int64_t fpa_fwd_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D, int32_t dtype) {
    return fwd_ws(B, H, T, D, dtype).total;
}

int64_t fpa_bwd_workspace_bytes(int64_t B, int64_t H, int64_t T, int64_t D, int32_t dtype) {
    return ws_layout(B, H, T, D, dtype).total * (int64_t)sizeof(float);
}

int64_t fpa_field_workspace_bytes(int64_t B, int64_t T, int64_t C, int64_t H) {
    return field_layout(B, T, C, H).total * (int64_t)sizeof(float);
}

int fpa_field_fwd(const FpaFieldFwdArgs *a, void *stream) {
    g_err.clear();
    if (a == nullptr) return fail(FPA_ERR_INVALID, "args is NULL");
    int rc = check_field(a->B, a->T, a->C, a->H, a->dtype, a->x, a->sx, a->weight, a->workspace);
    if (rc) return rc;
    if (!a->bias || !a->phi || !a->psi) return fail(FPA_ERR_INVALID, "bias, phi and psi must be non-NULL");
    const FieldLayout fl = field_layout(a->B, a->T, a->C, a->H);
    FieldParams p = {};
    p.x = a->x; p.sxb = a->sx[0]; p.sxt = a->sx[1];
    p.w = a->weight; p.bias = a->bias;
    p.lin = static_cast<float *>(a->workspace) + fl.lin;
    p.phi = a->phi; p.psi = a->psi;
    p.B = (int)a->B; p.T = (int)a->T; p.C = (int)a->C; p.H = (int)a->H; p.NO = 3 * (int)a->H; p.S = fl.S;
    p.TL = (int)field_tl(a->T);
    const hipError_t e = launch_field_fwd(p, a->dtype, reinterpret_cast<hipStream_t>(stream));
    return e != hipSuccess ? hip_fail(e, "fpa_field_fwd launch") : FPA_OK;
}

int fpa_field_bwd(const FpaFieldBwdArgs *a, void *stream) {
    g_err.clear();
    if (a == nullptr) return fail(FPA_ERR_INVALID, "args is NULL");
    int rc = check_field(a->B, a->T, a->C, a->H, a->dtype, a->x, a->sx, a->weight, a->workspace);
    if (rc) return rc;
    if (!a->dphi || !a->dpsi || !a->dweight || !a->dbias)
        return fail(FPA_ERR_INVALID, "dphi, dpsi, dweight and dbias must be non-NULL");
    if (a->dx && (a->sdx[0] < 0 || a->sdx[1] < 0)) return fail(FPA_ERR_INVALID, "dx strides must be non-negative");
    const FieldLayout fl = field_layout(a->B, a->T, a->C, a->H);
    FieldParams p = {};
    p.x = a->x; p.sxb = a->sx[0]; p.sxt = a->sx[1];
    p.dx = a->dx; p.sdxb = a->sdx[0]; p.sdxt = a->sdx[1];
    p.w = a->weight;
    p.lin = static_cast<float *>(a->workspace) + fl.lin;
    p.part = static_cast<float *>(a->workspace) + fl.part;
    p.dphi = a->dphi; p.dpsi = a->dpsi;
    p.dw = a->dweight; p.dbias = a->dbias;
    p.B = (int)a->B; p.T = (int)a->T; p.C = (int)a->C; p.H = (int)a->H; p.NO = 3 * (int)a->H; p.S = fl.S;
    p.TL = (int)field_tl(a->T);
    const hipError_t e = launch_field_bwd(p, a->dtype, reinterpret_cast<hipStream_t>(stream));
    return e != hipSuccess ? hip_fail(e, "fpa_field_bwd launch") : FPA_OK;
}

int fpa_fwd(const FpaFwdArgs *a, void *stream) {
    g_err.clear();
    if (a == nullptr) return fail(FPA_ERR_INVALID, "args is NULL");
    int rc = check_common(a->B, a->H, a->T, a->D, a->dtype, a->tau);
    if (rc) return rc;
    if ((rc = check_rows(a->q, a->sq, a->dtype, "q")) || (rc = check_rows(a->k, a->sk, a->dtype, "k")) ||
        (rc = check_rows(a->v, a->sv, a->dtype, "v")) || (rc = check_rows(a->o, a->so, a->dtype, "o")))
        return rc;
    if (a->sq[3] != 1 || a->sk[3] != 1 || a->sv[3] != 1 || a->so[3] != 1)
        return fail(FPA_ERR_INVALID, "the head dimension of q, k, v and o must be contiguous");
    if (!a->phi || !a->psi || !a->beta || !a->lse || !a->state)
        return fail(FPA_ERR_INVALID, "phi, psi, beta, lse and state must be non-NULL");
    if ((reinterpret_cast<uintptr_t>(a->workspace) & 255) != 0)
        return fail(FPA_ERR_INVALID, "workspace must be 256-byte aligned");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int64_t TP = tp_of(a->T);
    StatsParams sp;
    sp.phi = a->phi; sp.sphi = s3(a->sphi);
    sp.psi = a->psi; sp.spsi = s3(a->spsi);
    sp.beta = a->beta;
    sp.state = a->state;
    sp.H = (int)a->H; sp.T = (int)a->T; sp.TP = (int)TP; sp.NB = (int)(TP / G); sp.BH = (int)(a->B * a->H);
    sp.il2 = LOG2E / a->tau;
    const int ph = a->phases ? a->phases : (FPA_FWD_STATS | FPA_FWD_MAIN | FPA_FWD_MERGE);
    hipError_t e;
    if ((ph & FPA_FWD_STATS) && (e = launch_stats(sp, s)) != hipSuccess) return hip_fail(e, "fpa_stats launch");
    FwdParams fp;
    fp.q = a->q; fp.sq = s3(a->sq);
    fp.k = a->k; fp.sk = s3(a->sk);
    fp.v = a->v; fp.sv = s3(a->sv);
    fp.o = a->o; fp.so = s3(a->so);
    fp.beta = a->beta; fp.lse = a->lse; fp.state = a->state;
    fp.H = sp.H; fp.T = sp.T; fp.TP = sp.TP; fp.NB = sp.NB; fp.BH = sp.BH;
    fp.sc2 = LOG2E / sqrtf((float)a->D);
    const FwdWs fw = a->workspace ? fwd_ws(a->B, a->H, a->T, a->D, a->dtype) : FwdWs{};
    fp.ns = fw.ns;
    fp.rs0 = (int)fw.rs0;
    fp.ows = fw.ns ? a->workspace : nullptr;
    fp.oml = fw.ns ? reinterpret_cast<float *>(static_cast<char *>(a->workspace) + fw.obytes) : nullptr;
    if ((ph & FPA_FWD_MAIN) && (e = launch_fwd(fp, a->dtype, (int)a->D, s)) != hipSuccess)
        return hip_fail(e, "fpa_fwd launch");
    if (fp.ns && (ph & FPA_FWD_MERGE) && (e = launch_fwd_merge(fp, a->dtype, (int)a->D, s)) != hipSuccess)
        return hip_fail(e, "fpa_fwd_merge launch");
    return FPA_OK;
}

}  // extern "C"

namespace {

// The backward of fpa_bwd and fpa_bwd_noalloc: every check but the workspace's, then the launches
// with their scratch regions carved out of `wsp` (fpa_bwd_workspace_bytes bytes, 256-byte aligned;
// with split_ok false, the layout without split tiles).
int bwd_impl(const FpaBwdArgs *a, void *wsp, void *stream, bool split_ok = true) {
    int rc = check_common(a->B, a->H, a->T, a->D, a->dtype, a->tau);
    if (rc) return rc;
    if ((rc = check_rows(a->q, a->sq, a->dtype, "q")) || (rc = check_rows(a->k, a->sk, a->dtype, "k")) ||
        (rc = check_rows(a->v, a->sv, a->dtype, "v")) || (rc = check_rows(a->o, a->so, a->dtype, "o")) ||
        (rc = check_rows(a->dout, a->sdo, a->dtype, "do")) || (rc = check_rows(a->dq, a->sdq, a->dtype, "dq")) ||
        (rc = check_rows(a->dk, a->sdk, a->dtype, "dk")) || (rc = check_rows(a->dv, a->sdv, a->dtype, "dv")))
        return rc;
    if (a->sq[3] != 1 || a->sk[3] != 1 || a->sv[3] != 1 || a->so[3] != 1 || a->sdo[3] != 1 || a->sdq[3] != 1 ||
        a->sdk[3] != 1 || a->sdv[3] != 1)
        return fail(FPA_ERR_INVALID, "the head dimension of every (B, H, T, D) tensor must be contiguous");
    if (!a->beta || !a->lse || !a->state || !a->dphi || !a->dpsi || !a->dbeta)
        return fail(FPA_ERR_INVALID, "beta, lse, state, dphi, dpsi and dbeta must be non-NULL");
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    const int64_t TP = tp_of(a->T);
    const WsLayout wl = ws_layout(a->B, a->H, a->T, a->D, a->dtype, split_ok);
    float *ws = static_cast<float *>(wsp);
    BwdParams p;
    p.q = a->q; p.sq = s3(a->sq);
    p.k = a->k; p.sk = s3(a->sk);
    p.v = a->v; p.sv = s3(a->sv);
    p.o = a->o; p.so = s3(a->so);
    p.dout = a->dout; p.sdo = s3(a->sdo);
    p.dq = a->dq; p.sdq = s3(a->sdq);
    p.dk = a->dk; p.sdk = s3(a->sdk);
    p.dv = a->dv; p.sdv = s3(a->sdv);
    p.beta = a->beta; p.lse = a->lse; p.state = a->state;
    p.dphi = a->dphi; p.dpsi = a->dpsi; p.dbeta = a->dbeta;
    p.qinfo = ws + wl.qinfo;
    p.wsum = ws + wl.wsum; p.rsum = ws + wl.rsum;
    p.gd = ws + wl.gd; p.tbuf = ws + wl.tbuf; p.dbp = ws + wl.dbp;
    p.pkv = ws + wl.pkv; p.pks = ws + wl.pks; p.pq = ws + wl.pq; p.pqr = ws + wl.pqr;
    p.B = (int)a->B; p.H = (int)a->H; p.T = (int)a->T; p.TP = (int)TP; p.NB = (int)(TP / G);
    p.BH = (int)(a->B * a->H); p.NK32 = (int)((a->T + 31) / 32);
    p.sc2 = LOG2E / sqrtf((float)a->D);
    p.smscale = 1.0f / sqrtf((float)a->D);
    p.il2 = LOG2E / a->tau;
    const int ph = a->phases ? a->phases : 31;
    // The split tiles run only in the launch of both sides together; their merge follows it.
    const bool both = (ph & FPA_BWD_KEYS) && (ph & FPA_BWD_QUERIES);
    p.KS = both ? (int)wl.KS : 0;
    p.QS = both ? (int)wl.QS : p.T;
    hipError_t e;
    if ((ph & FPA_BWD_DELTA) && (e = launch_bwd_prep(p, a->dtype, (int)a->D, s)) != hipSuccess)
        return hip_fail(e, "fpa_bwd_prep launch");
    if (both) {
        if ((e = launch_bwd_kvq(p, a->dtype, (int)a->D, s)) != hipSuccess) return hip_fail(e, "fpa_bwd_kvq launch");
        if (p.KS > 0 && (e = launch_bwd_merge(p, a->dtype, (int)a->D, s)) != hipSuccess)
            return hip_fail(e, "fpa_bwd_merge launch");
    } else {
        if ((ph & FPA_BWD_KEYS) && (e = launch_bwd_kv(p, a->dtype, (int)a->D, s)) != hipSuccess)
            return hip_fail(e, "fpa_bwd_kv launch");
        if ((ph & FPA_BWD_QUERIES) && (e = launch_bwd_q(p, a->dtype, (int)a->D, s)) != hipSuccess)
            return hip_fail(e, "fpa_bwd_q launch");
    }
    if ((ph & (FPA_BWD_PHI | FPA_BWD_BETA)) && (e = launch_bwd_combine(p, s)) != hipSuccess)
        return hip_fail(e, "fpa_bwd_combine launch");
    return FPA_OK;
}

// Scratch of fpa_bwd_noalloc: one array per GPU, placed by the code object's loader (no allocation
// call), found once per device with hipGetSymbolAddress.  In host code `scratch` names a host-side
// stand-in, not device memory: only the address in g_scratch_ptr is ever passed on.
static __device__ __align__(256) char scratch[FPA_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 256;
std::mutex g_scratch_mu;
void *g_scratch_ptr[MAX_DEVICES] = {};

// Device address of this GPU's scratch (the current device), or nullptr with the error set.
void *scratch_of_current_device() {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        hip_fail(e, "fpa_bwd_noalloc: hipGetDevice");
        return nullptr;
    }
    if (dev < 0 || dev >= MAX_DEVICES) {
        fail(FPA_ERR_UNSUPPORTED, "fpa_bwd_noalloc: device index out of range");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "fpa_bwd_noalloc: hipGetSymbolAddress(scratch)");
            return nullptr;
        }
        g_scratch_ptr[dev] = p;
    }
    return g_scratch_ptr[dev];
}

}  // namespace

extern "C" {

int fpa_bwd(const FpaBwdArgs *a, void *stream) {
    g_err.clear();
    if (a == nullptr) return fail(FPA_ERR_INVALID, "args is NULL");
    if (a->workspace == nullptr) return fail(FPA_ERR_INVALID, "workspace must be non-NULL");
    if ((reinterpret_cast<uintptr_t>(a->workspace) & 255) != 0)
        return fail(FPA_ERR_INVALID, "workspace must be 256-byte aligned");
    return bwd_impl(a, a->workspace, stream);
}

int fpa_bwd_noalloc(const FpaBwdArgs *a, void *stream) {
    g_err.clear();
    if (a == nullptr) return fail(FPA_ERR_INVALID, "args is NULL");
    int rc = check_common(a->B, a->H, a->T, a->D, a->dtype, a->tau);
    if (rc) return rc;
    // The partial sums of split tiles are left out (every tile whole) when they alone would not fit.
    const bool split_ok = ws_layout(a->B, a->H, a->T, a->D, a->dtype).total * (int64_t)sizeof(float) <=
                          FPA_NOALLOC_SCRATCH_BYTES;
    const int64_t need = ws_layout(a->B, a->H, a->T, a->D, a->dtype, split_ok).total * (int64_t)sizeof(float);
    if (need > FPA_NOALLOC_SCRATCH_BYTES)
        return fail(FPA_ERR_UNSUPPORTED, "fpa_bwd_noalloc: this problem needs " + std::to_string(need) +
                                             " bytes of scratch, more than the " +
                                             std::to_string((int64_t)FPA_NOALLOC_SCRATCH_BYTES) +
                                             " it holds; call fpa_bwd with a workspace");
    void *ws = scratch_of_current_device();
    if (ws == nullptr) return FPA_ERR_HIP;
    return bwd_impl(a, ws, stream, split_ok);
}

}  // extern "C"
