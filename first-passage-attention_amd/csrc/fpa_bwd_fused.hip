// fpa_bwd_fused.hip -- the key-side and query-side backward tiles in one launch.
//
// Reference behaviour: _bwd_kv (kernel.py:177-265) and _bwd_q (kernel.py:286-340) of
// yliu-fort/first-passage-attention, which run as two launches there.  The two sides depend
// on the per-query preparation only, not on each other.  Their work is triangular (key tiles
// near 0 and query tiles near T cover the most blocks), so a launch of either side alone
// ends with the chip partly idle while its longest workgroups finish.  One grid holding both
// kinds of workgroup, ordered longest first by an estimate of their cost, keeps every CU busy
// to the end.  Each workgroup computes exactly what it computes in the separate kernels.
#include <algorithm>

#include "fpa_bwd_kv.h"
#include "fpa_bwd_q.h"

// Relative cost of one block iteration of the key side and of the query side, for the order
// of the fused grid (measured alone at D = 64 fp16: about 1.2; the fused launch is fastest with
// weights 5:4 to 6:5, 1% ahead of 3:2 and 4% ahead of 1:1 at cfg2, level at cfg4).
#ifndef FPA_FUSE_WKV
#define FPA_FUSE_WKV 5
#endif
#ifndef FPA_FUSE_WQ
#define FPA_FUSE_WQ 4
#endif
// Split the heaviest half of the key tiles and of the query tiles (two items each over halves of their
// block range) when the fused launch fills at most this percentage of the slots; 0 never splits.
// Measured at D = 64 fp16: 75% of the slots (B1 H12 T2048) 81 -> 59 us, 100% (B2 H8 T2048) 80.7 -> 79.0,
// 150% (B2 H12 T2048) 86 -> 102.
#ifndef FPA_BWD_SPLIT_FILL
#define FPA_BWD_SPLIT_FILL 100
#endif

namespace fpa {

// Workgroup slots of the fused grid (per head): key tiles and query tiles together.
constexpr int FUSED_MAX = 1024;

// Slot -> tile: a key tile index, or a query tile index with bit 15 set; in a split launch bits 13-14
// name the half of a split tile (1: the diagonal side, 2: the rest).  Passed by value (2 KB of kernel
// arguments); the index is uniform, so each workgroup reads one entry with a scalar load.
struct BwdOrder {
    uint16_t e[FUSED_MAX];
};

template <typename T, int D, int NW>
union BwdShared {
    KvShared<T, D, NW> kv;
    QShared<T, D, NW> q;
};

template <typename T, int D, int WPE, int NW>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
fpa_bwd_kvq_kernel(BwdParams p, BwdOrder ord) {
    __shared__ BwdShared<T, D, NW> sm;
    int slot, bh;
    xcd_work_item(slot, bh, p.BH, p.H, 2 * ((p.T + 32 * NW - 1) / (32 * NW)));
    const int e = __builtin_amdgcn_readfirstlane((int)ord.e[slot]);
    if (e & 0x8000)
        bwd_q_tile<T, D, NW>(p, sm.q, e & 0x7fff, bh);
    else
        bwd_kv_tile<T, D, NW>(p, sm.kv, e, bh);
}

// The same grid with the heaviest tiles split in halves (nslots items per head).
template <typename T, int D, int WPE, int NW>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
fpa_bwd_kvq_split_kernel(BwdParams p, BwdOrder ord, int nslots) {
    __shared__ BwdShared<T, D, NW> sm;
    int slot, bh;
    xcd_work_item(slot, bh, p.BH, p.H, nslots);
    const int e = __builtin_amdgcn_readfirstlane((int)ord.e[slot]);
    const int tile = e & 0x1fff, half = (e >> 13) & 3;
    if (e & 0x8000)
        bwd_q_tile<T, D, NW, true>(p, sm.q, tile, bh, half);
    else
        bwd_kv_tile<T, D, NW, true>(p, sm.kv, tile, bh, 0, half);
}

// Whether the fused launch applies to this dtype and D (both sides one launch shape, one dK / dV part,
// not fp32 at D = 64); it also needs at most FUSED_MAX slots per head.
template <typename T, int D>
constexpr bool kvq_fused() {
    return kv_wpe<T, D>() == q_wpe<T, D>() && kv_parts<T, D>() == 1 && !(sizeof(T) == 4 && D == 64);
}

template <typename T, int D>
static hipError_t launch_kvq_t(const BwdParams &p, hipStream_t s) {
    constexpr int NW = FPA_NW, BT = 32 * NW, WPE = kv_wpe<T, D>();
    const int nt = (p.T + BT - 1) / BT;  // key tiles; as many query tiles
    auto two_launches = [&]() {
        hipError_t e = launch_bwd_kv(p, sizeof(T) == 2 ? 0 : 1, D, s);
        return e != hipSuccess ? e : launch_bwd_q(p, sizeof(T) == 2 ? 0 : 1, D, s);
    };
    // No common launch shape, or (fp32 at D = 64, one wave per SIMD) two launches measured 2% faster.
    if constexpr (!kvq_fused<T, D>()) {
        return two_launches();
    } else {
        if (2 * nt > FUSED_MAX) return two_launches();
        // Block iterations of key tile kt (query blocks from its diagonal block to the end) and of
        // query tile qt (key blocks from its diagonal block down to 0), weighted by their cost.
        auto c_kv = [&](int kt) { return FPA_FUSE_WKV * (p.NB - kt * BT / G); };
        auto c_q = [&](int qt) { return FPA_FUSE_WQ * (std::min(p.NB - 1, (qt * BT + BT - 1) / G) + 1); };
        BwdOrder ord;
        int n = 0;
        if (p.KS == 0) {
            for (int kt = 0, qt = nt - 1; kt < nt || qt >= 0;) {  // merge, costliest first
                if (qt < 0 || (kt < nt && c_kv(kt) >= c_q(qt)))
                    ord.e[n++] = (uint16_t)kt++;
                else
                    ord.e[n++] = (uint16_t)(0x8000 | qt--);
            }
            hipLaunchKernelGGL((fpa_bwd_kvq_kernel<T, D, WPE, NW>), head_grid(n, p.H, p.BH), dim3(64 * NW), 0, s, p,
                               ord);
        } else {
            // Split launch: key tiles below KS / BT and query tiles from QS / BT on run as two halves,
            // their costs split where the kernels split their block ranges; all items by cost, costliest first.
            const int nks = p.KS / BT, q0s = p.QS / BT;
            int cost[FUSED_MAX];
            auto add = [&](int c, int e) { cost[n] = c; ord.e[n++] = (uint16_t)e; };
            for (int kt = 0; kt < nt; ++kt) {
                const int ib0 = kt * BT / G, nblk = p.NB - ib0;
                if (kt < nks) {
                    const int nnear = std::max(2, nblk / 2);
                    add(FPA_FUSE_WKV * nnear, kt | (1 << 13));
                    add(FPA_FUSE_WKV * (nblk - nnear), kt | (2 << 13));
                } else {
                    add(c_kv(kt), kt);
                }
            }
            for (int qt = 0; qt < nt; ++qt) {
                const int nblk = std::min(p.NB - 1, (qt * BT + BT - 1) / G) + 1;
                if (qt >= q0s) {
                    const int nnear = std::max(2, nblk / 2);
                    add(FPA_FUSE_WQ * nnear, 0x8000 | qt | (1 << 13));
                    add(FPA_FUSE_WQ * (nblk - nnear), 0x8000 | qt | (2 << 13));
                } else {
                    add(c_q(qt), 0x8000 | qt);
                }
            }
            int idx[FUSED_MAX];
            for (int i = 0; i < n; ++i) idx[i] = i;
            std::stable_sort(idx, idx + n, [&](int a, int b) { return cost[a] > cost[b]; });
            BwdOrder sorted;
            for (int i = 0; i < n; ++i) sorted.e[i] = ord.e[idx[i]];
            hipLaunchKernelGGL((fpa_bwd_kvq_split_kernel<T, D, WPE, NW>), head_grid(n, p.H, p.BH), dim3(64 * NW), 0, s,
                               p, sorted, n);
        }
        return hipGetLastError();
    }
}

template <typename T, int D>
static void split_t(int64_t BH, int64_t T_, int &nks, int &nqs) {
    constexpr int BT = 32 * FPA_NW;
    nks = nqs = 0;
    if constexpr (kvq_fused<T, D>()) {
        const int64_t nt = (T_ + BT - 1) / BT;
        if (nt < 4 || 2 * nt + nt > FUSED_MAX) return;
        if (100 * 2 * nt * BH > (int64_t)FPA_BWD_SPLIT_FILL * 8 * XCD_CUS * kv_wpe<T, D>()) return;
        nks = nqs = (int)(nt / 2);
    }
}

void bwd_split_tiles(int64_t BH, int64_t T, int dtype, int D, int &nks, int &nqs) {
    nks = nqs = 0;
    if (dtype == 0) {
        switch (D) {
            case 16: return split_t<f16, 16>(BH, T, nks, nqs);
            case 32: return split_t<f16, 32>(BH, T, nks, nqs);
            case 64: return split_t<f16, 64>(BH, T, nks, nqs);
            case 128: return split_t<f16, 128>(BH, T, nks, nqs);
            case 256: return split_t<f16, 256>(BH, T, nks, nqs);
        }
    } else {
        switch (D) {
            case 16: return split_t<float, 16>(BH, T, nks, nqs);
            case 32: return split_t<float, 32>(BH, T, nks, nqs);
            case 64: return split_t<float, 64>(BH, T, nks, nqs);
            case 128: return split_t<float, 128>(BH, T, nks, nqs);
            case 256: return split_t<float, 256>(BH, T, nks, nqs);
        }
    }
}

// The two halves of the split tiles added, in a fixed order: for each split key s < KS its dK (times
// 1/sqrt(D)), dV, W and dpsi; for each split query t in [QS, T) its dQ (times 1/sqrt(D)) and R; for each
// 32-key group of split keys its dbeta partial (the far half's added to the near half's).  One thread per
// 16-byte fp32 chunk of a row (the per-row scalars with the first chunk), then one per group.
template <typename T, int D>
__global__ void __launch_bounds__(256) fpa_bwd_merge_kernel(BwdParams p) {
    constexpr int CPR = D / 4;
    const int nqs = p.T - p.QS, ngk = p.KS / 32;
    const int64_t nk = (int64_t)p.BH * p.KS * CPR, nq = (int64_t)p.BH * nqs * CPR, ng = (int64_t)p.BH * ngk;
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    auto store4 = [](T *dst, const f32x4 &v) {
        if constexpr (sizeof(T) == 2)
            *reinterpret_cast<h4 *>(dst) = h4{(f16)v[0], (f16)v[1], (f16)v[2], (f16)v[3]};
        else
            *reinterpret_cast<f32x4 *>(dst) = v;
    };
    if (gid < nk) {
        const int64_t row = gid / CPR;
        const int c = 4 * (int)(gid - row * CPR);
        const int bh = (int)(row / p.KS), s = (int)(row - (int64_t)bh * p.KS), b = bh / p.H, h = bh % p.H;
        const float *r0 = p.pkv + row * 2 * D, *r1 = p.pkv + ((int64_t)p.BH * p.KS + row) * 2 * D;
        const f32x4 k0 = *reinterpret_cast<const f32x4 *>(r0 + c), k1 = *reinterpret_cast<const f32x4 *>(r1 + c);
        const f32x4 v0 = *reinterpret_cast<const f32x4 *>(r0 + D + c), v1 = *reinterpret_cast<const f32x4 *>(r1 + D + c);
        store4(static_cast<T *>(p.dk) + b * p.sdk.b + h * p.sdk.h + (int64_t)s * p.sdk.t + c, (k0 + k1) * p.smscale);
        store4(static_cast<T *>(p.dv) + b * p.sdv.b + h * p.sdv.h + (int64_t)s * p.sdv.t + c, v0 + v1);
        if (c == 0) {
            const f32x2 a0 = *reinterpret_cast<const f32x2 *>(p.pks + 2 * row);
            const f32x2 a1 = *reinterpret_cast<const f32x2 *>(p.pks + 2 * ((int64_t)p.BH * p.KS + row));
            p.wsum[(int64_t)bh * p.TP + s] = a0[0] + a1[0];
            p.dpsi[(int64_t)bh * p.T + s] = -p.beta[h] * (a0[1] + a1[1]);
        }
    } else if (gid < nk + nq) {
        const int64_t row = (gid - nk) / CPR;
        const int c = 4 * (int)(gid - nk - row * CPR);
        const int bh = (int)(row / nqs), t = p.QS + (int)(row - (int64_t)bh * nqs), b = bh / p.H, h = bh % p.H;
        const int64_t row1 = (int64_t)p.BH * nqs + row;
        const f32x4 q0 = *reinterpret_cast<const f32x4 *>(p.pq + row * D + c);
        const f32x4 q1 = *reinterpret_cast<const f32x4 *>(p.pq + row1 * D + c);
        store4(static_cast<T *>(p.dq) + b * p.sdq.b + h * p.sdq.h + (int64_t)t * p.sdq.t + c, (q0 + q1) * p.smscale);
        if (c == 0) p.rsum[(int64_t)bh * p.TP + t] = p.pqr[row] + p.pqr[row1];
    } else if (gid < nk + nq + ng) {
        const int64_t gi = gid - nk - nq;
        const int bh = (int)(gi / ngk), k = (int)(gi - (int64_t)bh * ngk);
        p.dbp[(int64_t)bh * p.NK32 + k] += p.dbp[((int64_t)p.BH + bh) * p.NK32 + k];
    }
}

template <typename T, int D>
static hipError_t launch_merge_t(const BwdParams &p, hipStream_t s) {
    const int64_t n = (int64_t)p.BH * (p.KS + (p.T - p.QS)) * (D / 4) + (int64_t)p.BH * (p.KS / 32);
    hipLaunchKernelGGL((fpa_bwd_merge_kernel<T, D>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p);
    return hipGetLastError();
}

hipError_t launch_bwd_merge(const BwdParams &p, int dtype, int D, hipStream_t s) {
    if (dtype == 0) {
        switch (D) {
            case 16: return launch_merge_t<f16, 16>(p, s);
            case 32: return launch_merge_t<f16, 32>(p, s);
            case 64: return launch_merge_t<f16, 64>(p, s);
            case 128: return launch_merge_t<f16, 128>(p, s);
            case 256: return launch_merge_t<f16, 256>(p, s);
        }
    } else {
        switch (D) {
            case 16: return launch_merge_t<float, 16>(p, s);
            case 32: return launch_merge_t<float, 32>(p, s);
            case 64: return launch_merge_t<float, 64>(p, s);
            case 128: return launch_merge_t<float, 128>(p, s);
            case 256: return launch_merge_t<float, 256>(p, s);
        }
    }
    return hipErrorInvalidValue;
}

hipError_t launch_bwd_kvq(const BwdParams &p, int dtype, int D, hipStream_t s) {
    if (dtype == 0) {
        switch (D) {
            case 16: return launch_kvq_t<f16, 16>(p, s);
            case 32: return launch_kvq_t<f16, 32>(p, s);
            case 64: return launch_kvq_t<f16, 64>(p, s);
            case 128: return launch_kvq_t<f16, 128>(p, s);
            case 256: return launch_kvq_t<f16, 256>(p, s);
        }
    } else {
        switch (D) {
            case 16: return launch_kvq_t<float, 16>(p, s);
            case 32: return launch_kvq_t<float, 32>(p, s);
            case 64: return launch_kvq_t<float, 64>(p, s);
            case 128: return launch_kvq_t<float, 128>(p, s);
            case 256: return launch_kvq_t<float, 256>(p, s);
        }
    }
    return hipErrorInvalidValue;
}

}  // namespace fpa
