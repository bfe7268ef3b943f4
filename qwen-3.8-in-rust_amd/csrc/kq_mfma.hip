// kq_mfma.hip — the entry points of the K-quant x Q8_K matmul: grouping of matrices into launches and the
// dispatch by type pair (the kernels and their launchers are in kq_mfma.h, one source file per type pair).
#include "kq_mfma.h"

namespace aq {
namespace {

// One launch over segments [i0, i1) of at most two K-quant types.
int launch_run(const Weight *const *ws, float *const *ys, const float *const *resids, int i0, int i1, const Act &x,
               size_t ncols, hipStream_t stream) {
    int t0 = 99, t1 = 0;
    for (int i = i0; i < i1; i++) {
        const int t = ws[i]->type;
        if (t == AQ_TYPE_F32) continue;
        t0 = t < t0 ? t : t0;
        t1 = t > t1 ? t : t1;
    }
    constexpr int Q4 = AQ_TYPE_Q4_K, Q5 = AQ_TYPE_Q5_K, Q6 = AQ_TYPE_Q6_K;
    if (t0 == Q4 && t1 == Q4) return kq_run_q4q4(ws, ys, resids, i0, i1, x, ncols, stream);
    if (t0 == Q5 && t1 == Q5) return kq_run_q5q5(ws, ys, resids, i0, i1, x, ncols, stream);
    if (t0 == Q6 && t1 == Q6) return kq_run_q6q6(ws, ys, resids, i0, i1, x, ncols, stream);
    if (t0 == Q4 && t1 == Q5) return kq_run_q4q5(ws, ys, resids, i0, i1, x, ncols, stream);
    if (t0 == Q4 && t1 == Q6) return kq_run_q4q6(ws, ys, resids, i0, i1, x, ncols, stream);
    return kq_run_q5q6(ws, ys, resids, i0, i1, x, ncols, stream);
}

} // namespace

int launch_kq_group(const Weight *const *ws, float *const *ys, const float *const *resids, int n, const Act &x,
                    size_t ncols, hipStream_t stream) {
    AQ_REQUIRE(n >= 1 && ws && ys, "kq_mfma: no matrices");
    if (q8_fine()) { // Q8_0 activations: one launch per matrix (matvec.rs:282-292 `one_row` for every type)
        for (int i = 0; i < n; i++) {
            const int rc = launch_matmul(*ws[i], x, ncols, ys[i], resids ? resids[i] : nullptr, stream);
            if (rc) return rc;
        }
        return 0;
    }
    AQ_REQUIRE(ncols >= 1 && ncols <= 8, "kq_mfma: ncols must be 1..8");
    int nq = 0; // the K-quant matrices come first; F32 ones (at most two) ride in the last launch
    while (nq < n && ws[nq]->type != AQ_TYPE_F32) nq++;
    AQ_REQUIRE(nq >= 1 && n - nq <= 2, "kq_mfma: K-quant matrices first, then at most two F32 ones");
    for (int i = 0; i < n; i++) {
        AQ_REQUIRE(i < nq ? is_kquant(ws[i]->type) : ws[i]->type == AQ_TYPE_F32, "kq_mfma: matrix types");
        AQ_REQUIRE(ws[i]->nb == ws[0]->nb || ws[i]->type == AQ_TYPE_F32, "kq_mfma: grouped matrices must share K");
        AQ_REQUIRE(ws[i]->cols == x.n, "kq_mfma: activation length != weight columns");
        AQ_REQUIRE(ws[i]->rows >= 1 && ws[i]->rows <= (1u << 30), "kq_mfma: rows");
    }
    // consecutive runs of at most three K-quant matrices and two types per launch
    int i0 = 0;
    while (i0 < nq) {
        int i1 = i0 + 1, ta = ws[i0]->type, tb = ta;
        while (i1 < nq && i1 - i0 < 3) {
            const int t = ws[i1]->type;
            if (t != ta && t != tb) {
                if (ta != tb) break;
                tb = t;
            }
            i1++;
        }
        if (i1 == nq) i1 = n; // the F32 segments join the last launch
        const int rc = launch_run(ws, ys, resids, i0, i1, x, ncols, stream);
        if (rc) return rc;
        i0 = i1;
    }
    return 0;
}

int launch_kq_mfma(const Weight &w, const Act &x, size_t ncols, float *y, const float *resid, hipStream_t stream) {
    const Weight *ws[1] = {&w};
    float *ys[1] = {y};
    const float *rs[1] = {resid};
    return launch_kq_group(ws, ys, rs, 1, x, ncols, stream);
}

} // namespace aq
