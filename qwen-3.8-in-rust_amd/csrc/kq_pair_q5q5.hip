// kq_pair_q5q5.hip — the K-quant matmul kernels for weight types Q5_K and Q5_K (kq_mfma.h).
#include "kq_mfma.h"

namespace aq {
int kq_run_q5q5(const Weight *const *ws, float *const *ys, const float *const *resids, int i0, int i1, const Act &x,
               size_t ncols, hipStream_t stream) {
    return launch_run_t<AQ_TYPE_Q5_K, AQ_TYPE_Q5_K>(ws, ys, resids, i0, i1, x, ncols, stream);
}
} // namespace aq
