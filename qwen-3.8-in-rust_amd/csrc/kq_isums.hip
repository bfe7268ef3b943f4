// kq_isums.hip — the K-quant matmul kernel (kq_mfma.h) instantiated with its integer outputs on, for the check of
// the exact lane sums and min products against the reference's integers (kdot.rs:37-140).
#include "kq_mfma.h"

namespace aq {
int kq_isums_run(const Weight &w, const Act &x, size_t ncols, float *y, int32_t *lanes, int32_t *mins,
                 hipStream_t stream) {
    switch (w.type) {
    case AQ_TYPE_Q4_K: return launch_isums_t<AQ_TYPE_Q4_K>(w, x, ncols, y, lanes, mins, stream);
    case AQ_TYPE_Q5_K: return launch_isums_t<AQ_TYPE_Q5_K>(w, x, ncols, y, lanes, mins, stream);
    case AQ_TYPE_Q6_K: return launch_isums_t<AQ_TYPE_Q6_K>(w, x, ncols, y, lanes, mins, stream);
    default: return fail(AQ_EINVAL, "kq isums: K-quant weights only");
    }
}
} // namespace aq
