// kq_mmq.hip -- small-batch (2..64 rows) K-quant products on MFMA tiles.
#include "kq_kernels.h"

namespace kq {

hipError_t launch_matmul_mfma(int kind, const void* W, int in_dim, int out_dim, int batch, const float* X,
                              float* Y, hipStream_t s) {
  (void)kind; (void)W; (void)in_dim; (void)out_dim; (void)batch; (void)X; (void)Y; (void)s;
  return hipErrorNotSupported;
}

}  // namespace kq
