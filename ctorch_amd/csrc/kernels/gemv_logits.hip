// Projection GEMV kernels with the LOGITS epilogue.
#include "kernels/gemv_impl.h"

dlk::gemv::Kernel dlk_gemv_kernel_logits(const dlk_gemv_params& p, int mt) {
    return dlk::gemv::resolve<DLK_EPI_LOGITS>(p, mt);
}
