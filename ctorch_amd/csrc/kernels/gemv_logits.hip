// Projection kernels with the LOGITS epilogue: the GEMV (one activation row) and the matrix-core variant.
#include "kernels/gemm_rows.h"

dlk::gemv::Kernel dlk_gemv_kernel_logits(const dlk_gemv_params& p, int mt) {
    return dlk::gemv::resolve<DLK_EPI_LOGITS>(p, mt);
}

dlk::gemv::Kernel dlk_gemm_kernel_logits(const dlk_gemv_params& p, int mt, int nc) {
    return dlk::gemm::resolve<DLK_EPI_LOGITS>(p, mt, nc);
}

dlk::gemv::Kernel dlk_gemm_reduce_logits(const dlk_gemv_params& p) {
    return dlk::gemm::resolve_reduce<DLK_EPI_LOGITS>(p);
}
