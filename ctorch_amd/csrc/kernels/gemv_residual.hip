// Projection kernels with the RESIDUAL epilogue: the GEMV (one activation row) and the matrix-core variant.
#include "kernels/gemm_tiles.h"

dlk::gemv::Kernel dlk_gemv_kernel_residual(const dlk_gemv_params& p, int mt) {
    return dlk::gemv::resolve<DLK_EPI_RESIDUAL>(p, mt);
}

dlk::gemv::Kernel dlk_gemm_kernel_residual(const dlk_gemv_params& p, int mt, int nc) {
    return dlk::gemm::resolve<DLK_EPI_RESIDUAL>(p, mt, nc);
}

dlk::gemv::Kernel dlk_gemm_reduce_residual(const dlk_gemv_params& p) {
    return dlk::gemm::resolve_reduce<DLK_EPI_RESIDUAL>(p);
}

dlk::gemv::Kernel dlk_tiles_kernel_residual(const dlk_gemv_params& p) {
    return dlk::tiles::resolve<DLK_EPI_RESIDUAL>(p);
}
