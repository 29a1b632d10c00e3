// Projection kernels with the STORE epilogue: the GEMV (one activation row) and the matrix-core variant.
#include "kernels/gemm_tiles.h"

dlk::gemv::Kernel dlk_gemv_kernel_store(const dlk_gemv_params& p, int mt) {
    return dlk::gemv::resolve<DLK_EPI_STORE>(p, mt);
}

dlk::gemv::Kernel dlk_gemm_kernel_store(const dlk_gemv_params& p, int mt, int nc) {
    return dlk::gemm::resolve<DLK_EPI_STORE>(p, mt, nc);
}

dlk::gemv::Kernel dlk_gemm_reduce_store(const dlk_gemv_params& p) {
    return dlk::gemm::resolve_reduce<DLK_EPI_STORE>(p);
}

dlk::gemv::Kernel dlk_tiles_kernel_store(const dlk_gemv_params& p) {
    return dlk::tiles::resolve<DLK_EPI_STORE>(p);
}

dlk::gemv::Kernel dlk_tiles_kernel_narrow(const dlk_gemv_params& p) {
    return dlk::tiles::resolve_narrow(p);
}
