// Projection GEMV kernels with the RESIDUAL epilogue.
#include "kernels/gemv_impl.h"

dlk::gemv::Kernel dlk_gemv_kernel_residual(const dlk_gemv_params& p, int mt) {
    return dlk::gemv::resolve<DLK_EPI_RESIDUAL>(p, mt);
}
