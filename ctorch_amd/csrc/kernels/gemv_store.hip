// Projection GEMV kernels with the STORE epilogue.
#include "kernels/gemv_impl.h"

dlk::gemv::Kernel dlk_gemv_kernel_store(const dlk_gemv_params& p, int mt) {
    return dlk::gemv::resolve<DLK_EPI_STORE>(p, mt);
}
