// Projection GEMV kernels with the SWIGLU epilogue.
#include "kernels/gemv_impl.h"

dlk::gemv::Kernel dlk_gemv_kernel_swiglu(const dlk_gemv_params& p, int mt) {
    return dlk::gemv::resolve<DLK_EPI_SWIGLU>(p, mt);
}
