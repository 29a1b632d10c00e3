// Projection GEMV kernels with the QKV epilogue.
#include "kernels/gemv_impl.h"

dlk::gemv::Kernel dlk_gemv_kernel_qkv(const dlk_gemv_params& p, int mt) {
    return dlk::gemv::resolve<DLK_EPI_QKV>(p, mt);
}
