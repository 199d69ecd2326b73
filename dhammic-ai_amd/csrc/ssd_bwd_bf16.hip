// bf16 instantiation of the backward column / row kernels (ssd_bwd_impl.h).
#include "ssd_bwd_impl.h"

hipError_t launch_bwd_col_bf16(const SsdDims& d, const SsdBufs& b, const SsdIn& in, const void* dy, void* dx,
                               void* dB, hipStream_t s) {
  return bwd_col_d<bf16>(d, b, in, dy, dx, dB, s);
}

hipError_t launch_bwd_row_bf16(const SsdDims& d, const SsdBufs& b, const SsdIn& in, const void* dy, void* dC,
                               hipStream_t s) {
  return bwd_row_d<bf16>(d, b, in, dy, dC, s);
}
