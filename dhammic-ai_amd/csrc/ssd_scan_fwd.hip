// Forward chunk scan entry: dtype dispatch and the LDS size the host checks.
#include "ssd_scan_fwd_impl.h"

hipError_t launch_chunk_scan_fwd_bf16(const SsdDims& d, const SsdBufs& b, const SsdIn& in, void* y, hipStream_t s);
hipError_t launch_chunk_scan_fwd_f32(const SsdDims& d, const SsdBufs& b, const SsdIn& in, void* y, hipStream_t s);

size_t lds_chunk_scan_fwd(int dtype, const SsdDims& d) {
  return lds_scan_fwd_hs(dtype == 1 ? 2 : 4, d, fwd_heads_per_block(dtype, d));
}

hipError_t launch_chunk_scan_fwd(int dtype, const SsdDims& d, const SsdBufs& b, const SsdIn& in, void* y,
                                 hipStream_t s) {
  return dtype == 1 ? launch_chunk_scan_fwd_bf16(d, b, in, y, s) : launch_chunk_scan_fwd_f32(d, b, in, y, s);
}
