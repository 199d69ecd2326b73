// bf16 instantiation of the forward chunk scan (ssd_scan_fwd_impl.h).
#include "ssd_scan_fwd_impl.h"
hipError_t launch_chunk_scan_fwd_bf16(const SsdDims& d, const SsdBufs& b, const SsdIn& in, void* y, hipStream_t s) {
  return scan_fwd_dispatch<bf16>(d, b, in, y, s);
}
