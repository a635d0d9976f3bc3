// SVDQuant W4A4, int4-g64 variant: placeholder launchers until the kernels land.
#include "common.h"
#include "kernels.h"

namespace cozyq {

hipError_t svdq_int4_quantize(const void*, bool, const float*, const void*, uint8_t*, uint16_t*,
                              void*, int, int, int, hipStream_t) {
    return hipErrorNotSupported;
}

hipError_t svdq_int4_gemm(const uint8_t*, const uint16_t*, const uint8_t*, const uint16_t*,
                          const void*, const void*, const void*, void*, bool, int, int, int, int,
                          hipStream_t) {
    return hipErrorNotSupported;
}

}  // namespace cozyq
