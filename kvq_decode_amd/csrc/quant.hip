// KIVI quantization kernels (bulk and on-append). Filled in below the decode path.
#include <hip/hip_runtime.h>

#include "kvq_internal.h"

namespace kvq {

hipError_t launch_quantize_cache(const QuantParams&, int, hipStream_t) {
    return hipErrorInvalidValue;
}

hipError_t launch_quantize_append(const QuantParams&, int, hipStream_t) {
    return hipErrorInvalidValue;
}

}  // namespace kvq
