// Quantized decode kernels (decode_q_impl.h) for head_dim 256.
#include "decode_q_impl.h"

namespace kvq {

hipError_t launch_decode_q_hd256(const DecodeParams& p, int kv_format, bool final_out,
                                int waves, int ring, hipStream_t stream) {
    return launch_decode_q_for<256>(p, kv_format, final_out, waves, ring, stream);
}

hipError_t launch_decode_q_units_hd256(const DecodeParams& p, int kv_format, int waves,
                                      int ring, hipStream_t stream) {
    return launch_decode_q_units_for<256>(p, kv_format, waves, ring, stream);
}

}  // namespace kvq
