// Quantized decode kernels (decode_q_impl.h) for head_dim 128.
#include "decode_q_impl.h"

namespace kvq {

hipError_t launch_decode_q_hd128(const DecodeParams& p, int kv_format, bool final_out,
                                int waves, int ring, hipStream_t stream) {
    return launch_decode_q_for<128>(p, kv_format, final_out, waves, ring, stream);
}

hipError_t launch_decode_q_units_hd128(const DecodeParams& p, int kv_format, int waves,
                                      int ring, hipStream_t stream) {
    return launch_decode_q_units_for<128>(p, kv_format, waves, ring, stream);
}

hipError_t launch_decode_q_units(const DecodeParams& p, int kv_format, int head_dim, int waves,
                                 int ring, hipStream_t stream) {
    switch (head_dim) {
        case 64: return launch_decode_q_units_hd64(p, kv_format, waves, ring, stream);
        case 128: return launch_decode_q_units_hd128(p, kv_format, waves, ring, stream);
        case 256: return launch_decode_q_units_hd256(p, kv_format, waves, ring, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_decode_q(const DecodeParams& p, int kv_format, int head_dim, bool final_out,
                           int waves, int ring, hipStream_t stream) {
    switch (head_dim) {
        case 64: return launch_decode_q_hd64(p, kv_format, final_out, waves, ring, stream);
        case 128: return launch_decode_q_hd128(p, kv_format, final_out, waves, ring, stream);
        case 256: return launch_decode_q_hd256(p, kv_format, final_out, waves, ring, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace kvq
