// Allocation-free decode: kvq_paged_decode_static (include/kvq.h).
//
// The split-KV and work-unit paths need a float workspace for the partial outputs and
// their LSEs (o_part, lse). kvq_paged_decode and kvq_decode_units take it from the
// caller; this entry point takes it from `scratch`, a file-scope device array of
// KVQ_STATIC_SCRATCH_BYTES that every GPU the library runs on holds until the process
// ends, so the call allocates nothing: for code under HIP graph capture, tight serving
// loops and harnesses that forbid allocation.
//
// In host code `scratch` names a host-side stand-in, not device memory. The device
// address of each GPU's copy comes from hipGetSymbolAddress, called once per device with
// that device current (the first call on the device), and is the only address host code
// hands to kernels.
//
// Contents persist between calls, and every call on a GPU shares that GPU's array: calls
// that overlap on one GPU (concurrent streams) race. Nothing needs clearing first - stage 1
// writes every partial row the merge reads (an empty split writes (0, -inf); a sequence's
// work-unit rows are written by the units that cover it).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "kvq.h"

namespace {

constexpr int64_t kScratchFloats = KVQ_STATIC_SCRATCH_BYTES / 4;
constexpr int kMaxDevices = 64;
constexpr int64_t kAlignFloats = 64;  // the lse part starts 256-byte aligned

__device__ __align__(256) float scratch[kScratchFloats];

std::mutex g_mutex;
float* g_ptr[kMaxDevices] = {};  // device address of `scratch` per device, once resolved

// The current device's address of `scratch`, resolved on the first call on that device.
int scratch_ptr(float** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return KVQ_ERR_HIP;
    std::lock_guard<std::mutex> lock(g_mutex);
    if (!g_ptr[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
            (void)hipGetLastError();  // clear the sticky error for the caller's next call
            return KVQ_ERR_HIP;
        }
        g_ptr[dev] = static_cast<float*>(p);
    }
    *out = g_ptr[dev];
    return KVQ_OK;
}

int64_t round_up(int64_t x) { return (x + kAlignFloats - 1) / kAlignFloats * kAlignFloats; }

}  // namespace

extern "C" int kvq_paged_decode_static(const kvq_decode_args* args, int32_t num_splits,
                                       int32_t units, kvq_stream_t stream) {
    if (!args) return KVQ_ERR_NULL_POINTER;
    if (units < 0) return KVQ_ERR_SPLITS;
    if (args->batch < 1 || args->q_heads < 1 || args->head_dim < 1 || args->max_blocks < 1)
        return KVQ_ERR_SHAPE;
    // the workspace of the partition the call runs, in floats
    int64_t rows = 0;
    if (units > 0) {
        rows = int64_t(args->q_heads) * (int64_t(units) + args->batch);
    } else {
        int32_t s = 1, pps = 1;
        const int st = kvq_normalize_splits(num_splits, args->max_blocks, &s, &pps);
        if (st != KVQ_OK) return st;
        if (s > 1) rows = int64_t(args->batch) * args->q_heads * s;
    }
    const int64_t o_floats = round_up(rows * args->head_dim);
    if (o_floats + rows > kScratchFloats) return KVQ_ERR_SCRATCH;
    float* base = nullptr;
    if (rows > 0) {
        const int st = scratch_ptr(&base);
        if (st != KVQ_OK) return st;
    }
    float* o_part = base;
    float* lse = base ? base + o_floats : nullptr;
    return units > 0 ? kvq_decode_units(args, units, o_part, lse, stream)
                     : kvq_paged_decode(args, num_splits, o_part, lse, stream);
}
