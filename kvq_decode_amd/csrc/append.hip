// fp16 KV write path: new K/V token rows scattered into their paged-cache slots.
//
// The page addressing is the one the reference's builder scatters with (reference.py:75-79:
// token i of sequence b lives in block block_table[b, i // block_size], slot
// i % block_size); the slot-mapping form is vLLM's reshape_and_cache (flat slot =
// block * block_size + offset, negative = padding token, not written). The write is a
// plain copy: 16-byte vector loads and stores, one workgroup per new token, both caches
// in the same pass. Nothing is read back, so the kernel is HBM-write bound with
// 2 * Hkv * D * 2 bytes per token (4 KiB at Hkv 8, D 128).
#include "kvq_internal.h"

namespace kvq {

namespace {

typedef uint32_t u4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void append_f16_kernel(const AppendParams p) {
    const int t = blockIdx.x;
    int64_t slot;
    if (p.slot_mapping) {
        slot = p.slot_mapping[t];
    } else {
        const int pos = p.seq_lens[t] - 1;  // the new token is the sequence's last
        if (pos < 0 || pos >= p.max_blocks * p.block_size) return;
        slot = (int64_t)p.bt[t * p.bt_sb + pos / p.block_size] * p.block_size +
               pos % p.block_size;
    }
    // padding tokens (slot < 0) and slots outside the pool write nothing
    if (slot < 0 || slot >= (int64_t)p.num_blocks * p.block_size) return;
    const int64_t blk = slot / p.block_size, tok = slot % p.block_size;
    const int per_head = p.head_dim / 8;  // 16-byte pieces per head row
    const int n = p.kv_heads * per_head;
    for (int i = threadIdx.x; i < 2 * n; i += blockDim.x) {
        const bool is_v = i >= n;
        const int j = is_v ? i - n : i;
        const int h = j / per_head, c = (j - h * per_head) * 8;
        const _Float16* src = (is_v ? p.v_new : p.k_new) + t * p.n_stok + h * p.n_sh + c;
        _Float16* dst = is_v ? p.v + blk * p.v_sblk + tok * p.v_stok + h * p.v_sh + c
                             : p.k + blk * p.k_sblk + tok * p.k_stok + h * p.k_sh + c;
        *(u4*)dst = *(const u4*)src;
    }
}

}  // namespace

hipError_t launch_append_f16(const AppendParams& p, hipStream_t stream) {
    hipLaunchKernelGGL(append_f16_kernel, dim3(p.tokens), dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace kvq
