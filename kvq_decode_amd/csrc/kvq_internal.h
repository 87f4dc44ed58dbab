// Internal interface between the C ABI (capi.cpp) and the HIP kernels (decode.hip,
// quant.hip). Not installed; the public boundary is include/kvq.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kvq.h"

namespace kvq {

// Kernel-side view of one decode call. Built on the host from kvq_decode_args after
// validation; passed by value as the kernel argument.
struct DecodeParams {
    const void* q;
    int64_t q_sb, q_sh;
    const void* k;
    int64_t k_sblk, k_stok, k_sh;
    const void* v;
    int64_t v_sblk, v_stok, v_sh;
    const int32_t* bt;
    int64_t bt_sb;
    const int32_t* seq_lens;
    void* out;  // fp16 output (single pass)
    int64_t o_sb, o_sh;
    float* o_part;  // split-KV workspace (stage 1)
    float* lse;
    const _Float16* k_scale;
    const _Float16* k_zero;
    const _Float16* v_scale;
    const _Float16* v_zero;
    int32_t batch, q_heads, kv_heads, group, block_size, max_blocks, num_blocks;
    int32_t cpp_shift;       // log2(block_size / 16): 16-token chunks per page
    int32_t k_group_chunks;  // 16-token chunks per K scale group (quantized formats)
    int32_t k_group_shift;   // log2(k_group_chunks)
    int32_t k_group_pages;   // pages per K scale group
    int32_t num_splits, pages_per_split;
    float scale_log2;        // softmax scale * log2(e)
    int32_t xcd_group;       // workgroup order (decode_common.h wg_coord): 0 plain, 1 grouped
    int32_t units;           // work units per kv head (decode_common.h UnitSpace); 0 = splits
    int32_t vg_shift;        // log2 of tokens per V (scale, zero) group, max(block_size, 32)
    int32_t kv_rep;          // q-head blocks per cache kv head (more than 16 q heads per kv
                             // head): the kernels' kv head v (kv_heads of them, `group` q
                             // heads each) reads the caches' kv head v / kv_rep; 1 otherwise
};

// Launches the decode kernel for the format/head_dim in `fmt`/`head_dim`. `final_out`
// selects the single-pass variant (writes p.out) over stage 1 (writes p.o_part/p.lse).
hipError_t launch_decode(const DecodeParams& p, int kv_format, int head_dim, bool final_out,
                         int waves_per_group, int pipeline, hipStream_t stream);

// Floats of LDS region 0 of the quantized decode kernels (decode_q_impl.h) with `waves`
// waves per workgroup and head dim `head_dim`: the cross-wave combine ([waves][group]
// [head_dim] accumulators + [waves][16] m and l), or the waves' staging tiles if larger
// (INT8 / FP8: a 16 head_dim-byte K tile and a 20 head_dim-byte V tile per wave; INT4: a V
// tile in 16 head_dim bytes per wave; the tiles are used before the combine).
__host__ __device__ inline int quant_lds_region0(int waves, int group, int kv_format,
                                                 int head_dim) {
    const int combine = waves * group * head_dim + 2 * waves * 16;
    const int tiles = waves * head_dim * (kv_format == KVQ_KV_INT4 ? 4 : 9);
    return combine > tiles ? combine : tiles;
}

// Quantized formats (decode_q_impl.h), head_dim 64, 128 or 256: stage 1 of the work units
// and the split / single-pass kernels. `ring` = chunks of loads in flight per wave: 1, 2 or
// 4 (head_dim 256: 1 or 2). Each head dim's kernels sit in a translation unit of their own
// (decode_q_d64.hip, decode_q.hip, decode_q_d256.hip).
hipError_t launch_decode_q_units(const DecodeParams& p, int kv_format, int head_dim, int waves,
                                 int ring, hipStream_t stream);
hipError_t launch_decode_q(const DecodeParams& p, int kv_format, int head_dim, bool final_out,
                           int waves_per_group, int ring, hipStream_t stream);
#define KVQ_DECL_QHD(D)                                                                       \
    hipError_t launch_decode_q_hd##D(const DecodeParams& p, int kv_format, bool final_out,    \
                                     int waves, int ring, hipStream_t stream);               \
    hipError_t launch_decode_q_units_hd##D(const DecodeParams& p, int kv_format, int waves,  \
                                           int ring, hipStream_t stream);
KVQ_DECL_QHD(64)
KVQ_DECL_QHD(128)
KVQ_DECL_QHD(256)
#undef KVQ_DECL_QHD

// Work units (decode_common.h UnitSpace): stage 1 over p.units units per kv head of
// `waves`-wave workgroups, and the merge of each sequence's partial rows into p.out.
// Batch at most kUnitMaxBatch.
constexpr int kUnitMaxBatch = 1024;  // a multiple of 64
hipError_t launch_decode_units(const DecodeParams& p, int kv_format, int head_dim, int waves,
                               int ring, hipStream_t stream);
hipError_t launch_merge_units(const DecodeParams& p, int head_dim, hipStream_t stream);

hipError_t launch_merge(const float* o_part, const float* lse, void* out, int64_t o_sb,
                        int64_t o_sh, int batch, int q_heads, int head_dim, int num_splits,
                        hipStream_t stream);

// Bulk quantization of fp16 paged caches into codes + scales (quant.hip).
struct QuantParams {
    const _Float16* k_src;
    const _Float16* v_src;
    int64_t s_sblk, s_stok, s_sh;
    uint8_t* k_codes;
    uint8_t* v_codes;
    int64_t k_sblk, k_stok, k_sh;
    int64_t v_sblk, v_stok, v_sh;
    _Float16* k_scale;
    _Float16* k_zero;
    _Float16* v_scale;
    _Float16* v_zero;
    const int32_t* bt;
    int64_t bt_sb;
    const int32_t* seq_lens;
    const _Float16* k_new;   // append only: [batch, kv_heads, head_dim]
    const _Float16* v_new;
    _Float16* k_resid;       // append only: [batch, kv_heads, k_group + 2, head_dim]: the
                             // open K group's rows, then their per-channel min and max
    int32_t batch, kv_heads, head_dim, block_size, max_blocks, num_blocks, k_group;
    int32_t bs_shift;        // log2(block_size) (a power of two)
    int32_t vg_shift;        // log2 of tokens per V (scale, zero) group, max(block_size, 32)
    int32_t max_groups;      // cdiv(max_blocks * block_size, k_group)
};

hipError_t launch_quantize_cache(const QuantParams& p, int kv_format, hipStream_t stream);
hipError_t launch_quantize_append(const QuantParams& p, int kv_format, hipStream_t stream);

// fp16 append (append.hip). Strides in elements. `tokens` new rows; row t goes to flat
// slot slot_mapping[t] when slot_mapping is set, else to position seq_lens[t] - 1 of
// sequence t through block_table.
struct AppendParams {
    const _Float16* k_new;
    const _Float16* v_new;
    int64_t n_stok, n_sh;
    _Float16* k;
    _Float16* v;
    int64_t k_sblk, k_stok, k_sh;
    int64_t v_sblk, v_stok, v_sh;
    const int32_t* bt;
    int64_t bt_sb;
    const int32_t* seq_lens;
    const int64_t* slot_mapping;
    int32_t tokens, kv_heads, head_dim, block_size, max_blocks, num_blocks;
};

hipError_t launch_append_f16(const AppendParams& p, hipStream_t stream);

}  // namespace kvq
