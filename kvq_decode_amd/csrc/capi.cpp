// C ABI of libkvq.so (declared in include/kvq.h): argument validation and dispatch.
// Every check here reads only the arguments - never device memory - and runs before
// any HIP call, so a rejected call has no side effects and needs no GPU.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kvq.h"
#include "kvq_internal.h"

namespace {

constexpr int kMaxGroup = 16;     // q heads per kv head served by one MFMA column block
constexpr int kLdsBudget = 64 * 1024;

bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

int ilog2(int64_t x) {
    int r = 0;
    while ((int64_t(1) << r) < x) ++r;
    return r;
}

int cdiv(int64_t a, int64_t b) { return int((a + b - 1) / b); }
// largest power of two <= x, and 1 for x < 1
int64_t pow2_floor(int64_t x) {
    int64_t p = 1;
    while (p * 2 <= x) p *= 2;
    return p;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// q-head blocks per kv head. The kernels serve at most kMaxGroup q heads per kv head (one
// MFMA column block), so a larger group G is cut into k blocks of G / k heads, k the
// smallest divisor of G with G / k <= kMaxGroup; each block runs as a kv head of its own
// that reads the same cache head, so the caches are read k times.
int head_blocks(int64_t q_heads, int64_t kv_heads) {
    const int64_t G = q_heads / kv_heads;
    int64_t k = (G + kMaxGroup - 1) / kMaxGroup;
    while (G % k) ++k;
    return int(k);
}

// kv heads of the kernels' grids: kv_heads * head_blocks
int64_t grid_heads(const kvq_decode_args* a) {
    return int64_t(a->kv_heads) * head_blocks(a->q_heads, a->kv_heads);
}

// The zero of each quantized scale pair is the fp16 right after its scale (interleaved
// (scale, zero) storage, include/kvq.h).
bool scale_pairs(const kvq_decode_args* a) {
    const uintptr_t ks = reinterpret_cast<uintptr_t>(a->k_scale);
    const uintptr_t vs = reinterpret_cast<uintptr_t>(a->v_scale);
    return reinterpret_cast<uintptr_t>(a->k_zero) == ks + 2 &&
           reinterpret_cast<uintptr_t>(a->v_zero) == vs + 2;
}

// Checks shared by every entry point that reads the caches. `need_out` is false for
// stage 1, which writes the workspace instead of args->out.
int check_decode_args(const kvq_decode_args* a, bool need_out) {
    if (!a) return KVQ_ERR_NULL_POINTER;
    if (!a->q || !a->k_cache || !a->v_cache || !a->block_table || !a->seq_lens)
        return KVQ_ERR_NULL_POINTER;
    if (need_out && !a->out) return KVQ_ERR_NULL_POINTER;
    if (a->batch < 1 || a->q_heads < 1 || a->kv_heads < 1 || a->max_blocks < 1 ||
        a->num_blocks < 1)
        return KVQ_ERR_SHAPE;
    if (a->batch > 65535 || a->kv_heads > 65535) return KVQ_ERR_UNSUPPORTED;
    if (a->q_heads % a->kv_heads != 0) return KVQ_ERR_SHAPE;
    if (grid_heads(a) > 65535) return KVQ_ERR_UNSUPPORTED;
    // The reference requires power-of-two head_dim >= 16 and block_size >= 16
    // (triton_fp16.py:197-198); anything else is a shape error here too.
    if (!is_pow2(a->head_dim) || a->head_dim < 16) return KVQ_ERR_SHAPE;
    if (!is_pow2(a->block_size) || a->block_size < 16) return KVQ_ERR_SHAPE;
    if (a->head_dim > 256) return KVQ_ERR_UNSUPPORTED;
    if (a->block_size > 4096) return KVQ_ERR_UNSUPPORTED;
    // token positions are 32-bit
    if (int64_t(a->max_blocks) * a->block_size > INT32_MAX) return KVQ_ERR_UNSUPPORTED;
    if (!(a->scale == a->scale)) return KVQ_ERR_SHAPE;  // NaN scale
    if (a->kv_format < KVQ_KV_F16 || a->kv_format > KVQ_KV_INT4) return KVQ_ERR_FORMAT;
    if (a->kv_format != KVQ_KV_F16) {
        if (!a->k_scale || !a->k_zero || !a->v_scale || !a->v_zero) return KVQ_ERR_FORMAT;
        if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256)
            return KVQ_ERR_UNSUPPORTED;
        // a K group spans at most the decode kernel's 64-page block-table window
        if (a->k_group < a->block_size || a->k_group % a->block_size != 0 ||
            !is_pow2(a->k_group) || a->k_group / a->block_size > 64)
            return KVQ_ERR_UNSUPPORTED;
        if (!scale_pairs(a)) return KVQ_ERR_FORMAT;
        if (!aligned16(a->k_scale) || !aligned16(a->v_scale)) return KVQ_ERR_ALIGNMENT;
        // The quantized kernels address a chunk from its block's 64-bit address: the pool
        // may have any size; offsets inside a block are checked below.
        if (a->k_stride_blk < 0 || a->v_stride_blk < 0 || a->k_stride_tok < 0 ||
            a->v_stride_tok < 0)
            return KVQ_ERR_UNSUPPORTED;
    }
    // Vector loads: 16-byte aligned bases and row strides that keep every row aligned.
    const int64_t vec = a->kv_format == KVQ_KV_F16 ? 8 : 16;  // elements per 16 bytes
    if (!aligned16(a->q) || !aligned16(a->k_cache) || !aligned16(a->v_cache))
        return KVQ_ERR_ALIGNMENT;
    if (need_out && !aligned16(a->out)) return KVQ_ERR_ALIGNMENT;
    if (a->q_stride_b % 8 || a->q_stride_h % 8) return KVQ_ERR_ALIGNMENT;
    if (need_out && (a->o_stride_b % 8 || a->o_stride_h % 8)) return KVQ_ERR_ALIGNMENT;
    if (a->k_stride_blk % vec || a->k_stride_tok % vec || a->k_stride_head % vec)
        return KVQ_ERR_ALIGNMENT;
    if (a->v_stride_blk % vec || a->v_stride_tok % vec || a->v_stride_head % vec)
        return KVQ_ERR_ALIGNMENT;
    // Block offsets are 32 x 32 -> 64-bit products of the block index and the block
    // stride in bytes, which must therefore stay below 2^32.
    const int64_t esz = a->kv_format == KVQ_KV_F16 ? 2 : 1;
    if (a->k_stride_blk < 0 || a->v_stride_blk < 0 ||
        a->k_stride_blk * esz >= (int64_t(1) << 32) || a->v_stride_blk * esz >= (int64_t(1) << 32))
        return KVQ_ERR_UNSUPPORTED;
    // A token's offset inside its block is a 32-bit byte offset.
    if (int64_t(a->block_size) * a->k_stride_tok * esz >= (int64_t(1) << 31) ||
        int64_t(a->block_size) * a->v_stride_tok * esz >= (int64_t(1) << 31))
        return KVQ_ERR_UNSUPPORTED;
    // Lane offsets inside a 16-token chunk are 32-bit byte offsets.
    const int64_t lim = int64_t(1) << 30;
    if (a->k_stride_tok < 0 || a->v_stride_tok < 0 || 16 * a->k_stride_tok + a->head_dim > lim ||
        16 * a->v_stride_tok + a->head_dim > lim)
        return KVQ_ERR_UNSUPPORTED;
    return KVQ_OK;
}

kvq::DecodeParams make_params(const kvq_decode_args* a) {
    kvq::DecodeParams p{};
    p.q = a->q;
    p.q_sb = a->q_stride_b;
    p.q_sh = a->q_stride_h;
    p.k = a->k_cache;
    p.k_sblk = a->k_stride_blk;
    p.k_stok = a->k_stride_tok;
    p.k_sh = a->k_stride_head;
    p.v = a->v_cache;
    p.v_sblk = a->v_stride_blk;
    p.v_stok = a->v_stride_tok;
    p.v_sh = a->v_stride_head;
    p.bt = a->block_table;
    p.bt_sb = a->bt_stride_b;
    p.seq_lens = a->seq_lens;
    p.out = a->out;
    p.o_sb = a->o_stride_b;
    p.o_sh = a->o_stride_h;
    p.k_scale = static_cast<const _Float16*>(a->k_scale);
    p.k_zero = static_cast<const _Float16*>(a->k_zero);
    p.v_scale = static_cast<const _Float16*>(a->v_scale);
    p.v_zero = static_cast<const _Float16*>(a->v_zero);
    p.batch = a->batch;
    p.q_heads = a->q_heads;
    p.kv_rep = head_blocks(a->q_heads, a->kv_heads);
    p.kv_heads = a->kv_heads * p.kv_rep;
    p.group = a->q_heads / p.kv_heads;
    p.block_size = a->block_size;
    p.max_blocks = a->max_blocks;
    p.num_blocks = a->num_blocks;
    p.cpp_shift = ilog2(a->block_size / 16);
    p.vg_shift = ilog2(a->block_size) > 5 ? ilog2(a->block_size) : 5;
    p.k_group_chunks = a->kv_format == KVQ_KV_F16 ? 0 : a->k_group / 16;
    p.k_group_shift = a->kv_format == KVQ_KV_F16 ? 0 : ilog2(a->k_group / 16);
    p.k_group_pages = a->kv_format == KVQ_KV_F16 ? 0 : a->k_group / a->block_size;
    p.scale_log2 = a->scale * 1.4426950408889634f;
    // grouped XCD order (the kv heads of a unit on one XCD, so one L2 serves a line they
    // share) for the quantized caches and for fp16 rows shorter than a 128-byte line (head
    // dims 16 and 32: the vLLM layout puts 2 or 4 heads' rows of a token in one line, which
    // the plain order fetched once per head, on different XCDs; measured at B8 x 32k,
    // 32 q / 8 kv heads: stage 1 D = 32 89.3 -> 69.0 us, D = 16 85.1 -> 50.0 us); plain for
    // fp16 rows of whole lines (measured about 1% faster there)
    p.xcd_group = a->kv_format != KVQ_KV_F16 || a->head_dim < 64;
    return p;
}

// Dynamic LDS of a decode workgroup of `waves` waves serving `group` q heads per kernel kv
// head: the cross-wave combine ([waves][group][head_dim] + [waves][16] m and l floats);
// fp16: or the waves' K staging tiles (16 rows of head_dim halves each), which the combine
// reuses; quantized: region 0 (combine or staging tiles), a K-scale slot of 4 head_dim
// bytes per wave and 32 head_dim bytes of q in k-operand order.
int64_t lds_need(int group, int head_dim, int kv_format, int waves) {
    const int64_t combine = int64_t(4) * (int64_t(waves) * group * head_dim + 32 * waves);
    if (kv_format == KVQ_KV_F16) {
        const int64_t stage = int64_t(waves) * 32 * head_dim;
        return combine > stage ? combine : stage;
    }
    return int64_t(4) * (kvq::quant_lds_region0(waves, group, kv_format, head_dim) +
                         int64_t(head_dim) * waves) +
           32 * int64_t(head_dim);
}

int64_t lds_bytes(const kvq_decode_args* a, int waves) {
    const int group = int(a->q_heads / grid_heads(a));  // q heads per kernel kv head
    return lds_need(group, a->head_dim, a->kv_format, waves);
}

// Waves per workgroup: the caller's choice if given, else as many as give each wave at
// least 8 chunks of the split (at most 8), within the LDS budget of the cross-wave
// combine. Returns 0 when the caller's choice is invalid.
int pick_waves(const kvq_decode_args* a, int pages_per_split) {
    if (a->waves_per_group != 0) {
        const int w = a->waves_per_group;
        if (w != 1 && w != 2 && w != 4 && w != 8 && w != 16) return 0;
        if (w == 16 && a->kv_format != KVQ_KV_F16) return 0;  // quantized: up to 8
        return lds_bytes(a, w) <= kLdsBudget ? w : 0;
    }
    // At most 8 waves: 16-wave workgroups need 4 waves per SIMD, which caps the kernels
    // at 128 VGPRs and makes them spill.
    const int64_t chunks = int64_t(pages_per_split) * (a->block_size / 16);
    int w = 8;
    while (w > 1 && chunks < 8 * w) w >>= 1;
    while (w > 1 && lds_bytes(a, w) > kLdsBudget) w >>= 1;
    return w;
}

// Loads in flight per wave, in 16-token chunks (the depth of the kernels' register
// ring): the caller's 1, 2 or 4 (head_dim 256: 1 or 2), else 2 (measured best for
// every format on MI355X; the chunk-pair kernel of the quantized formats keeps one pair
// in flight at depths 1 and 2, three at 4). Returns 0 when invalid.
int pick_pipeline(const kvq_decode_args* a) {
    const int r = a->pipeline;
    if (r == 0) return 2;
    if (r != 1 && r != 2 && r != 4) return 0;
    if (r == 4 && a->head_dim > 128) return 0;
    return r;
}

int hip_status(hipError_t e) { return e == hipSuccess ? KVQ_OK : KVQ_ERR_HIP; }

// Checks for the quantize entry points: args->k_cache / v_cache (codes) and the scale /
// zero tensors are the destinations; kv_format must be a quantized format.
int check_quant_args(const kvq_decode_args* a) {
    if (!a) return KVQ_ERR_NULL_POINTER;
    if (!a->k_cache || !a->v_cache || !a->block_table || !a->seq_lens) return KVQ_ERR_NULL_POINTER;
    if (a->kv_format < KVQ_KV_INT8 || a->kv_format > KVQ_KV_INT4) return KVQ_ERR_FORMAT;
    if (!a->k_scale || !a->k_zero || !a->v_scale || !a->v_zero) return KVQ_ERR_FORMAT;
    if (!scale_pairs(a)) return KVQ_ERR_FORMAT;
    if (!aligned16(a->k_scale) || !aligned16(a->v_scale)) return KVQ_ERR_ALIGNMENT;
    if (a->batch < 1 || a->kv_heads < 1 || a->max_blocks < 1 || a->num_blocks < 1)
        return KVQ_ERR_SHAPE;
    if (!is_pow2(a->block_size) || a->block_size < 16) return KVQ_ERR_SHAPE;
    if (!is_pow2(a->head_dim) || a->head_dim < 16) return KVQ_ERR_SHAPE;
    // the head dims the quantized decode reads (check_decode_args): a cache the decode
    // could not read is not written
    if (a->head_dim != 64 && a->head_dim != 128 && a->head_dim != 256) return KVQ_ERR_UNSUPPORTED;
    if (a->k_group < a->block_size || a->k_group % a->block_size != 0) return KVQ_ERR_UNSUPPORTED;
    if (a->batch > 65535 || a->kv_heads > 65535) return KVQ_ERR_UNSUPPORTED;
    // 1-D grids over (kv head, K group) and (kv head, 64-row tile); tokens are int32
    const int64_t tokens = int64_t(a->max_blocks) * a->block_size;
    if (tokens > INT32_MAX || int64_t(a->kv_heads) * ((tokens + 63) / 64) > INT32_MAX)
        return KVQ_ERR_UNSUPPORTED;
    if (a->k_stride_blk % 16 || a->k_stride_tok % 16 || a->k_stride_head % 16 ||
        a->v_stride_blk % 16 || a->v_stride_tok % 16 || a->v_stride_head % 16)
        return KVQ_ERR_ALIGNMENT;
    return KVQ_OK;
}

kvq::QuantParams make_quant_params(const kvq_decode_args* a) {
    kvq::QuantParams p{};
    p.k_codes = static_cast<uint8_t*>(const_cast<void*>(a->k_cache));
    p.v_codes = static_cast<uint8_t*>(const_cast<void*>(a->v_cache));
    p.k_sblk = a->k_stride_blk;
    p.k_stok = a->k_stride_tok;
    p.k_sh = a->k_stride_head;
    p.v_sblk = a->v_stride_blk;
    p.v_stok = a->v_stride_tok;
    p.v_sh = a->v_stride_head;
    p.k_scale = static_cast<_Float16*>(const_cast<void*>(a->k_scale));
    p.k_zero = static_cast<_Float16*>(const_cast<void*>(a->k_zero));
    p.v_scale = static_cast<_Float16*>(const_cast<void*>(a->v_scale));
    p.v_zero = static_cast<_Float16*>(const_cast<void*>(a->v_zero));
    p.bt = a->block_table;
    p.bt_sb = a->bt_stride_b;
    p.seq_lens = a->seq_lens;
    p.batch = a->batch;
    p.kv_heads = a->kv_heads;
    p.head_dim = a->head_dim;
    p.block_size = a->block_size;
    p.max_blocks = a->max_blocks;
    p.num_blocks = a->num_blocks;
    p.k_group = a->k_group;
    p.bs_shift = ilog2(a->block_size);
    p.vg_shift = p.bs_shift > 5 ? p.bs_shift : 5;
    p.max_groups = cdiv(int64_t(a->max_blocks) * a->block_size, a->k_group);
    return p;
}

// Checks for the fp16 append entry points: args->k_cache / v_cache are the destinations
// (kv_format fp16); the new rows are read with 16-byte loads.
int check_append_args(const kvq_decode_args* a, const void* k_new, const void* v_new,
                      int64_t n_stok, int64_t n_sh) {
    if (!a || !k_new || !v_new || !a->k_cache || !a->v_cache) return KVQ_ERR_NULL_POINTER;
    if (a->kv_format != KVQ_KV_F16) return KVQ_ERR_FORMAT;
    if (a->kv_heads < 1 || a->num_blocks < 1) return KVQ_ERR_SHAPE;
    if (!is_pow2(a->head_dim) || a->head_dim < 16) return KVQ_ERR_SHAPE;
    if (!is_pow2(a->block_size) || a->block_size < 16) return KVQ_ERR_SHAPE;
    if (n_stok < 0 || n_sh < 0 || a->k_stride_blk < 0 || a->k_stride_tok < 0 ||
        a->k_stride_head < 0 || a->v_stride_blk < 0 || a->v_stride_tok < 0 ||
        a->v_stride_head < 0)
        return KVQ_ERR_SHAPE;
    if (!aligned16(k_new) || !aligned16(v_new) || !aligned16(a->k_cache) ||
        !aligned16(a->v_cache))
        return KVQ_ERR_ALIGNMENT;
    if (n_stok % 8 || n_sh % 8 || a->k_stride_blk % 8 || a->k_stride_tok % 8 ||
        a->k_stride_head % 8 || a->v_stride_blk % 8 || a->v_stride_tok % 8 ||
        a->v_stride_head % 8)
        return KVQ_ERR_ALIGNMENT;
    return KVQ_OK;
}

kvq::AppendParams make_append_params(const kvq_decode_args* a, const void* k_new,
                                     const void* v_new, int64_t n_stok, int64_t n_sh) {
    kvq::AppendParams p{};
    p.k_new = static_cast<const _Float16*>(k_new);
    p.v_new = static_cast<const _Float16*>(v_new);
    p.n_stok = n_stok;
    p.n_sh = n_sh;
    p.k = static_cast<_Float16*>(const_cast<void*>(a->k_cache));
    p.v = static_cast<_Float16*>(const_cast<void*>(a->v_cache));
    p.k_sblk = a->k_stride_blk;
    p.k_stok = a->k_stride_tok;
    p.k_sh = a->k_stride_head;
    p.v_sblk = a->v_stride_blk;
    p.v_stok = a->v_stride_tok;
    p.v_sh = a->v_stride_head;
    p.bt = a->block_table;
    p.bt_sb = a->bt_stride_b;
    p.seq_lens = a->seq_lens;
    p.kv_heads = a->kv_heads;
    p.head_dim = a->head_dim;
    p.block_size = a->block_size;
    p.max_blocks = a->max_blocks;
    p.num_blocks = a->num_blocks;
    return p;
}

// The work-unit kernels count a kv head's chunks over the whole batch in 32-bit integers:
// every sequence contributes at most cdiv(max_blocks * block_size, 16) of them, and the
// batch's total must stay below 2^31 (then the unit arithmetic's products stay below 2^62).
bool units_fit(int64_t batch, int64_t max_blocks, int64_t block_size) {
    return batch * ((max_blocks * block_size + 15) / 16) <= INT32_MAX;
}

// Checks of the work-unit entry points; fills the launch parameters. The units kernels
// read every seq_len of the batch in one workgroup (batch <= kUnitMaxBatch).
int units_params(const kvq_decode_args* args, int32_t units, float* o_part, float* lse,
                 kvq::DecodeParams* p, int* waves, int* pipe) {
    int st = check_decode_args(args, true);
    if (st != KVQ_OK) return st;
    if (!o_part || !lse) return KVQ_ERR_NULL_POINTER;
    if (args->batch > kvq::kUnitMaxBatch) return KVQ_ERR_UNSUPPORTED;
    if (!units_fit(args->batch, args->max_blocks, args->block_size)) return KVQ_ERR_UNSUPPORTED;
    if (units < 1 || int64_t(units) * grid_heads(args) > INT32_MAX ||
        int64_t(units) + args->batch > INT32_MAX)
        return KVQ_ERR_SPLITS;
    *waves = args->waves_per_group == 0 ? 2 : args->waves_per_group;
    if (*waves != 1 && *waves != 2 && *waves != 4) return KVQ_ERR_UNSUPPORTED;
    *pipe = pick_pipeline(args);
    if (*pipe == 0 || lds_bytes(args, *waves) > kLdsBudget) return KVQ_ERR_UNSUPPORTED;
    *p = make_params(args);
    p->o_part = o_part;
    p->lse = lse;
    p->units = units;
    return KVQ_OK;
}

// Head dims below 128 move fewer bytes per 16-token chunk through about the same per-chunk
// work, so they need proportionally more waves in flight. Measured on MI355X (32 q / 8 kv
// heads, full steps): fp16 at head_dim 64 0.43 -> 0.72 of peak at batch 8 x 32k and 0.37
// -> 0.57 at batch 1 x 64k, at head_dim 32 0.14 -> 0.27; quantized work units +1-19% at
// head_dim 64. The quantized split plan (single sequences) measured 2-9% slower with the
// extra waves and keeps the 128 plan, and so does head_dim 256 everywhere.
// Waves-per-CU factor of the head dims below 128, whose chunks carry fewer bytes for the
// same per-chunk work: 128 / D, except that head dims 16 and 32 take 64 / D. Their rows
// share 128-byte lines between kv heads, which the grouped XCD order serves from one L2, so
// part of their bytes come from L2 and fewer waves keep HBM busy (measured at B8 x 32k,
// 32 q / 8 kv heads, stage 1: D = 32 68.3 us at 8 waves per CU, 66.3 at 4; D = 16 49.3 us
// at 16, 46.2-46.9 at 8).
int64_t head_dim_scale(int32_t head_dim) {
    return head_dim >= 128 ? 1 : head_dim >= 64 ? 128 / head_dim : 64 / head_dim;
}

}  // namespace

extern "C" {

const char* kvq_version(void) { return "kvq 0.1.0 gfx950"; }

int kvq_cache_format_version(void) { return KVQ_CACHE_FORMAT_VERSION; }

int kvq_head_blocks(int32_t q_heads, int32_t kv_heads) {
    if (q_heads < 1 || kv_heads < 1 || q_heads % kv_heads != 0) return KVQ_ERR_SHAPE;
    return head_blocks(q_heads, kv_heads);
}

const char* kvq_status_string(int status) {
    switch (status) {
        case KVQ_OK: return "ok";
        case KVQ_ERR_NULL_POINTER: return "null pointer";
        case KVQ_ERR_SHAPE: return "inconsistent shape";
        case KVQ_ERR_UNSUPPORTED: return "unsupported configuration";
        case KVQ_ERR_ALIGNMENT: return "misaligned pointer or stride";
        case KVQ_ERR_SPLITS: return "invalid split configuration";
        case KVQ_ERR_FORMAT: return "invalid kv format or missing scales";
        case KVQ_ERR_HIP: return "HIP launch error";
        case KVQ_ERR_SCRATCH: return "workspace exceeds the static scratch buffer";
        default: return "unknown status";
    }
}

int kvq_choose_num_splits(int32_t batch, int32_t kv_heads, int32_t block_size,
                          int32_t max_pages, int32_t cu_count, int32_t target_per_cu,
                          int32_t min_tokens_per_split) {
    if (batch < 1 || kv_heads < 1 || block_size < 1 || max_pages < 0 || cu_count < 1 ||
        target_per_cu < 1 || min_tokens_per_split < 0)
        return KVQ_ERR_SHAPE;
    const int64_t want = cdiv(int64_t(target_per_cu) * cu_count, int64_t(batch) * kv_heads);
    int64_t p2 = 1;
    while (p2 < want) p2 <<= 1;
    const int64_t per = min_tokens_per_split / block_size;
    int64_t cap = max_pages / (per > 1 ? per : 1);
    if (cap < 1) cap = 1;
    const int64_t s = p2 < cap ? p2 : cap;
    return int(s < 1 ? 1 : s);
}

int kvq_plan_decode(int32_t batch, int32_t q_heads, int32_t kv_heads, int32_t block_size,
                    int32_t max_pages, int32_t kv_format, int32_t head_dim, int32_t cu_count,
                    int32_t* splits_out, int32_t* waves_out) {
    if (!splits_out || !waves_out) return KVQ_ERR_NULL_POINTER;
    if (batch < 1 || kv_heads < 1 || max_pages < 1 || cu_count < 1) return KVQ_ERR_SHAPE;
    // kv_heads counts the kernels' kv heads, each serving at most kMaxGroup q heads
    if (q_heads < kv_heads || q_heads % kv_heads || q_heads / kv_heads > kMaxGroup)
        return KVQ_ERR_SHAPE;
    if (!is_pow2(block_size) || block_size < 16) return KVQ_ERR_SHAPE;
    if (!is_pow2(head_dim) || head_dim < 16) return KVQ_ERR_SHAPE;
    if (kv_format < KVQ_KV_F16 || kv_format > KVQ_KV_INT4) return KVQ_ERR_FORMAT;
    const bool quant = kv_format != KVQ_KV_F16;
    const int64_t chunks = int64_t(max_pages) * (block_size / 16);
    const int64_t pairs = int64_t(batch) * kv_heads;
    // INT4 moves half the bytes per token of INT8 / FP8 through the same per-chunk work,
    // so it needs twice the waves in flight to keep HBM busy
    const int64_t waves_per_cu =
        kv_format == KVQ_KV_INT4 ? 8 : quant ? 4 : 2 * head_dim_scale(head_dim);
    // quantized: 256-chunk partitions while (sequence, kv head) pairs alone do not fill
    // the CUs, 64-chunk partitions beyond (large batches, where ragged lengths need small
    // work items to balance)
    const int64_t chunks_per_wave = quant ? (pairs > cu_count ? 64 : 256) : 512;
    int64_t per_pair = pow2_floor(waves_per_cu * cu_count / pairs);
    const int64_t balance = pow2_floor(cdiv(chunks, chunks_per_wave));
    if (per_pair < balance) per_pair = balance;
    const int64_t cap = pow2_floor(chunks / 4);
    if (per_pair > cap) per_pair = cap;
    // fp16: up to 2 waves per workgroup (head_dim 64: 4). Quantized: one wave per 8 units
    // of per_pair, up to 4 (INT4: 8), so that long or many sequences get fewer, larger
    // splits (less partial traffic)
    int64_t wf = 2 * head_dim_scale(head_dim);
    if (wf > 4) wf = 4;
    int64_t waves = per_pair < wf ? per_pair : wf;
    if (quant) {
        const int64_t wmax = kv_format == KVQ_KV_INT4 ? 8 : 4;
        waves = per_pair / 8;
        waves = waves < 1 ? 1 : (waves > wmax ? wmax : waves);
    }
    // fewer, smaller workgroups (more splits, the same waves per pair) where a workgroup's
    // LDS would pass the budget (large q-head groups at head dim 256)
    while (waves > 1 && lds_need(q_heads / kv_heads, head_dim, kv_format, int(waves)) > kLdsBudget)
        waves >>= 1;
    *waves_out = int32_t(waves);
    *splits_out = int32_t(per_pair / waves);
    return KVQ_OK;
}

int kvq_plan_units(int32_t batch, int32_t q_heads, int32_t kv_heads, int32_t block_size,
                   int32_t max_pages, int32_t kv_format, int32_t head_dim, int32_t cu_count,
                   int32_t* units_out, int32_t* waves_out) {
    if (!units_out || !waves_out) return KVQ_ERR_NULL_POINTER;
    int32_t splits = 0, split_waves = 0;
    const int st = kvq_plan_decode(batch, q_heads, kv_heads, block_size, max_pages, kv_format,
                                   head_dim, cu_count, &splits, &split_waves);
    if (st != KVQ_OK) return st;
    *units_out = 0;
    *waves_out = 0;
    // A single sequence cannot be ragged. Where the split plan runs one pass, units pay a
    // merge and per-sequence segment starts, which only contexts of 4096 tokens or more
    // amortize (measured on MI355X: fp16 B64 at 1k tokens +17%, at 8k +3% uniform and
    // -26% ragged)
    if (batch < 2 || batch > kvq::kUnitMaxBatch) return KVQ_OK;
    if (!units_fit(batch, max_pages, block_size)) return KVQ_OK;
    if (splits < 2 && int64_t(max_pages) * block_size < 4096) return KVQ_OK;
    // Waves per CU and per unit workgroup, measured on MI355X: fp16 2 in workgroups of 2;
    // INT8 / FP8 4 in workgroups of 4; INT4 (half the bytes of a chunk for about the
    // same per-chunk work) 8 in workgroups of 2. Below head_dim 128 the waves per CU grow
    // by 128 / head_dim and the fp16 / INT4 workgroups to up to 4 waves (head_dim 64: fp16
    // 4 per CU in workgroups of 4, INT4 16 in workgroups of 4)
    const bool int4 = kv_format == KVQ_KV_INT4;
    const int64_t scale = head_dim_scale(head_dim);
    const int64_t waves_per_cu = (kv_format == KVQ_KV_F16 ? 2 : int4 ? 8 : 4) * scale;
    int64_t waves = kv_format == KVQ_KV_F16 || int4 ? 2 * scale : 4;
    if (waves > 4) waves = 4;
    // smaller unit workgroups, more units, where the LDS would pass the budget
    while (waves > 1 && lds_need(q_heads / kv_heads, head_dim, kv_format, int(waves)) > kLdsBudget)
        waves >>= 1;
    const int64_t units = waves_per_cu * cu_count / (waves * int64_t(kv_heads));
    *units_out = int32_t(units < 1 ? 1 : units);
    *waves_out = int32_t(waves);
    return KVQ_OK;
}

int kvq_normalize_splits(int32_t num_splits, int32_t max_pages, int32_t* splits_out,
                         int32_t* pages_per_split_out) {
    if (!splits_out || !pages_per_split_out) return KVQ_ERR_NULL_POINTER;
    if (max_pages < 1) return KVQ_ERR_SHAPE;
    int s = num_splits < 1 ? 1 : (num_splits > max_pages ? max_pages : num_splits);
    int pps = max_pages;
    if (s > 1) {
        pps = cdiv(max_pages, s);
        s = cdiv(max_pages, pps);
    }
    *splits_out = s;
    *pages_per_split_out = pps;
    return KVQ_OK;
}

int kvq_decode_split(const kvq_decode_args* args, int32_t num_splits, int32_t pages_per_split,
                     float* o_part, float* lse, kvq_stream_t stream) {
    int st = check_decode_args(args, false);
    if (st != KVQ_OK) return st;
    if (!o_part || !lse) return KVQ_ERR_NULL_POINTER;
    if (num_splits < 1 || pages_per_split < 1 || num_splits > 65535) return KVQ_ERR_SPLITS;
    // the 1-D decode grid: kv_heads * (splits * batch rounded up to a multiple of 8)
    if ((int64_t(num_splits) * args->batch + 7) / 8 * 8 * grid_heads(args) > INT32_MAX)
        return KVQ_ERR_UNSUPPORTED;
    if (int64_t(num_splits) * pages_per_split < args->max_blocks) return KVQ_ERR_SPLITS;
    const int waves = pick_waves(args, pages_per_split);
    const int pipe = pick_pipeline(args);
    if (waves == 0 || pipe == 0) return KVQ_ERR_UNSUPPORTED;
    kvq::DecodeParams p = make_params(args);
    p.o_part = o_part;
    p.lse = lse;
    p.num_splits = num_splits;
    p.pages_per_split = pages_per_split;
    return hip_status(kvq::launch_decode(p, args->kv_format, args->head_dim, false, waves, pipe,
                                         reinterpret_cast<hipStream_t>(stream)));
}

int kvq_decode_merge(const float* o_part, const float* lse, void* out, int64_t o_stride_b,
                     int64_t o_stride_h, int32_t batch, int32_t q_heads, int32_t head_dim,
                     int32_t num_splits, kvq_stream_t stream) {
    if (!o_part || !lse || !out) return KVQ_ERR_NULL_POINTER;
    if (batch < 1 || q_heads < 1 || num_splits < 1) return KVQ_ERR_SHAPE;
    if (batch > 65535) return KVQ_ERR_UNSUPPORTED;
    if (!is_pow2(head_dim) || head_dim < 16) return KVQ_ERR_SHAPE;
    if (head_dim > 256) return KVQ_ERR_UNSUPPORTED;
    return hip_status(kvq::launch_merge(o_part, lse, out, o_stride_b, o_stride_h, batch, q_heads,
                                        head_dim, num_splits,
                                        reinterpret_cast<hipStream_t>(stream)));
}

int kvq_decode_single(const kvq_decode_args* args, kvq_stream_t stream) {
    int st = check_decode_args(args, true);
    if (st != KVQ_OK) return st;
    if ((int64_t(args->batch) + 7) / 8 * 8 * grid_heads(args) > INT32_MAX) return KVQ_ERR_UNSUPPORTED;
    const int waves = pick_waves(args, args->max_blocks);
    const int pipe = pick_pipeline(args);
    if (waves == 0 || pipe == 0) return KVQ_ERR_UNSUPPORTED;
    kvq::DecodeParams p = make_params(args);
    p.num_splits = 1;
    p.pages_per_split = args->max_blocks;
    return hip_status(kvq::launch_decode(p, args->kv_format, args->head_dim, true, waves, pipe,
                                         reinterpret_cast<hipStream_t>(stream)));
}

int kvq_paged_decode(const kvq_decode_args* args, int32_t num_splits, float* o_part, float* lse,
                     kvq_stream_t stream) {
    int st = check_decode_args(args, true);
    if (st != KVQ_OK) return st;
    int32_t s = 1, pps = 1;
    st = kvq_normalize_splits(num_splits, args->max_blocks, &s, &pps);
    if (st != KVQ_OK) return st;
    if (s == 1) return kvq_decode_single(args, stream);
    st = kvq_decode_split(args, s, pps, o_part, lse, stream);
    if (st != KVQ_OK) return st;
    return kvq_decode_merge(o_part, lse, args->out, args->o_stride_b, args->o_stride_h,
                            args->batch, args->q_heads, args->head_dim, s, stream);
}

int kvq_decode_units_split(const kvq_decode_args* args, int32_t units, float* o_part,
                           float* lse, kvq_stream_t stream) {
    kvq::DecodeParams p;
    int waves = 0, pipe = 0;
    const int st = units_params(args, units, o_part, lse, &p, &waves, &pipe);
    if (st != KVQ_OK) return st;
    return hip_status(kvq::launch_decode_units(p, args->kv_format, args->head_dim, waves, pipe,
                                               reinterpret_cast<hipStream_t>(stream)));
}

int kvq_decode_units_merge(const kvq_decode_args* args, int32_t units, const float* o_part,
                           const float* lse, kvq_stream_t stream) {
    kvq::DecodeParams p;
    int waves = 0, pipe = 0;
    const int st = units_params(args, units, const_cast<float*>(o_part), const_cast<float*>(lse),
                                &p, &waves, &pipe);
    if (st != KVQ_OK) return st;
    return hip_status(kvq::launch_merge_units(p, args->head_dim,
                                              reinterpret_cast<hipStream_t>(stream)));
}

int kvq_decode_units(const kvq_decode_args* args, int32_t units, float* o_part, float* lse,
                     kvq_stream_t stream) {
    const int st = kvq_decode_units_split(args, units, o_part, lse, stream);
    if (st != KVQ_OK) return st;
    return kvq_decode_units_merge(args, units, o_part, lse, stream);
}

int kvq_quantize_cache(const kvq_decode_args* args, const void* k_src, const void* v_src,
                       int64_t src_stride_blk, int64_t src_stride_tok, int64_t src_stride_head,
                       kvq_stream_t stream) {
    int st = check_quant_args(args);
    if (st != KVQ_OK) return st;
    if (!k_src || !v_src) return KVQ_ERR_NULL_POINTER;
    if (src_stride_blk < 0 || src_stride_tok < 0 || src_stride_head < 0) return KVQ_ERR_SHAPE;
    // the quantizers read 8 channels (16 bytes) per lane
    if (!aligned16(k_src) || !aligned16(v_src) || src_stride_blk % 8 || src_stride_tok % 8 ||
        src_stride_head % 8)
        return KVQ_ERR_ALIGNMENT;
    kvq::QuantParams p = make_quant_params(args);
    p.k_src = static_cast<const _Float16*>(k_src);
    p.v_src = static_cast<const _Float16*>(v_src);
    p.s_sblk = src_stride_blk;
    p.s_stok = src_stride_tok;
    p.s_sh = src_stride_head;
    return hip_status(kvq::launch_quantize_cache(p, args->kv_format,
                                                 reinterpret_cast<hipStream_t>(stream)));
}

int kvq_quantize_append(const kvq_decode_args* args, const void* k_new, const void* v_new,
                        void* k_resid, kvq_stream_t stream) {
    int st = check_quant_args(args);
    if (st != KVQ_OK) return st;
    if (!k_new || !v_new || !k_resid) return KVQ_ERR_NULL_POINTER;
    if (!aligned16(k_new) || !aligned16(v_new) || !aligned16(k_resid)) return KVQ_ERR_ALIGNMENT;
    kvq::QuantParams p = make_quant_params(args);
    p.k_new = static_cast<const _Float16*>(k_new);
    p.v_new = static_cast<const _Float16*>(v_new);
    p.k_resid = static_cast<_Float16*>(k_resid);
    return hip_status(kvq::launch_quantize_append(p, args->kv_format,
                                                  reinterpret_cast<hipStream_t>(stream)));
}

int kvq_append_kv(const kvq_decode_args* args, const void* k_new, const void* v_new,
                  kvq_stream_t stream) {
    if (!args) return KVQ_ERR_NULL_POINTER;
    const int64_t row = int64_t(args->kv_heads) * args->head_dim;
    int st = check_append_args(args, k_new, v_new, row, args->head_dim);
    if (st != KVQ_OK) return st;
    if (!args->block_table || !args->seq_lens) return KVQ_ERR_NULL_POINTER;
    if (args->batch < 1 || args->max_blocks < 1 || args->bt_stride_b < args->max_blocks)
        return KVQ_ERR_SHAPE;
    if (args->batch > INT32_MAX / 2) return KVQ_ERR_UNSUPPORTED;
    kvq::AppendParams p = make_append_params(args, k_new, v_new, row, args->head_dim);
    p.tokens = args->batch;
    return hip_status(kvq::launch_append_f16(p, reinterpret_cast<hipStream_t>(stream)));
}

int kvq_reshape_and_cache(const kvq_decode_args* args, const void* k_new, const void* v_new,
                          int64_t new_stride_tok, int64_t new_stride_head,
                          const int64_t* slot_mapping, int32_t num_tokens,
                          kvq_stream_t stream) {
    int st = check_append_args(args, k_new, v_new, new_stride_tok, new_stride_head);
    if (st != KVQ_OK) return st;
    if (!slot_mapping) return KVQ_ERR_NULL_POINTER;
    if (num_tokens < 0) return KVQ_ERR_SHAPE;
    if (num_tokens == 0) return KVQ_OK;
    kvq::AppendParams p = make_append_params(args, k_new, v_new, new_stride_tok,
                                             new_stride_head);
    p.slot_mapping = slot_mapping;
    p.tokens = num_tokens;
    return hip_status(kvq::launch_append_f16(p, reinterpret_cast<hipStream_t>(stream)));
}

}  // extern "C"
