/*
 * kvq.h - C ABI of libkvq.so, the MI355X (gfx950) paged-KV GQA decode attention library.
 *
 * The reference (pawaryd/kvq-decode, package `bpt`) runs this path as three Triton kernels
 * launched from Python by `paged_decode_attention_triton` (src/bpt/triton_fp16.py:183-247).
 * Each entry point below replaces one of those launches, or the whole wrapper, and says
 * which. Signatures use plain pointers, element strides and sizes only.
 *
 * Conventions
 *  - Every function returns a kvq_status (0 = KVQ_OK, negative = error). Argument checks
 *    run on the host from the arguments alone, before any HIP call, and never read device
 *    memory, so a failed check has no side effects and needs no GPU.
 *  - Launches are asynchronous on `stream` (a hipStream_t; NULL = the null stream). No
 *    entry point synchronizes, allocates or frees device memory; the caller owns every
 *    buffer, including the split-KV workspace. Calls are re-entrant.
 *  - Strides are in elements of the tensor they describe (fp16 elements for fp16
 *    tensors, bytes for uint8 code tensors). The innermost dimension of q, out and the
 *    caches is contiguous.
 *  - Layout (vLLM style, reference src/bpt/reference.py:3-9):
 *        q            [batch, q_heads, head_dim]                 fp16
 *        k/v cache    [num_blocks, block_size, kv_heads, head_dim] fp16, or codes (below)
 *        block_table  [batch, max_blocks] int32
 *        seq_lens     [batch] int32
 *        out          [batch, q_heads, head_dim]                 fp16
 *  - Every seq_len must be >= 1 (reference asserts it, triton_fp16.py:201). The library
 *    does not read seq_lens on the host; a seq_len < 1 yields a zero output row, and a
 *    seq_len above max_blocks * block_size is clamped to it. Block-table entries are
 *    clamped to [0, num_blocks) on the device so a bad table cannot address memory
 *    outside the cache.
 */
#ifndef KVQ_H
#define KVQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* kvq_stream_t; /* the same type as hipStream_t */

typedef enum kvq_status {
    KVQ_OK = 0,
    KVQ_ERR_NULL_POINTER = -1,  /* a required pointer is NULL */
    KVQ_ERR_SHAPE = -2,         /* sizes inconsistent (e.g. q_heads % kv_heads != 0) */
    KVQ_ERR_UNSUPPORTED = -3,   /* valid for the reference, not built here (e.g. head_dim 512) */
    KVQ_ERR_ALIGNMENT = -4,     /* pointer or stride breaks the 16-byte vector-load alignment */
    KVQ_ERR_SPLITS = -5,        /* num_splits / pages_per_split inconsistent with max_blocks */
    KVQ_ERR_FORMAT = -6,        /* unknown kv_format or missing scale/zero tensors */
    KVQ_ERR_HIP = -7,           /* a HIP launch failed (hipGetLastError) */
    KVQ_ERR_SCRATCH = -8        /* the workspace exceeds the static scratch buffer */
} kvq_status;

/* KV cache storage formats. F16 is the reference's format; the quantized ones follow the
 * KIVI-style spec the reference's byte model assumes (src/bpt/roofline.py:6-9, 22-31):
 * asymmetric fp16 scale + zero, K per channel over groups of k_group tokens, V per token.
 *   INT8      codes uint8 [nb, bs, Hkv, D],     x = c * s + z, z = min, s = (max-min)/255
 *   FP8_E4M3  codes uint8 [nb, bs, Hkv, D],     OCP e4m3fn bits, x = f(c) * s + z,
 *                                               z = (max+min)/2, s = (max-min)/896
 *   INT4      codes uint8 [nb, bs, Hkv, D/2],   two codes per byte (low nibble = even
 *                                               channel), z = min, s = (max-min)/15
 *   k_scale, k_zero  fp16 [nb, Hkv, D]: group g of sequence b lives in block
 *                    block_table[b][g * k_group / block_size]
 *   v_scale, v_zero  fp16 [nb, Hkv, VG], VG = max(block_size, 32): the pairs of tokens
 *                    [j * VG, (j + 1) * VG) of sequence b live in block
 *                    block_table[b][j * VG / block_size], token t at index t % VG (with
 *                    16-token pages, a page pair's 32 pairs of one kv head fill one
 *                    128-byte line; other blocks' entries are unused)
 * Sharing: the pairs of a K or V group are written into the group's lead block (the
 * block of its first token), also for the tokens of the group's other blocks, so a lead
 * block must belong to one sequence. Two sequences that share a block that leads a
 * group but not the group's other blocks (prefix caching, beam forks; with 16-token
 * pages page 2j leads the V group of pages 2j and 2j + 1) overwrite each other's pairs:
 * copy such a block on write, or share whole groups only.
 * The quantized formats decode at head_dim D = 64, 128 or 256 (fp16: 16-256), and the
 * quantizers (kvq_quantize_cache, kvq_quantize_append) write exactly those head dims:
 * any other returns KVQ_ERR_UNSUPPORTED from both, so no cache is written that no decode
 * can read.
 * Scale and zero are stored interleaved: one fp16 [nb, Hkv, D, 2] (K) and one
 * [nb, Hkv, VG, 2] (V) tensor of (scale, zero) pairs, so that a decode loads both of a
 * token (V) or a channel (K) with one access. k_scale / v_scale point at element 0 of that
 * tensor and k_zero / v_zero one element (2 bytes) after it.                           */
typedef enum kvq_kv_format {
    KVQ_KV_F16 = 0,
    KVQ_KV_INT8 = 1,
    KVQ_KV_FP8_E4M3 = 2,
    KVQ_KV_INT4 = 3
} kvq_kv_format;

/* Version of the on-device quantized cache format above: code layout and nibble order,
 * the interleaved (scale, zero) pairs, the K group's pairs in the group's first block, the
 * quantization formulas (kvq_quantize_cache) and their rounding. A cache written under
 * one version is read correctly only by libraries reporting the same version. */
#define KVQ_CACHE_FORMAT_VERSION 2

/* KVQ_CACHE_FORMAT_VERSION of the loaded library (no reference counterpart). */
int kvq_cache_format_version(void);

/* Everything that describes one decode call's inputs and output. Mirrors the arguments of
 * paged_decode_attention_triton (triton_fp16.py:183-191) and the strides its launches pass
 * (triton_fp16.py:221-230, 237-247). */
typedef struct kvq_decode_args {
    const void* q;            /* fp16 [batch, q_heads, head_dim] */
    int64_t q_stride_b, q_stride_h;
    const void* k_cache;      /* [num_blocks, block_size, kv_heads, head_dim or head_dim/2] */
    int64_t k_stride_blk, k_stride_tok, k_stride_head;
    const void* v_cache;
    int64_t v_stride_blk, v_stride_tok, v_stride_head;
    const int32_t* block_table; /* [batch, max_blocks] */
    int64_t bt_stride_b;
    const int32_t* seq_lens;    /* [batch] */
    void* out;                /* fp16 [batch, q_heads, head_dim] */
    int64_t o_stride_b, o_stride_h;
    int32_t batch, q_heads, kv_heads, head_dim, block_size, max_blocks, num_blocks;
    float scale;              /* softmax scale; the reference defaults to 1/sqrt(head_dim) */
    int32_t kv_format;        /* kvq_kv_format */
    int32_t k_group;          /* tokens per K scale group (quantized formats; 128) */
    const void* k_scale;      /* fp16 (scale, zero) pairs [num_blocks, kv_heads, head_dim, 2] */
    const void* k_zero;       /* = k_scale + 2 bytes */
    const void* v_scale;      /* fp16 (scale, zero) pairs [num_blocks, kv_heads, VG, 2], VG =
                                 max(block_size, 32) */
    const void* v_zero;       /* = v_scale + 2 bytes */
    int32_t waves_per_group;  /* tuning: waves per (kv head, split) workgroup, one of
                                 1, 2, 4, 8, 16; 0 = the library's choice */
    int32_t pipeline;         /* tuning: depth of the load ring in 16-token chunks, 1, 2
                                 or 4 (head_dim 256: 1 or 2); deeper rings keep more
                                 loads in flight with fewer waves per SIMD; 0 = the
                                 library's choice (2) */
} kvq_decode_args;

/* Library version string, e.g. "kvq 0.1.0 gfx950". */
const char* kvq_version(void);

/* Human-readable name of a kvq_status. */
const char* kvq_status_string(int status);

/* Split-count heuristic, triton_fp16.py:175-180 (choose_num_splits):
 *   S = max(1, min(next_pow2(cdiv(target_per_cu * cu_count, batch * kv_heads)),
 *                  max_pages / max(1, min_tokens_per_split / block_size)))
 * The reference's constants are target_per_cu = 8, min_tokens_per_split = 512
 * (triton_fp16.py:166-167). Returns S >= 1, or a negative kvq_status. */
int kvq_choose_num_splits(int32_t batch, int32_t kv_heads, int32_t block_size,
                          int32_t max_pages, int32_t cu_count, int32_t target_per_cu,
                          int32_t min_tokens_per_split);

/* q-head blocks per kv head (no reference counterpart; the reference's kernel takes any
 * q_heads / kv_heads group, triton_fp16.py:196). The kernels serve at most 16 q heads per
 * kv head in one MFMA column block, so a group G > 16 is cut into k blocks of G / k heads,
 * k the smallest divisor of G with G / k <= 16, and each block runs as a kv head of its own
 * that reads the same cache head: the caches are read k times, and the kernels' grids
 * count kv_heads * k kv heads. Pass kv_heads * k as `kv_heads` (and q_heads unchanged) to
 * kvq_plan_decode and kvq_plan_units. Returns k (1 for G <= 16), or KVQ_ERR_SHAPE when q_heads is not a
 * positive multiple of kv_heads. The decode entry points return KVQ_ERR_UNSUPPORTED when
 * kv_heads * k exceeds 65535. */
int kvq_head_blocks(int32_t q_heads, int32_t kv_heads);

/* MI355X work plan used when the caller gives no split count; takes the place of the
 * heuristic above (triton_fp16.py:175-180) on this hardware. It sizes the decomposition
 * in waves, because a workgroup here holds several waves that combine through LDS:
 *   per_pair = pow2_floor(T * cu_count / (batch * kv_heads)), T = 2 s waves per CU (fp16,
 *              s = max(1, 128 / head_dim); head dims 16 and 32: 64 / head_dim), 4 (INT8,
 *              FP8) or 8 (INT4), raised to
 *              pow2_floor(cdiv(chunks, C)) (C = 512 chunks per wave for fp16; quantized
 *              256, or 64 when batch * kv_heads > cu_count, so that uneven sequence
 *              lengths still balance), capped at pow2_floor(chunks / 4);
 *              chunks = max_pages * block_size / 16
 *   waves = min(min(2 s, 4), per_pair) for fp16; clamp(per_pair / 8, 1, Wq) for quantized
 *           (Wq = 4; INT4 8),
 *   splits = per_pair / waves
 * fp16 streams fastest with about 2 waves per CU, each 2 chunks (16 KB) ahead, spread
 * over at least one workgroup per CU; more waves in flight lower the achieved bandwidth.
 * The quantized kernels run best with about 4 (INT4: 8) waves per CU, at most 8 splits per
 * (sequence, kv head) and, for large ragged batches, several waves per workgroup on small
 * partitions (all measured on MI355X for batch 1..64 and 32k..128k contexts). fp16 head
 * dims below 128 move fewer bytes per chunk through about the same per-chunk work and
 * need s times the waves (the quantized split plans measured slower with them); at 16 and
 * 32 the kv heads' rows share 128-byte lines, served from one L2 by the grouped XCD order,
 * so half of 128 / head_dim suffices.
 * A workgroup's LDS (its waves' cross-wave combine, proportional to waves * q heads per
 * kv head * head_dim, or their staging tiles) must fit 64 KB: where it would not (large
 * q-head groups at head dim 256), waves is halved and splits doubled until it does.
 * kv_heads counts the kernels' kv heads (kv_heads * kvq_head_blocks(q_heads, kv_heads))
 * and q_heads all q heads: q_heads / kv_heads is 1..16 (KVQ_ERR_SHAPE otherwise).
 * head_dim is a power of two >= 16 (KVQ_ERR_SHAPE otherwise). Writes
 * both outputs (splits before kvq_normalize_splits); returns KVQ_OK or an error. */
int kvq_plan_decode(int32_t batch, int32_t q_heads, int32_t kv_heads, int32_t block_size,
                    int32_t max_pages, int32_t kv_format, int32_t head_dim, int32_t cu_count,
                    int32_t* splits_out, int32_t* waves_out);

/* Work-unit plan, the library's default for batches of 2 to 1024 sequences (no reference
 * counterpart; it takes the place of the split heuristic, triton_fp16.py:175-180). For
 * 2 <= batch <= 1024 with batch * cdiv(max_pages * block_size, 16) < 2^31, when
 * kvq_plan_decode gives splits >= 2 or the longest context (max_pages * block_size) is at
 * least 4096 tokens:
 *   units = T * cu_count / (waves * kv_heads) (at least 1), with T waves per CU and
 *           `waves` per unit workgroup: fp16 T = 2 s, waves = min(2 s, 4); INT8 / FP8
 *           T = 4 s, waves = 4; INT4 T = 8 s, waves = min(2 s, 4)
 *           (s as in kvq_plan_decode),
 * for kvq_decode_units; otherwise units = waves = 0 (use kvq_plan_decode's split plan).
 * As in kvq_plan_decode, waves is halved (and units doubled) until a workgroup's LDS fits
 * 64 KB, and q_heads / kv_heads must be 1..16.
 * Units balance ragged batches (a static split count sizes every sequence's splits by
 * the longest one); on uniform batches the two plans run within a few percent of each
 * other on MI355X. Returns KVQ_OK or an error. */
int kvq_plan_units(int32_t batch, int32_t q_heads, int32_t kv_heads, int32_t block_size,
                   int32_t max_pages, int32_t kv_format, int32_t head_dim, int32_t cu_count,
                   int32_t* units_out, int32_t* waves_out);

/* Split normalization, triton_fp16.py:211-217: clamps num_splits to [1, max_pages], then
 * pages_per_split = cdiv(max_pages, S) and S = cdiv(max_pages, pages_per_split).
 * Writes both; returns KVQ_OK or an error. */
int kvq_normalize_splits(int32_t num_splits, int32_t max_pages, int32_t* splits_out,
                         int32_t* pages_per_split_out);

/* Stage 1 of split-KV; replaces the _split_kernel launch (triton_fp16.py:219-230, kernel
 * :83-144). Grid (kv_heads, num_splits, batch). Split s of sequence b covers pages
 * [s*pps, min((s+1)*pps, cdiv(seq_len, block_size))) and writes the normalized partial
 * output and its natural-log LSE:
 *   o_part fp32 [batch, q_heads, num_splits, head_dim], lse fp32 [batch, q_heads, num_splits]
 * An empty split writes o = 0, lse = -inf (triton_fp16.py:138-141). */
int kvq_decode_split(const kvq_decode_args* args, int32_t num_splits, int32_t pages_per_split,
                     float* o_part, float* lse, kvq_stream_t stream);

/* Stage 2; replaces the _merge_kernel launch (triton_fp16.py:231-234, kernel :147-163):
 * out[b, h] = sum_s w_s o_part[b, h, s] / sum_s w_s, w_s = exp(lse_s - max_s lse_s).
 * out is fp16 with the given strides. */
int kvq_decode_merge(const float* o_part, const float* lse, void* out, int64_t o_stride_b,
                     int64_t o_stride_h, int32_t batch, int32_t q_heads, int32_t head_dim,
                     int32_t num_splits, kvq_stream_t stream);

/* Single pass; replaces the _paged_decode_kernel launch (triton_fp16.py:237-247, kernel
 * :25-80). Grid (kv_heads, 1, batch); writes args->out directly. */
int kvq_decode_single(const kvq_decode_args* args, kvq_stream_t stream);

/* The whole op after split selection (triton_fp16.py:207-247 minus the heuristic):
 * normalizes num_splits as kvq_normalize_splits does; if the result is 1, runs the single
 * pass, otherwise stage 1 then stage 2. o_part and lse must hold
 * batch*q_heads*S*head_dim and batch*q_heads*S floats for the normalized S (NULL allowed
 * when S == 1). */
int kvq_paged_decode(const kvq_decode_args* args, int32_t num_splits, float* o_part,
                     float* lse, kvq_stream_t stream);

/* Work-unit decode (no reference counterpart: another partition of the same two stages,
 * triton_fp16.py:83-163, for ragged and large batches; every kv_format, batch at most 1024,
 * and batch * cdiv(max_blocks * block_size, 16) below 2^31 so that a kv head's chunk count
 * over the batch fits the kernels' 32-bit arithmetic; KVQ_ERR_UNSUPPORTED otherwise).
 * Per kv head, the 16-token chunks of all sequences, concatenated in batch order
 * (sequence b has cdiv(seq_lens[b], 16) chunks, N in total), are cut into
 * NU = min(units, N) equal ranges; one workgroup of args->waves_per_group waves (0 = 2;
 * 1, 2 or 4) per (kv head, range) runs the part of each sequence its range overlaps, its
 * waves sharing each part, so the work per workgroup does not depend on how the lengths
 * are spread. Partial row of (range u, sequence b) = u + b. Workspace:
 *   o_part fp32 [q_heads, units + batch, head_dim], lse fp32 [q_heads, units + batch].
 * kvq_decode_units runs stage 1 (kvq_decode_units_split) and stage 2
 * (kvq_decode_units_merge: each sequence's partial rows into args->out; an empty sequence
 * gets a zero row). The output equals kvq_paged_decode's to rounding. */
int kvq_decode_units(const kvq_decode_args* args, int32_t units, float* o_part, float* lse,
                     kvq_stream_t stream);
int kvq_decode_units_split(const kvq_decode_args* args, int32_t units, float* o_part,
                           float* lse, kvq_stream_t stream);
int kvq_decode_units_merge(const kvq_decode_args* args, int32_t units, const float* o_part,
                           const float* lse, kvq_stream_t stream);

/* Bulk KIVI quantization of fp16 paged caches (no reference counterpart: the reference's
 * quantized KV is "not started", README.md:16; its byte model is roofline.py:6-9).
 * For each sequence b and kv head, writes codes for the seq_lens[b] valid token slots of
 * both caches, K scales/zeros per channel per k_group tokens (stored in the group's first
 * block) and V scales/zeros per token. Slots past a sequence's length are not written;
 * seq_lens[b] is limited to the max_blocks * block_size slots its table row addresses.
 * A token whose block-table entry lies outside [0, num_blocks) is neither read nor
 * written (it does not enter its K group's min / max), a K group whose first page lies
 * outside the pool (where its (scale, zero) pairs would go) writes nothing, and a token
 * whose V group's first page lies outside the pool gets no V codes or pair.
 * k_src/v_src: fp16 caches with the given element strides (args->k_cache / v_cache are
 * the destination code caches, args->kv_format the target format); 16-byte aligned, with
 * strides that are multiples of 8 elements (KVQ_ERR_ALIGNMENT otherwise): each lane
 * reads 8 channels of a row at once. */
int kvq_quantize_cache(const kvq_decode_args* args, const void* k_src, const void* v_src,
                       int64_t src_stride_blk, int64_t src_stride_tok,
                       int64_t src_stride_head, kvq_stream_t stream);

/* Quantize-on-append (no reference counterpart; KIVI write path). For each sequence b,
 * the token at position p = seq_lens[b] - 1 is new: k_new/v_new fp16 [batch, kv_heads,
 * head_dim] hold it. V is quantized per token into its slot immediately. K is written
 * to the fp16 residual k_resid [batch, kv_heads, k_group + 2, head_dim] at row p % k_group;
 * rows k_group and k_group + 1 hold the per-channel min and max of the group's rows so far
 * (the append keeps them; kvq_decode_amd.quant.init_k_residual fills all of it after a
 * bulk quantization). The channels whose min or max the new row moves are re-encoded from
 * the residual rows 0..p%k_group, the others keep their codes, so the cache always equals
 * kvq_quantize_cache of all tokens so far. Appends are sequential per sequence: position
 * p follows p - 1 (or the bulk quantization and init_k_residual).
 * args->seq_lens must already count the new token. A sequence whose seq_lens[b] is below
 * 1 or above max_blocks * block_size writes nothing (codes, pairs and residual), and a
 * row whose block-table entry lies outside [0, num_blocks) is not written (a K group
 * whose first page lies outside the pool writes nothing, nor does a V row whose V group's
 * first page does), as kvq_append_kv skips such slots. k_new, v_new and k_resid are contiguous and 16-byte aligned (KVQ_ERR_ALIGNMENT
 * otherwise). */
int kvq_quantize_append(const kvq_decode_args* args, const void* k_new, const void* v_new,
                        void* k_resid, kvq_stream_t stream);

/* fp16 append, the unquantized counterpart of kvq_quantize_append. For each sequence b
 * the token at position p = seq_lens[b] - 1 is new: k_new / v_new fp16 [batch, kv_heads,
 * head_dim] (contiguous) are copied into slot p % block_size of block
 * block_table[b][p / block_size] of args->k_cache / v_cache - the page addressing the
 * reference's builder scatters with (reference.py:75-79). args->seq_lens must already
 * count the new token; args->kv_format must be KVQ_KV_F16 (q, out and the split fields
 * are not used). A position outside the block table or a block outside the pool writes
 * nothing. */
int kvq_append_kv(const kvq_decode_args* args, const void* k_new, const void* v_new,
                  kvq_stream_t stream);

/* vLLM's reshape_and_cache for fp16 caches (the reference has no write path; its layout
 * is vLLM's, reference.py:3-8). Row t of k_new / v_new (element strides new_stride_tok,
 * new_stride_head; head_dim contiguous) goes to flat slot s = slot_mapping[t] =
 * block * block_size + offset of args->k_cache / v_cache. s < 0 marks a padding token
 * and s >= num_blocks * block_size is outside the pool: neither writes anything. Uses
 * only the cache fields, kv_heads, head_dim, block_size and num_blocks of args. */
int kvq_reshape_and_cache(const kvq_decode_args* args, const void* k_new, const void* v_new,
                          int64_t new_stride_tok, int64_t new_stride_head,
                          const int64_t* slot_mapping, int32_t num_tokens,
                          kvq_stream_t stream);

/* Bytes of the static device buffer kvq_paged_decode_static takes its workspace from: 16 MiB
 * per GPU the library runs on, held until the process ends. */
#define KVQ_STATIC_SCRATCH_BYTES (16 * 1024 * 1024)

/* Allocation-free decode. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid allocation). units == 0: kvq_paged_decode(args, num_splits, ...); units > 0:
 * kvq_decode_units(args, units, ...) - same kernels, same results - with the split-KV
 * workspace (o_part, lse) taken from a static device buffer of KVQ_STATIC_SCRATCH_BYTES
 * instead of caller memory. The call allocates and frees nothing; its first call on a device
 * resolves that device's copy of the buffer (hipGetSymbolAddress). Returns KVQ_ERR_SCRATCH
 * when the workspace, (o_part + lse floats) * 4 bytes with the lse part 256-byte aligned,
 * exceeds the buffer: splits batch * q_heads * S * (head_dim + 1) floats for the normalized
 * split count S (none for a single pass), units q_heads * (units + batch) *
 * (head_dim + 1). Every call on a GPU shares that GPU's buffer: calls that overlap on one
 * GPU (concurrent streams) race. */
int kvq_paged_decode_static(const kvq_decode_args* args, int32_t num_splits, int32_t units,
                            kvq_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* KVQ_H */
