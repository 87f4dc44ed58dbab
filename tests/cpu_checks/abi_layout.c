/* Prints the size and every field offset of struct kvq_decode_args as the C compiler lays
 * it out from include/kvq.h, one "name offset size" line per field and a final
 * "sizeof N" line. tests/test_capi.py compares them with the ctypes mirror that every
 * Python call passes through the ABI. */
#include <stddef.h>
#include <stdio.h>

#include "kvq.h"

#define FIELD(f) printf("%s %zu %zu\n", #f, offsetof(kvq_decode_args, f), \
                        sizeof(((kvq_decode_args*)0)->f))

int main(void) {
    FIELD(q);
    FIELD(q_stride_b);
    FIELD(q_stride_h);
    FIELD(k_cache);
    FIELD(k_stride_blk);
    FIELD(k_stride_tok);
    FIELD(k_stride_head);
    FIELD(v_cache);
    FIELD(v_stride_blk);
    FIELD(v_stride_tok);
    FIELD(v_stride_head);
    FIELD(block_table);
    FIELD(bt_stride_b);
    FIELD(seq_lens);
    FIELD(out);
    FIELD(o_stride_b);
    FIELD(o_stride_h);
    FIELD(batch);
    FIELD(q_heads);
    FIELD(kv_heads);
    FIELD(head_dim);
    FIELD(block_size);
    FIELD(max_blocks);
    FIELD(num_blocks);
    FIELD(scale);
    FIELD(kv_format);
    FIELD(k_group);
    FIELD(k_scale);
    FIELD(k_zero);
    FIELD(v_scale);
    FIELD(v_zero);
    FIELD(waves_per_group);
    FIELD(pipeline);
    printf("sizeof %zu\n", sizeof(kvq_decode_args));
    return 0;
}
