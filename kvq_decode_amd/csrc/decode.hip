// Paged-KV GQA decode attention for gfx950 (MI355X): split-KV stage 1, single pass and
// the LSE merge (stage 2).
//
// Replaces the reference's Triton kernels _paged_decode_kernel, _split_kernel and
// _merge_kernel (pawaryd/kvq-decode src/bpt/triton_fp16.py:25-80, 83-144, 147-163).
// Same math: per (sequence, kv head) an online softmax over the sequence's pages with all
// `group` query heads of the kv head served from one K/V read; split s covers pages
// [s*pps, min((s+1)*pps, cdiv(len, bs))) and stores the normalized partial plus its LSE;
// the merge weighs partials by exp(lse - max lse).
//
// Work decomposition (gfx950, wave64, MFMA):
//   workgroup = (kv head, split, sequence), W waves; the split's 16-token chunks are cut
//   into W contiguous runs, one per wave; waves combine their (m, l, acc) through LDS.
//   Per chunk and wave:
//     S^T[16 tok x 16 heads] = K[16 tok x D] . Q^T[D x 16 heads]    D/32 x mfma 16x16x32 f16
//         A = K: lane (tok = l%16, g = l/16) holds K[tok][32*st + 8*g + 0..7]. K is loaded
//         in whole rows (each 16-byte load instruction covers 1 KB = 512/D full token
//         rows, every 128-byte line in one instruction) and reaches the A layout through
//         a per-wave XOR-swizzled LDS tile (ds_write_b128 / ds_read_b128, conflict-free).
//         Loading the A layout directly (16 rows x 64 B per instruction) streams about
//         11% slower on MI355X with nt loads (measured);
//         B = Q^T: the same k-mapping, heads >= group are zero padding.
//     online softmax on the C layout: lane holds S^T[4g + r][head l%16], r = 0..3;
//     O^T[D x 16 heads] += V^T[D x 16 tok] . P^T[16 tok x 16 heads]  D/16 x mfma 16x16x16
//         B = P^T is exactly the QK C layout (no data movement);
//         A = V^T: lane (i = l%16, g) needs V[4g + r][d] for one d per tile - it loads the
//         D/16 contiguous halves V[4g + r][(D/16)*i ...] of 4 token rows (16 lanes cover one
//         full 256-byte row) and transposes them in registers; tile t then holds
//         d = (D/16)*i + t, so the accumulator lane (head l%16, g) ends with
//         O[head][(D/16)*(4g + r) + t].
//   The running max is lazy (see kLazyMax), so the common chunk has no cross-lane
//   reduction at all; a max update uses two v_permlane swaps.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "decode_common.h"

namespace kvq {

// One 16-token chunk of one kv head, fp16 cache, as held by one lane. K in row layout:
// load i holds K[RPL*i + l/PC][8*(l%PC) .. +8] (PC = D/8 16-byte pieces per row, RPL =
// 64/PC rows per load); V as the PV product's A operand needs it (see the file header).
// Head dim 16 (the reference's smallest) is the exception: one 8-byte load per lane
// gives the 16x16x16 QK product's A operand directly (lane (i16, g): row i16, halves
// 4g .. 4g + 3), held in the low half of k[0].
template <int D>
struct ChunkF16 {
    static constexpr int NST = D / 32;   // K loads per chunk = k-steps of the QK product
    static constexpr int KN = D >= 32 ? NST : 1;
    static constexpr int DV = D / 16;
    static constexpr int PC = D / 8;     // 16-byte pieces per K row
    static constexpr int RPL = 64 / PC;  // K rows per load instruction
    // a lane's D/16 halves of a V row (D = 16: the one half in element 0 of a pair)
    typedef typename HalfVec<(DV > 1 ? DV : 2)>::type vrow;
    h8 k[KN];
    vrow v[4];
};

// Per-lane byte offsets of a chunk's loads from the chunk's first row (the page base
// and slot are wave-uniform): K load i row min(RPL*i + l/PC, last), piece l%PC; V rows
// min(4g + r, last), halves [(D/16)(l%16), +D/16). `last` = valid tokens - 1 of the
// chunk: rows past the sequence are redirected to its last valid row, so unused page
// slots (whatever they hold) are never read; their scores are masked to -inf in
// chunk_f16.
template <int D>
struct F16LaneOff {
    uint32_t k[ChunkF16<D>::KN], v[4];
};

template <int D>
__device__ __forceinline__ F16LaneOff<D> f16_lane_offsets(const DecodeParams& p, int i16, int g,
                                                          int last) {
    typedef ChunkF16<D> C;
    const int lane = __lane_id();
    F16LaneOff<D> o;
    if constexpr (D == 16) {
        o.k[0] = (uint32_t)(min(i16, last) * (int)p.k_stok + 4 * g) * 2u;
    } else {
#pragma unroll
        for (int i = 0; i < C::NST; ++i)
            o.k[i] = (uint32_t)(min(C::RPL * i + lane / C::PC, last) * (int)p.k_stok +
                                8 * (lane % C::PC)) * 2u;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
        o.v[r] = (uint32_t)(min(4 * g + r, last) * (int)p.v_stok + C::DV * i16) * 2u;
    return o;
}

// Cache policy of the chunk loads: NT, the streaming hint (buffer_load ... nt). Every
// byte of the cache is read once per step; measured on MI355X, nt streaming reads run
// about 10% faster than default-policy ones.
constexpr int kNT = 2;

// D/16 consecutive halves (2, 4, 8, 16 or 32 bytes) at byte offset `off` of a page (head dim
// 16: the one half in element 0 of a pair).
template <int DV>
__device__ __forceinline__ typename HalfVec<(DV > 1 ? DV : 2)>::type load_vrow(
    __amdgpu_buffer_rsrc_t r, uint32_t off) {
    typedef typename HalfVec<(DV > 1 ? DV : 2)>::type vrow;
    if constexpr (DV == 1) {
        const uint32_t x = __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, kNT);
        return __builtin_bit_cast(vrow, x);
    } else if constexpr (DV == 2) {
        return __builtin_bit_cast(vrow, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kNT));
    } else if constexpr (DV == 4) {
        return __builtin_bit_cast(vrow, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kNT));
    } else if constexpr (DV == 8) {
        return __builtin_bit_cast(vrow, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kNT));
    } else {
        typedef uint32_t u8v __attribute__((ext_vector_type(8)));
        const auto a = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kNT);
        const auto b = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16, 0, kNT);
        const u8v x = __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
        return __builtin_bit_cast(vrow, x);
    }
}

// Loads chunk c (16 tokens of the caches' kv head kvh) from physical block `phys` through
// buffer resources at the chunk's first row (64-bit scalar address math once per chunk,
// 32-bit lane offsets).
template <int D>
__device__ __forceinline__ void load_chunk_f16(const DecodeParams& p, int kvh, int c,
                                               const F16LaneOff<D>& lo, int phys,
                                               ChunkF16<D>& ch) {
    constexpr int DV = D / 16;
    const int slot = (c & ((1 << p.cpp_shift) - 1)) << 4;
    const char* kb = (const char*)p.k + block_offset(phys, 2 * p.k_sblk) +
                     2 * ((int64_t)slot * p.k_stok + (int64_t)kvh * p.k_sh);
    const char* vb = (const char*)p.v + block_offset(phys, 2 * p.v_sblk) +
                     2 * ((int64_t)slot * p.v_stok + (int64_t)kvh * p.v_sh);
    const auto rk = page_rsrc(kb), rv = page_rsrc(vb);
    if constexpr (D == 16) {
        const u2 x = __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(rk, lo.k[0], 0, kNT));
        const u4v w = {x[0], x[1], 0u, 0u};
        ch.k[0] = __builtin_bit_cast(h8, w);
    }
#pragma unroll
    for (int st = 0; st < D / 32; ++st)
        ch.k[st] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(rk, lo.k[st], 0,
                                                                                kNT));
#pragma unroll
    for (int r = 0; r < 4; ++r) ch.v[r] = load_vrow<DV>(rv, lo.v[r]);
}

// The wave's K staging tile: 16 rows of D halves, 16-byte piece j of row r stored at
// slot j ^ (r & (PC - 1)). Both the row-layout writes (16 lanes = 16 pieces of one row
// for D = 128) and the A-layout reads (16 lanes = 16 rows, one piece) then touch 16
// distinct slots modulo 256 bytes: no LDS bank conflicts at D = 128 and 256.
template <int D>
__device__ __forceinline__ uint32_t kstage_off(int row, int piece) {
    constexpr int PC = D / 8;
    return (uint32_t)(row * 2 * D + 16 * (piece ^ (row & (PC - 1))));
}

// The PV product's A operand of tile t from a lane's 4 token rows (its D/16 halves of each):
// {v[0][t], v[1][t], v[2][t], v[3][t]}. With 2-half rows (head dim 32) the halves are
// picked by v_perm, two instructions; element-wise, the compiler assembled them through
// scratch memory.
template <int D>
__device__ __forceinline__ h4 pv_rows(const typename ChunkF16<D>::vrow* v, int t) {
    if constexpr (ChunkF16<D>::DV == 2) {
        const uint32_t sel = t ? 0x07060302u : 0x05040100u;
        const u2 w = {__builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, v[1]),
                                            __builtin_bit_cast(uint32_t, v[0]), sel),
                      __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, v[3]),
                                            __builtin_bit_cast(uint32_t, v[2]), sel)};
        return __builtin_bit_cast(h4, w);
    } else {
        h4 a;
#pragma unroll
        for (int r = 0; r < 4; ++r) a[r] = v[r][t];
        return a;
    }
}

// Two lanes' worth of rows for a 16x16x32 product: chunk a's in k-slots 0-3, b's in 4-7.
template <int D>
__device__ __forceinline__ h8 pv_rows2(const ChunkF16<D>& a, const ChunkF16<D>& b, int t) {
    return __builtin_shufflevector(pv_rows<D>(a.v, t), pv_rows<D>(b.v, t), 0, 1, 2, 3, 4, 5, 6, 7);
}

// One chunk: QK^T, softmax update, PV. MASK handles the sequence's partial last chunk.
// `kst` is the wave's K staging tile in LDS (32 * D bytes).
template <int D, bool MASK>
__device__ __forceinline__ void chunk_f16(const ChunkF16<D>& ch, const h8* qop, float sl2,
                                          int valid, int g, char* kst, SoftmaxState<D>& st) {
    typedef ChunkF16<D> C;
    constexpr int NST = C::NST;
    constexpr int DV = C::DV;
    typedef typename ChunkF16<D>::vrow vrow;
    const int lane = __lane_id();
    f4 s = (f4)0.f;
    if constexpr (D == 16) {  // the loaded halves are the A operand; q in qop[0]'s low half
        const h4 kop = {ch.k[0][0], ch.k[0][1], ch.k[0][2], ch.k[0][3]};
        const h4 qo = {qop[0][0], qop[0][1], qop[0][2], qop[0][3]};
        s = __builtin_amdgcn_mfma_f32_16x16x16f16(kop, qo, s, 0, 0, 0);
    } else {
#pragma unroll
        for (int i = 0; i < NST; ++i)
            *(h8*)(kst + kstage_off<D>(C::RPL * i + lane / C::PC, lane % C::PC)) = ch.k[i];
        h8 kop[NST];
#pragma unroll
        for (int k = 0; k < NST; ++k)
            kop[k] = *(const h8*)(kst + kstage_off<D>(lane & 15, 4 * k + g));
#pragma unroll
        for (int k = 0; k < NST; ++k)
            s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop[k], qop[k], s, 0, 0, 0);
    }
    float s2[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) s2[r] = s[r] * sl2;
    if (MASK) {
        // Tokens past seq_len (their rows were loaded from the last valid token) get
        // score -inf, hence p = 0.
#pragma unroll
        for (int r = 0; r < 4; ++r) s2[r] = 4 * g + r < valid ? s2[r] : -INFINITY;
    }
    const float lm = fmaxf(fmaxf(s2[0], s2[1]), fmaxf(s2[2], s2[3]));
    float alpha = 1.f;
    if (__builtin_amdgcn_ballot_w64(lm > st.m + kLazyMax) != 0) {
        const float mn = fmaxf(st.m, rows_max(lm));
        alpha = fast_exp2(st.m - mn);
        st.m = mn;
    }
    st.l *= alpha;
    float pr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) pr[r] = fast_exp2(s2[r] - st.m);
    st.l += (pr[0] + pr[1]) + (pr[2] + pr[3]);
    h4 pop;
#pragma unroll
    for (int r = 0; r < 4; ++r) pop[r] = (_Float16)pr[r];
    // The rescale by alpha (1 unless the lazy max moved) is applied tile by tile right
    // before each tile's MFMA, unconditionally: a conditional rescale would make the
    // compiler keep a second copy of the accumulator, and the scheduling barrier keeps it
    // from hoisting all multiplies (and their registers) ahead of the MFMAs.
#pragma unroll
    for (int t = 0; t < DV; ++t) {
        const h4 a = pv_rows<D>(ch.v, t);
        st.acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, pop, st.acc[t] * alpha, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Two chunks a, b at once, for head dims up to 64, whose chunks carry few bytes for the
// same softmax work: each chunk's QK^T into its own accumulator (the two K tiles staged in
// turn through the wave's tile: its LDS operations run in order), one softmax update over
// the lane's 8 scores, and one 16x16x32 PV product per tile over both chunks' 32 tokens
// (k-slots 8g + r: chunk a's token 4g + r, 8g + 4 + r: chunk b's; the lane's P values
// are already in that order). Both chunks are fully valid.
template <int D>
__device__ __forceinline__ void chunk_pair_f16(const ChunkF16<D>& ca, const ChunkF16<D>& cb,
                                               const h8* qop, float sl2, int g, char* kst,
                                               SoftmaxState<D>& st) {
    typedef ChunkF16<D> C;
    constexpr int NST = C::NST;
    constexpr int DV = C::DV;
    const int lane = __lane_id();
    f4 s[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const ChunkF16<D>& ch = j ? cb : ca;
#pragma unroll
        for (int i = 0; i < NST; ++i)
            *(h8*)(kst + kstage_off<D>(C::RPL * i + lane / C::PC, lane % C::PC)) = ch.k[i];
        h8 kop[NST];
#pragma unroll
        for (int k = 0; k < NST; ++k)
            kop[k] = *(const h8*)(kst + kstage_off<D>(lane & 15, 4 * k + g));
        s[j] = (f4)0.f;
#pragma unroll
        for (int k = 0; k < NST; ++k)
            s[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop[k], qop[k], s[j], 0, 0, 0);
    }
    float s2[8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        s2[r] = s[0][r] * sl2;
        s2[4 + r] = s[1][r] * sl2;
    }
    float lm = fmaxf(fmaxf(s2[0], s2[1]), fmaxf(s2[2], s2[3]));
    lm = fmaxf(lm, fmaxf(fmaxf(s2[4], s2[5]), fmaxf(s2[6], s2[7])));
    float alpha = 1.f;
    if (__builtin_amdgcn_ballot_w64(lm > st.m + kLazyMax) != 0) {
        const float mn = fmaxf(st.m, rows_max(lm));
        alpha = fast_exp2(st.m - mn);
        st.m = mn;
    }
    st.l *= alpha;
    float pr[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) pr[r] = fast_exp2(s2[r] - st.m);
    st.l += ((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7]));
    h8 pop;
#pragma unroll
    for (int r = 0; r < 8; ++r) pop[r] = (_Float16)pr[r];
#pragma unroll
    for (int t = 0; t < DV; ++t) {
        const h8 a = pv_rows2<D>(ca, cb, t);
        st.acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pop, st.acc[t] * alpha, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Reference max a quad-step stream starts from: finite, so that a slot that has seen no
// valid token yet (all scores -inf) gets p = 2^(-inf - m) = 0 rather than NaN, and its
// first real scores rescale it by 2^(m - m') = 0.
constexpr float kQuadM0 = -1e30f;

// Four chunks at once, for head dim 32 and at most 4 q heads per kv head: the 16
// MFMA columns hold 4 chunk slots x 4 heads (column j: head j & 3, slot j >> 2), so every
// column's softmax works on real scores (the single-chunk step runs it on 16 columns, of
// which G are heads). Each chunk's QK^T goes into its own accumulator against the same Q^T
// (head j & 3 in column j) and each lane keeps its slot's scores; PV is two 16x16x32
// products, over chunks (0, 1) and (2, 3) (k-slots 8g + r: the pair's first chunk's token
// 4g + r, 8g + 4 + r: the second's), each lane's P in its slot's half of its product and
// zeros elsewhere. A lane's state is its slot's stream; f16_quad_range merges the 4 streams
// of a head (columns j, j ^ 4, j ^ 8, j ^ 12) at the end. Slot s takes its chunk's first
// valid_s tokens (MASK; 0 = an empty slot). Measured at B8 x 32k, 32 q / 8 kv heads, stage 1
// at the default plan: head dim 32 95.1 -> 88.2 us against chunk pairs, but head dim 64
// 85.7 -> 94.6 us (its 4-chunk ring has nothing in flight while a quad computes).
template <int D, bool MASK>
__device__ __forceinline__ void chunk_quad_f16(const ChunkF16<D>* ch, const h8* qop, float sl2,
                                               int valid0, int valid1, int valid2, int valid3,
                                               int g, char* kst, SoftmaxState<D>& st) {
    typedef ChunkF16<D> C;
    constexpr int NST = C::NST;
    constexpr int DV = C::DV;
    const int lane = __lane_id();
    const int slot = (lane & 15) >> 2;
    f4 s[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
        for (int i = 0; i < NST; ++i)
            *(h8*)(kst + kstage_off<D>(C::RPL * i + lane / C::PC, lane % C::PC)) = ch[j].k[i];
        h8 kop[NST];
#pragma unroll
        for (int k = 0; k < NST; ++k)
            kop[k] = *(const h8*)(kst + kstage_off<D>(lane & 15, 4 * k + g));
        s[j] = (f4)0.f;
#pragma unroll
        for (int k = 0; k < NST; ++k)
            s[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop[k], qop[k], s[j], 0, 0, 0);
    }
    float s2[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float x = slot == 0 ? s[0][r] : slot == 1 ? s[1][r] : slot == 2 ? s[2][r] : s[3][r];
        s2[r] = x * sl2;
    }
    if (MASK) {
        const int v = slot == 0 ? valid0 : slot == 1 ? valid1 : slot == 2 ? valid2 : valid3;
#pragma unroll
        for (int r = 0; r < 4; ++r) s2[r] = 4 * g + r < v ? s2[r] : -INFINITY;
    }
    const float lm = fmaxf(fmaxf(s2[0], s2[1]), fmaxf(s2[2], s2[3]));
    float alpha = 1.f;
    if (__builtin_amdgcn_ballot_w64(lm > st.m + kLazyMax) != 0) {
        const float mn = fmaxf(st.m, rows_max(lm));
        alpha = fast_exp2(st.m - mn);
        st.m = mn;
    }
    st.l *= alpha;
    float pr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) pr[r] = fast_exp2(s2[r] - st.m);
    st.l += (pr[0] + pr[1]) + (pr[2] + pr[3]);
    h8 b01, b23;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const _Float16 x = (_Float16)pr[r], z = (_Float16)0.f;
        b01[r] = slot == 0 ? x : z;
        b01[4 + r] = slot == 1 ? x : z;
        b23[r] = slot == 2 ? x : z;
        b23[4 + r] = slot == 3 ? x : z;
    }
#pragma unroll
    for (int t = 0; t < DV; ++t) {
        const h8 a01 = pv_rows2<D>(ch[0], ch[1], t), a23 = pv_rows2<D>(ch[2], ch[3], t);
        st.acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a01, b01, st.acc[t] * alpha, 0, 0, 0);
        st.acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a23, b23, st.acc[t], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// f16_range for head dim 32 and at most 4 q heads per kv head: quad steps over a
// 4-chunk ring (chunks w_lo + 4k .. w_lo + 4k + 3; the wave's last full chunks, fewer than
// 4, fill the first slots of a masked step, the sequence's partial last chunk slot 0 of
// one more), then the 4 slot streams of each head merged and stored as in f16_range.
template <int D, int W, bool FINAL>
__device__ __forceinline__ void f16_quad_range(const DecodeParams& p, int kvh, int b,
                                               int seq_len, int w_lo, int w_hi, int wave,
                                               int64_t part_base, int64_t part_stride) {
    constexpr int NST = D / 32;
    constexpr int DV = D / 16;
    const int lane = threadIdx.x & 63;
    const int i16 = lane & 15, g = lane >> 4;
    const int G = p.group;
    const int head = i16 & 3;  // column j holds head j & 3
    const bool head_ok = head < G;
    const int c_full = seq_len >> 4;
    const int kvc = cache_head(p, kvh);
    h8 qop[NST];
    {
        const _Float16* qrow = (const _Float16*)p.q + (int64_t)b * p.q_sb +
                               (int64_t)(kvh * G + (head_ok ? head : 0)) * p.q_sh + 8 * g;
#pragma unroll
        for (int k = 0; k < NST; ++k) {
            h8 x = *(const h8*)(qrow + 32 * k);
            qop[k] = head_ok ? x : (h8)(_Float16)0;
        }
    }
    SoftmaxState<D> st;
#pragma unroll
    for (int t = 0; t < DV; ++t) st.acc[t] = (f4)0.f;
    st.m = kQuadM0;
    st.l = 0.f;
    const float sl2 = p.scale_log2;
    extern __shared__ __attribute__((aligned(16))) float smem[];
    char* kst = (char*)smem + wave * 32 * D;

    const int r_hi = min(w_hi, c_full);
    if (w_lo < r_hi) {
        const F16LaneOff<D> lo = f16_lane_offsets<D>(p, i16, g, 15);
        const int last = r_hi - 1;
        ChunkF16<D> ring[4];
        int pg_cur = chunk_pages<4>(p, b, w_lo, last, 0, 0);
        int pg_nxt = chunk_pages<4>(p, b, w_lo + 4, last, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            load_chunk_f16<D>(p, kvc, min(w_lo + i, last), lo,
                              __builtin_amdgcn_readlane(pg_cur, i), ring[i]);
            __builtin_amdgcn_sched_barrier(0);
        }
        for (int c0 = w_lo; c0 < r_hi; c0 += 4) {
            pg_cur = pg_nxt;  // pages of chunks c0 + 4 .. c0 + 7
            pg_nxt = chunk_pages<4>(p, b, c0 + 8, last, 0, 0);
            const int n = min(r_hi - c0, 4);
            if (n == 4)
                chunk_quad_f16<D, false>(ring, qop, sl2, 16, 16, 16, 16, g, kst, st);
            else
                chunk_quad_f16<D, true>(ring, qop, sl2, 16, n > 1 ? 16 : 0, n > 2 ? 16 : 0, 0,
                                        g, kst, st);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                load_chunk_f16<D>(p, kvc, min(c0 + 4 + i, last), lo,
                                  __builtin_amdgcn_readlane(pg_cur, i), ring[i]);
        }
    }
    if (w_lo <= r_hi && r_hi < w_hi) {  // this wave owns the partial last chunk c_full
        const int c = r_hi;
        const int valid = seq_len - (c << 4);
        const int pg = chunk_pages<1>(p, b, c, c, 0, 0);
        ChunkF16<D> q4[4];
        load_chunk_f16<D>(p, kvc, c, f16_lane_offsets<D>(p, i16, g, valid - 1),
                          __builtin_amdgcn_readlane(pg, 0), q4[0]);
        q4[1] = q4[0];
        q4[2] = q4[0];
        q4[3] = q4[0];
        chunk_quad_f16<D, true>(q4, qop, sl2, valid, 0, 0, 0, g, kst, st);
    }

    // the 4 slot streams of each head: columns j, j ^ 4, j ^ 8, j ^ 12
#pragma unroll
    for (int x = 4; x <= 8; x <<= 1) {
        const float m_o = __shfl_xor(st.m, x), l_o = __shfl_xor(st.l, x);
        const float M = fmaxf(st.m, m_o);
        const float wa = fast_exp2(st.m - M), wb = fast_exp2(m_o - M);
        st.l = wa * st.l + wb * l_o;
#pragma unroll
        for (int t = 0; t < DV; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                st.acc[t][r] = wa * st.acc[t][r] + wb * __shfl_xor(st.acc[t][r], x);
        st.m = M;
    }
    __syncthreads();  // every wave is done with its staging tile
    combine_store<D, W, FINAL>(p, st.acc, 1.f, 0.f, st.m, rows_sum(st.l), wave, i16, g, kvh, b,
                               part_base, part_stride);
}

// Ring depth of f16_range: head dims up to 64 run chunk pairs and keep at least 2 chunks
// in flight.
template <int D, int P>
constexpr int f16_ring() { return D <= 64 && P < 2 ? 2 : P; }

// The rows of the Q^T operand of kv head kvh of sequence b, unmasked: lane (i16, g) loads
// Q[head][32*k + 8*g + 0..7] of head i16, or of head 0 for the padding lanes i16 >= group,
// whose operand q_operand then zeroes. Loads only, so a caller can issue them ahead.
template <int D>
__device__ __forceinline__ void load_q_raw(const DecodeParams& p, int kvh, int b, h8* qraw) {
    const int lane = threadIdx.x & 63;
    const int i16 = lane & 15, g = lane >> 4;
    const int G = p.group;
    const _Float16* qrow = (const _Float16*)p.q + (int64_t)b * p.q_sb +
                           (int64_t)(kvh * G + (i16 < G ? i16 : 0)) * p.q_sh +
                           (D == 16 ? 4 : 8) * g;
    if constexpr (D == 16) {  // halves 4g .. 4g + 3, in the low half of qraw[0]
        const u2 x = *(const u2*)qrow;
        const u4v w = {x[0], x[1], 0u, 0u};
        qraw[0] = __builtin_bit_cast(h8, w);
    }
#pragma unroll
    for (int k = 0; k < D / 32; ++k) qraw[k] = *(const h8*)(qrow + 32 * k);
}

template <int D>
__device__ __forceinline__ void q_operand(const DecodeParams& p, const h8* qraw, h8* qop) {
    const bool head_ok = (threadIdx.x & 15) < p.group;
#pragma unroll
    for (int k = 0; k < ChunkF16<D>::KN; ++k) qop[k] = head_ok ? qraw[k] : (h8)(_Float16)0;
}

// The first loads of a wave's range, issued ahead by the work units for their guessed
// first segment (decode_common.h for_unit_segments) and not used there: the q rows of
// sequence b, the raw block-table entries of the ring's first two fills for the range
// [w_lo, last], and the ring's first fill itself (chunks w_lo .. w_lo + PR - 1 at their
// pages clamped into the pool, so a wrong guess reads valid memory and is not used).
template <int D, int P>
struct F16Pre {
    h8 qraw[ChunkF16<D>::KN];
    ChunkF16<D> ring[f16_ring<D, P>()];
    int pg_cur, pg_nxt;
    int b, w_lo, last;
    bool live;
};

template <int D, int P>
__device__ __forceinline__ F16Pre<D, P> f16_prefetch(const DecodeParams& p, int kvh,
                                                     const SegGuess& gs) {
    constexpr int PR = f16_ring<D, P>();
    F16Pre<D, P> f;
    f.live = false;
    if constexpr (D == 128) {  // the other head dims' kernels take no prefetch (registers)
        f.live = gs.live;
        f.b = gs.b;
        f.w_lo = gs.w_lo;
        f.last = min(gs.w_hi, gs.seq_len >> 4) - 1;
        // indices stay inside row b of the table: chunks >= 0 and <= max(last, 0)
        const int last0 = max(f.last, 0);
        load_q_raw<D>(p, kvh, gs.b, f.qraw);
        f.pg_cur = chunk_pages_raw<PR>(p, gs.b, min(f.w_lo, last0), last0, 0, 0);
        f.pg_nxt = chunk_pages_raw<PR>(p, gs.b, min(f.w_lo + PR, last0), last0, 0, 0);
        const int lane = threadIdx.x & 63;
        const F16LaneOff<D> lo = f16_lane_offsets<D>(p, lane & 15, lane >> 4, 15);
        const int pg = clamp_page(p, f.pg_cur);
#pragma unroll
        for (int i = 0; i < PR; ++i) {
            load_chunk_f16<D>(p, cache_head(p, kvh), min(f.w_lo + i, last0), lo,
                              __builtin_amdgcn_readlane(pg, i), f.ring[i]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    return f;
}

// P-deep register ring: chunk c + P is loaded while chunk c computes, the block-table
// entries of chunks c + 2P .. c + 3P - 1 meanwhile. Every load is issued on every path
// (chunks past the wave's last fully valid chunk re-read that chunk and are not used), so
// the compiler's vmcnt waits count exactly the loads in flight behind the awaited chunk
// and never drain the ring. The sequence's partial last chunk is handled once after it.
//
// f16_range runs one wave's chunk range [w_lo, w_hi) of sequence b (of length seq_len)
// for kv head kvh and stores the workgroup's result (partial rows part_base + h *
// part_stride, or the output row for FINAL).
//
// `pre` holds loads issued ahead for a guessed range (f16_prefetch); with use_pre, those
// that match this range (same sequence; same first chunk and last full chunk) replace the
// range's own.
template <int D, int W, bool FINAL, int P>
__device__ __forceinline__ void f16_range(const DecodeParams& p, int kvh, int b, int seq_len,
                                          int w_lo, int w_hi, int wave, int64_t part_base,
                                          int64_t part_stride, const F16Pre<D, P>& pre,
                                          bool use_pre) {
    constexpr int NST = D / 32;
    constexpr int DV = D / 16;
    if constexpr (D == 32) {
        if (p.group <= 4) {
            f16_quad_range<D, W, FINAL>(p, kvh, b, seq_len, w_lo, w_hi, wave, part_base,
                                        part_stride);
            return;
        }
    }

    const int lane = threadIdx.x & 63;
    const int i16 = lane & 15, g = lane >> 4;
    const int c_full = seq_len >> 4;  // chunks below this index are fully valid
    const int kvc = cache_head(p, kvh);
    const bool pre_b = use_pre && pre.live && pre.b == b;

    // Q^T operand: lane (head i16, g) holds Q[head][32*k + 8*g + 0..7] (D = 16:
    // Q[head][4g .. 4g + 3]); padded heads = 0.
    h8 qop[ChunkF16<D>::KN];
    if (pre_b) {
        q_operand<D>(p, pre.qraw, qop);
    } else {
        h8 qraw[ChunkF16<D>::KN];
        load_q_raw<D>(p, kvh, b, qraw);
        q_operand<D>(p, qraw, qop);
    }

    SoftmaxState<D> st;
#pragma unroll
    for (int t = 0; t < DV; ++t) st.acc[t] = (f4)0.f;
    st.m = -INFINITY;
    st.l = 0.f;
    const float sl2 = p.scale_log2;

    // this wave's K staging tile (the LDS of the cross-wave combine is reused after the
    // barrier below)
    extern __shared__ __attribute__((aligned(16))) float smem[];
    char* kst = (char*)smem + wave * 32 * D;

    // Head dims up to 64 run chunk pairs (w_lo + 2k, w_lo + 2k + 1), the wave's odd last
    // full chunk alone; the ring holds at least 2 chunks (depth 1 runs as 2), so the ring
    // depth never changes the arithmetic.
    constexpr bool PAIRS = D >= 32 && D <= 64;
    constexpr int PR = f16_ring<D, P>();
    const int r_hi = min(w_hi, c_full);
    if (w_lo < r_hi) {
        const F16LaneOff<D> lo = f16_lane_offsets<D>(p, i16, g, 15);
        const int last = r_hi - 1;
        ChunkF16<D> ring[PR];
        int pg_cur, pg_nxt;
        if (pre_b && pre.w_lo == w_lo && pre.last == last) {  // the first fill is in flight
            pg_cur = clamp_page(p, pre.pg_cur);
            pg_nxt = clamp_page(p, pre.pg_nxt);
#pragma unroll
            for (int i = 0; i < PR; ++i) ring[i] = pre.ring[i];
        } else {
            pg_cur = chunk_pages<PR>(p, b, w_lo, last, 0, 0);
            pg_nxt = chunk_pages<PR>(p, b, w_lo + PR, last, 0, 0);
            // Issued slot by slot: a slot's loads moved behind a later slot's would make
            // the ring's waits (vmcnt counts the loads issued after the awaited one) drain
            // it.
#pragma unroll
            for (int i = 0; i < PR; ++i) {
                load_chunk_f16<D>(p, kvc, min(w_lo + i, last), lo,
                                  __builtin_amdgcn_readlane(pg_cur, i), ring[i]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        for (int c0 = w_lo; c0 < r_hi; c0 += PR) {
            pg_cur = pg_nxt;  // pages of chunks c0 + PR .. c0 + 2PR - 1
            pg_nxt = chunk_pages<PR>(p, b, c0 + 2 * PR, last, 0, 0);
            if constexpr (PAIRS) {
#pragma unroll
                for (int i = 0; i < PR; i += 2) {
                    const int c = c0 + i;
                    if (c + 1 < r_hi)
                        chunk_pair_f16<D>(ring[i], ring[i + 1], qop, sl2, g, kst, st);
                    else if (c < r_hi)
                        chunk_f16<D, false>(ring[i], qop, sl2, 16, g, kst, st);
                    load_chunk_f16<D>(p, kvc, min(c + PR, last), lo,
                                      __builtin_amdgcn_readlane(pg_cur, i), ring[i]);
                    load_chunk_f16<D>(p, kvc, min(c + 1 + PR, last), lo,
                                      __builtin_amdgcn_readlane(pg_cur, i + 1), ring[i + 1]);
                }
            } else {
#pragma unroll
                for (int i = 0; i < PR; ++i) {
                    if (c0 + i < r_hi) chunk_f16<D, false>(ring[i], qop, sl2, 16, g, kst, st);
                    load_chunk_f16<D>(p, kvc, min(c0 + i + PR, last), lo,
                                      __builtin_amdgcn_readlane(pg_cur, i), ring[i]);
                }
            }
        }
    }
    if (w_lo <= r_hi && r_hi < w_hi) {  // this wave owns the partial last chunk c_full
        const int c = r_hi;
        const int valid = seq_len - (c << 4);
        const int pg = chunk_pages<1>(p, b, c, c, 0, 0);
        ChunkF16<D> ch;
        load_chunk_f16<D>(p, kvc, c, f16_lane_offsets<D>(p, i16, g, valid - 1),
                          __builtin_amdgcn_readlane(pg, 0), ch);
        chunk_f16<D, true>(ch, qop, sl2, valid, g, kst, st);
    }

    __syncthreads();  // every wave is done with its staging tile
    combine_store<D, W, FINAL>(p, st.acc, 1.f, 0.f, st.m, rows_sum(st.l), wave, i16, g, kvh, b,
                               part_base, part_stride);
}

// Split-KV stage 1 / single pass: workgroup = (kv head, split, sequence), W waves.
template <int D, int W, bool FINAL, int P>
__global__ __launch_bounds__(W * 64)
void decode_f16_kernel(const DecodeParams p) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const WgCoord wc = wg_coord(p, FINAL ? 1 : p.num_splits);
    if (!wc.live) return;
    const WaveRange wr = wave_range<W>(p, wc.b, wc.split, wave);
    const F16Pre<D, P> none{};
    f16_range<D, W, FINAL, P>(p, wc.kvh, wc.b, wr.seq_len, wr.w_lo, wr.w_hi, wave,
                              split_part_base(p, wc.b, wc.split), p.num_splits, none, false);
}

// Work units (decode_common.h UnitSpace): workgroup = (kv head, unit), W waves; the unit
// runs one segment per sequence its chunk range overlaps, its waves sharing each segment.
template <int D, int W, int P>
__global__ __launch_bounds__(W * 64)
void decode_f16_units_kernel(const DecodeParams p) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    for_unit_segments<W>(
        p, [&](int kvh, const SegGuess& gs) { return f16_prefetch<D, P>(p, kvh, gs); },
        [&](int kvh, int b, int seq_len, int w_lo, int w_hi, int64_t base, int64_t stride,
            const F16Pre<D, P>& pf, bool first) {
            f16_range<D, W, false, P>(p, kvh, b, seq_len, w_lo, w_hi, wave, base, stride, pf,
                                      first);
        });
}

// Merges the S partial rows row0 .. row0 + S - 1 into the fp16 output row `out`.
template <int D>
__device__ __forceinline__ void merge_rows(const float* __restrict__ o_part,
                                           const float* __restrict__ lse, int64_t row0, int S,
                                           _Float16* __restrict__ out) {
    constexpr int PER = D >= 32 ? D / 32 : 1;  // columns per thread (1..8)
    const int t = threadIdx.x, lane32 = t & 31, grp = t >> 5;
    const bool cols = lane32 * PER < D;  // head dim 16: lanes 16-31 of a group hold none
    float m = -INFINITY, wsum = 0.f;
    float acc[PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) acc[e] = 0.f;
#pragma unroll 4
    for (int s = grp; s < S; s += 8) {
        const float l = lse[row0 + s] * kLog2e;
        const float* src = o_part + (row0 + s) * D + (cols ? lane32 * PER : 0);
        float o[PER];
#pragma unroll
        for (int e = 0; e < PER; ++e) o[e] = cols ? src[e] : 0.f;
        if (l > m) {  // the running max grows: rescale what is summed so far
            const float r = fast_exp2(m - l);  // 0 while nothing is summed (m = -inf)
            wsum *= r;
#pragma unroll
            for (int e = 0; e < PER; ++e) acc[e] *= r;
            m = l;
        }
        const float w = l > -INFINITY ? fast_exp2(l - m) : 0.f;
        wsum += w;
#pragma unroll
        for (int e = 0; e < PER; ++e) acc[e] += w * o[e];
    }
    __shared__ float sm_acc[8][D];
    __shared__ float sm_m[8], sm_w[8];
#pragma unroll
    for (int e = 0; e < PER; ++e)
        if (cols) sm_acc[grp][lane32 * PER + e] = acc[e];
    if (lane32 == 0) {
        sm_m[grp] = m;
        sm_w[grp] = wsum;
    }
    __syncthreads();
    float M = -INFINITY;
#pragma unroll
    for (int g = 0; g < 8; ++g) M = fmaxf(M, sm_m[g]);
    for (int d = t; d < D; d += 256) {
        float o = 0.f, W = 0.f;
        if (M > -INFINITY) {
#pragma unroll
            for (int g = 0; g < 8; ++g) {
                const float r = sm_m[g] > -INFINITY ? fast_exp2(sm_m[g] - M) : 0.f;
                o += r * sm_acc[g][d];
                W += r * sm_w[g];
            }
        }
        out[d] = (_Float16)(W > 0.f ? o / W : 0.f);
    }
}

// Stage 2 (reference _merge_kernel, triton_fp16.py:147-163): out = sum_s w_s o_s / sum_s w_s
// with w_s = exp(lse_s - max lse). One workgroup of 256 threads per (q head, sequence) = 8
// groups of 32 threads; a thread owns D/32 consecutive columns and its group folds splits
// g, g+8, ... with a running max (in log2 units), rescaling its sums when the max grows,
// so every load of a split is independent of the others and of the max (one memory round
// trip instead of a max pass before the sum). The 8 groups are then combined through LDS
// against their common max. Empty splits (lse = -inf) get weight 0.
template <int D>
__global__ __launch_bounds__(256) void merge_kernel(const float* __restrict__ o_part,
                                                    const float* __restrict__ lse,
                                                    _Float16* __restrict__ out, int64_t o_sb,
                                                    int64_t o_sh, int q_heads, int S) {
    const int hq = blockIdx.x, b = blockIdx.y;
    merge_rows<D>(o_part, lse, ((int64_t)b * q_heads + hq) * S, S,
                  out + (int64_t)b * o_sb + (int64_t)hq * o_sh);
}

// Stage 2 of the work units (decode_common.h UnitSpace): sequence b's partials of q head hq
// are rows hq * (units + B) + u + b for its units u = first .. last, where first / last
// hold its first / last chunk. Workgroup = (q head, sequence), 256 threads; the prefix P_b
// and the total N come from one block reduction over seq_lens (thread t sums sequences
// t, t + 256, ...; B <= kUnitMaxBatch).
template <int D>
__global__ __launch_bounds__(256) void merge_units_kernel(const DecodeParams p) {
    const int hq = blockIdx.x, b = blockIdx.y, t = threadIdx.x;
    const int cap = p.max_blocks * p.block_size;
    const int n_b = cdiv(min(max(p.seq_lens[b], 0), cap), 16);
    int n_t = 0, n_pre = 0;
#pragma unroll
    for (int j = 0; j < kUnitMaxBatch / 256; ++j) {
        const int bb = t + 256 * j;
        const int n = bb < p.batch ? cdiv(min(max(p.seq_lens[bb], 0), cap), 16) : 0;
        n_t += n;
        n_pre += bb < b ? n : 0;
    }
    const int tot = wave_sum(n_t), pre = wave_sum(n_pre);
    __shared__ int red[2][4];
    if ((t & 63) == 0) {
        red[0][t >> 6] = tot;
        red[1][t >> 6] = pre;
    }
    __syncthreads();
    UnitSpace us;
    us.N = red[0][0] + red[0][1] + red[0][2] + red[0][3];
    us.NU = min(p.units, us.N);
    const int P = red[1][0] + red[1][1] + red[1][2] + red[1][3];
    _Float16* out = (_Float16*)p.out + (int64_t)b * p.o_sb + (int64_t)hq * p.o_sh;
    if (n_b == 0) {  // an empty sequence has no partials: a zero row
        for (int d = t; d < D; d += 256) out[d] = (_Float16)0.f;
        return;
    }
    const int first = unit_of(us, P), last = unit_of(us, (int64_t)P + n_b - 1);
    merge_rows<D>(p.o_part, p.lse, (int64_t)hq * (p.units + p.batch) + first + b,
                  last - first + 1, out);
}

template <int D, int W, bool FINAL, int P>
static hipError_t launch_f16(const DecodeParams& p, hipStream_t stream) {
    const dim3 grid(decode_grid(p.xcd_group, p.kv_heads, FINAL ? 1 : p.num_splits, p.batch));
    // the larger of the cross-wave combine ([W][G][D] + [W][16] m, l floats) and the
    // waves' K staging tiles (32 * D bytes each)
    const size_t combine = sizeof(float) * (W * p.group * D + 2 * W * 16);
    const size_t stage = (size_t)W * 32 * D;
    const size_t shmem = combine > stage ? combine : stage;
    hipLaunchKernelGGL((decode_f16_kernel<D, W, FINAL, P>), grid, dim3(W * 64), shmem, stream, p);
    return hipGetLastError();
}

template <int D, bool FINAL, int P>
static hipError_t launch_f16_w(const DecodeParams& p, int waves, hipStream_t stream) {
    switch (waves) {
        case 1: return launch_f16<D, 1, FINAL, P>(p, stream);
        case 2: return launch_f16<D, 2, FINAL, P>(p, stream);
        case 4: return launch_f16<D, 4, FINAL, P>(p, stream);
        case 8: return launch_f16<D, 8, FINAL, P>(p, stream);
        case 16: return launch_f16<D, 16, FINAL, P>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

template <int D, bool FINAL>
static hipError_t launch_f16_p(const DecodeParams& p, int waves, int ring, hipStream_t stream) {
    switch (ring) {
        case 1: return launch_f16_w<D, FINAL, 1>(p, waves, stream);
        case 2: return launch_f16_w<D, FINAL, 2>(p, waves, stream);
        case 4:
            if constexpr (D <= 128) return launch_f16_w<D, FINAL, 4>(p, waves, stream);
            return hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
}

template <int D>
static hipError_t launch_f16_d(const DecodeParams& p, bool final_out, int waves, int ring,
                               hipStream_t stream) {
    return final_out ? launch_f16_p<D, true>(p, waves, ring, stream)
                     : launch_f16_p<D, false>(p, waves, ring, stream);
}

template <int D, int W>
static hipError_t launch_units_w(const DecodeParams& p, int ring, hipStream_t stream) {
    const dim3 grid((unsigned)(p.kv_heads * p.units));
    const size_t combine = sizeof(float) * (W * p.group * D + 2 * W * 16);
    const size_t stage = (size_t)W * 32 * D;
    const size_t shmem = combine > stage ? combine : stage;
    switch (ring) {
        case 1:
            hipLaunchKernelGGL((decode_f16_units_kernel<D, W, 1>), grid, dim3(W * 64), shmem,
                               stream, p);
            break;
        case 2:
            hipLaunchKernelGGL((decode_f16_units_kernel<D, W, 2>), grid, dim3(W * 64), shmem,
                               stream, p);
            break;
        case 4:
            if constexpr (D <= 128) {
                hipLaunchKernelGGL((decode_f16_units_kernel<D, W, 4>), grid, dim3(W * 64), shmem,
                                   stream, p);
                break;
            }
            return hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int D>
static hipError_t launch_units_d(const DecodeParams& p, int waves, int ring,
                                 hipStream_t stream) {
    switch (waves) {
        case 1: return launch_units_w<D, 1>(p, ring, stream);
        case 2: return launch_units_w<D, 2>(p, ring, stream);
        case 4: return launch_units_w<D, 4>(p, ring, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_decode_units(const DecodeParams& p, int kv_format, int head_dim, int waves,
                               int ring, hipStream_t stream) {
    if (kv_format != KVQ_KV_F16)
        return launch_decode_q_units(p, kv_format, head_dim, waves, ring, stream);
    switch (head_dim) {
        case 16: return launch_units_d<16>(p, waves, ring, stream);
        case 32: return launch_units_d<32>(p, waves, ring, stream);
        case 64: return launch_units_d<64>(p, waves, ring, stream);
        case 128: return launch_units_d<128>(p, waves, ring, stream);
        case 256: return launch_units_d<256>(p, waves, ring, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_merge_units(const DecodeParams& p, int head_dim, hipStream_t stream) {
    const dim3 grid(p.q_heads, p.batch);
    switch (head_dim) {
        case 16: hipLaunchKernelGGL(merge_units_kernel<16>, grid, dim3(256), 0, stream, p); break;
        case 32: hipLaunchKernelGGL(merge_units_kernel<32>, grid, dim3(256), 0, stream, p); break;
        case 64: hipLaunchKernelGGL(merge_units_kernel<64>, grid, dim3(256), 0, stream, p); break;
        case 128: hipLaunchKernelGGL(merge_units_kernel<128>, grid, dim3(256), 0, stream, p); break;
        case 256: hipLaunchKernelGGL(merge_units_kernel<256>, grid, dim3(256), 0, stream, p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_decode(const DecodeParams& p, int kv_format, int head_dim, bool final_out,
                         int waves, int pipe, hipStream_t stream) {
    if (kv_format != KVQ_KV_F16)
        return launch_decode_q(p, kv_format, head_dim, final_out, waves, pipe, stream);
    switch (head_dim) {
        case 16: return launch_f16_d<16>(p, final_out, waves, pipe, stream);
        case 32: return launch_f16_d<32>(p, final_out, waves, pipe, stream);
        case 64: return launch_f16_d<64>(p, final_out, waves, pipe, stream);
        case 128: return launch_f16_d<128>(p, final_out, waves, pipe, stream);
        case 256: return launch_f16_d<256>(p, final_out, waves, pipe, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_merge(const float* o_part, const float* lse, void* out, int64_t o_sb,
                        int64_t o_sh, int batch, int q_heads, int head_dim, int num_splits,
                        hipStream_t stream) {
    const dim3 grid(q_heads, batch);
    _Float16* o = (_Float16*)out;
    switch (head_dim) {
        case 16:
            hipLaunchKernelGGL(merge_kernel<16>, grid, dim3(256), 0, stream, o_part, lse, o,
                               o_sb, o_sh, q_heads, num_splits);
            break;
        case 32:
            hipLaunchKernelGGL(merge_kernel<32>, grid, dim3(256), 0, stream, o_part, lse, o,
                               o_sb, o_sh, q_heads, num_splits);
            break;
        case 64:
            hipLaunchKernelGGL(merge_kernel<64>, grid, dim3(256), 0, stream, o_part, lse, o,
                               o_sb, o_sh, q_heads, num_splits);
            break;
        case 128:
            hipLaunchKernelGGL(merge_kernel<128>, grid, dim3(256), 0, stream, o_part, lse, o,
                               o_sb, o_sh, q_heads, num_splits);
            break;
        case 256:
            hipLaunchKernelGGL(merge_kernel<256>, grid, dim3(256), 0, stream, o_part, lse, o,
                               o_sb, o_sh, q_heads, num_splits);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace kvq
