// Paged-KV GQA decode attention over KIVI-quantized KV for gfx950: INT8, FP8-e4m3 (OCP
// e4m3fn) and packed INT4 codes with fp16 scale and zero-point, K per channel over groups
// of k_group tokens, V per token. The reference plans this (README.md:7, :16 "not
// started"); its byte model (src/bpt/roofline.py:6-9, 22-31) fixes the format's costs.
//
// Same workgroup/wave decomposition and MFMA layouts as the fp16 kernel (decode.hip); the
// dequantization is folded into the two products instead of being applied per element.
//
//   code c -> fp16 h, exactly and without a bias: h = c * w / F
//     INT8  h = c * 2^-24: the code is the mantissa of an fp16 subnormal (one v_perm per
//           two codes); F = 2^24, w = 1
//     INT4  nibbles masked in place: low nibbles (even codes) c * 2^-24 (w = 1), high
//           nibbles (odd codes) c * 2^-20 (w = 16); F = 2^24. Five VALU ops per 8 codes
//           for K; V takes whole bytes and the high nibbles (QFmt<KVQ_KV_INT4>::vtiles)
//     FP8   h = f(c) (v_cvt_scalef32_pk_f16_fp8, exact OCP e4m3fn); F = 1, w = 1
//   MI355X's MFMAs take fp16 subnormal inputs exactly (measured: a 32-term product sum of
//   subnormal A operands agrees with an exact sum to fp32 rounding).
//   K (x = c * s_d + z_d, per channel d):
//     q.k = sum_d q'_d c_d + C = F * sum_d (q'_d / w_d) h_d + C,   q' = q * s,
//     C = sum_d q_d z_d.  q'' = q' / w is held as hi + lo fp16 parts (recomputed per K
//     group); the MFMA chains give R = sum q'' h, and the log2-domain score is
//     R * (F * scale * log2 e) + C * scale * log2 e.
//   V (x = c * s_t + z_t, per token t):
//     sum_t p_t x_td = (F / w_d) * sum_t p''_t h_td + sum_t p_t z_t,  p'' = p * s_t as
//     hi + lo fp16 parts (the PV MFMA's B operand); the second sum is one fp32 scalar per
//     head (`corr`), added once at the end.
//
// Kernels:
//   decode_q2_kernel (1 to 4 q heads per kv head): the 16 MFMA columns hold 2 chunks x
//     4 heads x {hi, lo}. Column j: head j & 3, chunk (j >> 2) & 1 of the pair, part j >> 3.
//     The QK product runs the D/32 k-steps of each chunk against the same q'' operand into
//     two accumulators, and each column keeps its own chunk's, so one softmax pass covers
//     32 tokens; the PV product contracts both chunks in one 16x16x32 MFMA per tile:
//     k-slots 8g + r hold the first chunk's token 4g + r, 8g + 4 + r the second's;
//     each lane's p sits in the half of its own chunk, zeros in the other. The two chunks'
//     softmax streams of a head (columns j, j ^ 4) are merged once at the end.
//   decode_q2_kernel with SPLIT (5 to 8 heads): the columns hold {hi, lo} x 8 heads and
//     both chunks of the pair (chunk_pair_wide); the hi lane of a head weights one chunk,
//     its lo lane the other, and they swap the parts each column needs.
//   decode_q_kernel (5 to 16 heads; with pairs only where they do not apply: K groups of
//     one chunk, head dim 256, more than 8 heads): one chunk per step; up to 8 heads the
//     columns hold {hi, lo} x 8 heads (one QK chain), above that two chains.
// Head dims 64, 128 and 256 (decode_q.hip, decode_q_d64.hip and decode_q_d256.hip each
// instantiate one); 256 runs the single-chunk kernel with at most 2 chunks in flight.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "decode_common.h"

namespace kvq {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// v_perm_b32: byte k of the result is byte sel.k of {hi:lo} (0-3 = lo, 4-7 = hi, 12 = 0x00).
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// Byte e of a and byte e of b as the low bytes of two halves: [a.e, 0, b.e, 0].
__device__ __forceinline__ uint32_t pair_bytes(uint32_t a, uint32_t b, int e) {
    return perm(b, a, 0x0C040C00u + 0x00010001u * (uint32_t)e);
}

// Initial reference max of an online-softmax stream: finite, so that a stream that has
// seen no token yet (m = kM0, l = 0) rescales by exp2(kM0 - m') = 0 or 1 without NaN, and
// masked scores (-inf) give p = 0.
constexpr float kM0 = -1e30f;

template <int FMT, int D>
struct QFmt;

// Per format and head dim D (64, 128 or 256):
//   NST = k-steps of the QK product (32 channels each), DV = PV tiles (16 channels each);
//   KLOADS / VLOADS = K / V load instructions per 16-token chunk (whole rows), VBYTES =
//   bytes of each of its 4 token rows a lane needs for the PV operand, TILE = bytes of the
//   wave's LDS staging tiles (K rows for INT8 / FP8, then V rows), CPL = K-group channels
//   whose (scale, zero) pairs one lane loads.
//
// INT8 / FP8 share the byte layout: K rows of D bytes, PCS = D/16 pieces of 16 bytes per
// row, RPL = 64/PCS rows per load instruction (load j: lane l holds row RPL j + l/PCS,
// piece l%PCS - every 128-byte line in one instruction). After the LDS staging (kstage_q)
// lane (token l%16, g) holds pieces 4j + g for j < D/64; k-step st = 2j + u uses dwords
// 2u, 2u+1, i.e. channels 64*(st/2) + 16g + 8*(st%2) + e in order. V: D/16 bytes of each
// token row per lane (regrouped from whole rows by vstage_i8), tile t = byte t of the
// lane's D/16.
template <int D>
struct QFmtBytes {
    static_assert(D == 64 || D == 128 || D == 256, "quantized head_dim 64, 128 or 256");
    static constexpr int NST = D / 32, DV = D / 16;
    static constexpr int PCS = D / 16, RPL = 64 / PCS;
    static constexpr int KLOADS = D / 64, VLOADS = D / 64, VBYTES = D / 16;
    static constexpr int TILE = 16 * D + 20 * D;  // K tile, then the padded V tile
    static constexpr int CPL = D / 64;
    __device__ static int chan_base(int st, int g) { return 64 * (st >> 1) + 16 * g + 8 * (st & 1); }
    static constexpr bool permuted() { return false; }
};

template <int D>
struct QFmt<KVQ_KV_INT8, D> : QFmtBytes<D> {
    static constexpr float F = 16777216.f;  // 2^24
    __device__ static h8 kop(const u4v* kr, int st) {
        const u4v x = kr[st >> 1];
        const uint32_t d0 = x[2 * (st & 1)], d1 = x[2 * (st & 1) + 1];
        u4v o;
        o[0] = perm(0u, d0, 0x0C010C00u);
        o[1] = perm(0u, d0, 0x0C030C02u);
        o[2] = perm(0u, d1, 0x0C010C00u);
        o[3] = perm(0u, d1, 0x0C030C02u);
        return __builtin_bit_cast(h8, o);
    }
    // V^T operand dwords: tile t of token pairs (0, 1) and (2, 3) of the lane's 4 rows.
    __device__ static void vtiles(const uint32_t (*v)[D / 64], uint32_t* a01, uint32_t* a23) {
#pragma unroll
        for (int t = 0; t < D / 16; ++t) {
            a01[t] = pair_bytes(v[0][t >> 2], v[1][t >> 2], t & 3);
            a23[t] = pair_bytes(v[2][t >> 2], v[3][t >> 2], t & 3);
        }
    }
};

// FP8: gfx950 converts OCP e4m3fn to fp16 exactly in hardware (two codes per
// v_cvt_scalef32_pk_f16_fp8, scale 1.0), so h = f(c) with F = 1.
__device__ __forceinline__ uint32_t f8_lo(uint32_t x) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, 1.0f, false));
}
__device__ __forceinline__ uint32_t f8_hi(uint32_t x) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, 1.0f, true));
}

template <int D>
struct QFmt<KVQ_KV_FP8_E4M3, D> : QFmtBytes<D> {
    static constexpr float F = 1.f;
    __device__ static h8 kop(const u4v* kr, int st) {
        const u4v x = kr[st >> 1];
        const uint32_t d0 = x[2 * (st & 1)], d1 = x[2 * (st & 1) + 1];
        u4v o;
        o[0] = f8_lo(d0);
        o[1] = f8_hi(d0);
        o[2] = f8_lo(d1);
        o[3] = f8_hi(d1);
        return __builtin_bit_cast(h8, o);
    }
    __device__ static void vtiles(const uint32_t (*v)[D / 64], uint32_t* a01, uint32_t* a23) {
#pragma unroll
        for (int k = 0; k < D / 64; ++k) {
            // bytes [a0, b0, a1, b1] and [a2, b2, a3, b3] of token pairs, two codes per cvt
            const uint32_t x0 = perm(v[1][k], v[0][k], 0x05010400u);
            const uint32_t x1 = perm(v[1][k], v[0][k], 0x07030602u);
            const uint32_t y0 = perm(v[3][k], v[2][k], 0x05010400u);
            const uint32_t y1 = perm(v[3][k], v[2][k], 0x07030602u);
            a01[4 * k + 0] = f8_lo(x0);
            a01[4 * k + 1] = f8_hi(x0);
            a01[4 * k + 2] = f8_lo(x1);
            a01[4 * k + 3] = f8_hi(x1);
            a23[4 * k + 0] = f8_lo(y0);
            a23[4 * k + 1] = f8_hi(y0);
            a23[4 * k + 2] = f8_lo(y1);
            a23[4 * k + 3] = f8_hi(y1);
        }
    }
};

// INT4: K rows of D/2 bytes; lane (token, g) holds the row's bytes [8g, +8) (D = 64, one
// 8-byte load), [16g, +16) (D = 128, one 16-byte load) or [16g, +16) and [64 + 16g, +16)
// (D = 256, two loads). K-step st uses dword st of the lane's codes: halves in code order
// {0,4, 1,5, 2,6, 3,7} of channels chan_base(st, g), the odd codes at 2^-20 (w = 16). V:
// the lane needs D/32 bytes (D/16 codes) of each of its 4 token rows; the rows are loaded
// whole and regrouped through LDS (vstage_i4). Tiles 2k, 2k + 1 come from byte k of the
// lane's bytes: tile 2k takes the whole byte (code 2k + 16 code 2k+1, a subnormal below
// 2^-16 - no mask), tile 2k + 1 the odd code alone at 2^-20; tile_weights turns the sums
// back into codes 2k and 2k + 1. One v_perm and one v_and per two tiles of a token pair.
template <int D>
struct QFmt<KVQ_KV_INT4, D> {
    static_assert(D == 64 || D == 128 || D == 256, "quantized head_dim 64, 128 or 256");
    static constexpr float F = 16777216.f;  // 2^24
    static constexpr int NST = D / 32, DV = D / 16;
    static constexpr int KLOADS = D == 256 ? 2 : 1, VLOADS = D == 256 ? 2 : 1;
    static constexpr int VBYTES = D / 32;
    static constexpr int TILE = 16 * D;
    static constexpr int CPL = D / 64;
    __device__ static int chan_base(int st, int g) {
        return 128 * (st >> 2) + (D == 64 ? 16 : 32) * g + 8 * (st & 3);
    }
    static constexpr bool permuted() { return true; }
    __device__ static h8 kop(const u4v* kr, int st) {
        const uint32_t x = kr[st >> 2][st & 3], y = x >> 8;
        u4v o;
        o[0] = x & 0x000F000Fu;
        o[1] = x & 0x00F000F0u;
        o[2] = y & 0x000F000Fu;
        o[3] = y & 0x00F000F0u;
        return __builtin_bit_cast(h8, o);
    }
    __device__ static void vtiles(const uint32_t (*v)[(D / 32 + 3) / 4], uint32_t* a01,
                                  uint32_t* a23) {
#pragma unroll
        for (int k = 0; k < D / 32; ++k) {
            const uint32_t x = pair_bytes(v[0][k >> 2], v[1][k >> 2], k & 3);
            const uint32_t y = pair_bytes(v[2][k >> 2], v[3][k >> 2], k & 3);
            a01[2 * k] = x;
            a01[2 * k + 1] = x & 0x00F000F0u;
            a23[2 * k] = y;
            a23[2 * k + 1] = y & 0x00F000F0u;
        }
    }
};

// Dwords of each token row a lane holds for the PV operand (INT4 at D = 64: the low half
// of one dword).
template <int FMT, int D>
constexpr int vrow_dwords() {
    return (QFmt<FMT, D>::VBYTES + 3) / 4;
}

// Raw codes of one 16-token chunk as held by one lane, the V (scale, zero) pair of token
// 4g + (l & 3) (vsz, scale in the low half; pv_weights gives every lane of the quad the
// pairs of all 4 of its tokens 4g .. 4g + 3; for the first chunk of a chunk pair, of the
// chunk the lane's column holds), and (lane l) the pairs of channels CPL l .. CPL l + CPL - 1
// of the chunk's K group (ksz). The group data is loaded with every chunk that
// may start a group's use, not only with a group's first one: loads issued on every path
// keep the compiler's wait counts exact, so no chunk waits for loads it does not use.
template <int FMT, int D>
struct ChunkQ {
    u4v k[QFmt<FMT, D>::KLOADS];
    u4v vr[QFmt<FMT, D>::VLOADS];  // V whole rows (vstage_i4 / vstage_i8 give the layouts)
    uint32_t vsz;
    uint32_t ksz[QFmt<FMT, D>::CPL];
};

// Per-lane byte offsets of a chunk's loads inside its page (the page base and the slot
// are wave-uniform), `last` = valid tokens - 1 of the chunk:
//   K, INT4 (rows of D/2 bytes): row min(l%16, last), the lane's bytes (QFmt<INT4>) - one
//     instruction (two at D = 256) covers all 16 rows;
//   K, INT8 / FP8 (rows of D bytes): load j row min(RPL j + l/PCS, last), bytes
//     [16(l%PCS), +16) - each instruction covers whole rows (every 128-byte line in one
//     instruction); the rows reach the k-operand layout through the wave's LDS tile
//     (kstage_q);
//   V, the same whole-row pattern: INT4 rows of 32 bytes (D = 64: row min(l/4, last),
//     bytes [8(l%4), +8)), 64 bytes (row l/4, bytes [16(l%4), +16)) or 128 bytes (load j
//     row 8j + l/8, bytes [16(l%8), +16)); INT8 / FP8 as their K (regrouped by vstage_*);
//   the V (scale, zero) pair of token 4g + (l & 3) (4 bytes: the 64 bytes of the chunk's
//   16 pairs reach the wave once per row of 16 lanes, not once per lane), vs2 the same
//   token of the chunk pair's chunk (l >> 2) & 1, 64 bytes further for the second chunk,
//   vs3 that of chunk (l >> 3) & 1, and the K group's pairs of channels CPL l .. CPL l + CPL - 1 (4 CPL bytes).
struct QLaneOff {
    uint32_t k[4], v[4], vs, vs2, vs3, ks;
};

template <int FMT, int D>
__device__ __forceinline__ QLaneOff lane_offsets(const DecodeParams& p, int i16, int g,
                                                 int last) {
    typedef QFmt<FMT, D> Q;
    const int lane = __lane_id();
    const int ks = (int)p.k_stok, vs = (int)p.v_stok;
    QLaneOff o;
    if constexpr (FMT == KVQ_KV_INT4) {
        const int row = min(i16, last) * ks;
#pragma unroll
        for (int j = 0; j < Q::KLOADS; ++j)
            o.k[j] = (uint32_t)(row + (D == 64 ? 8 * g : 64 * j + 16 * g));
        if constexpr (D == 256) {  // 128-byte rows: 8 per instruction
#pragma unroll
            for (int j = 0; j < 2; ++j)
                o.v[j] = (uint32_t)(min(8 * j + (lane >> 3), last) * vs + 16 * (lane & 7));
        } else {  // 32- or 64-byte rows: 16 per instruction
            o.v[0] = (uint32_t)(min(lane >> 2, last) * vs + (D == 64 ? 8 : 16) * (lane & 3));
        }
    } else {
        constexpr int PCS = Q::PCS, RPL = Q::RPL;
#pragma unroll
        for (int j = 0; j < Q::KLOADS; ++j) {
            const int row = min(RPL * j + lane / PCS, last);
            o.k[j] = (uint32_t)(row * ks + 16 * (lane % PCS));
            o.v[j] = (uint32_t)(row * vs + 16 * (lane % PCS));
        }
    }
    o.vs = 16 * g + 4 * (lane & 3);
    o.vs2 = o.vs + 64 * ((lane >> 2) & 1);
    o.vs3 = o.vs + 64 * ((lane >> 3) & 1);
    o.ks = 4 * Q::CPL * lane;
    return o;
}

// Addressing of one kv head's data, made once per wave: the head's base in each tensor
// (64-bit) and the strides a chunk's address needs. A chunk's loads go through buffer
// resources based at its block - base + block * block stride, a 64-bit scalar product, so
// pools of any size work - with the token slot as one 32-bit scalar offset (soffset) and
// the lane's 32-bit offset (voffset): a few scalar operations per chunk and no vector
// address arithmetic. Offsets inside a block are below 2^31 bytes (checked on the host).
struct QBase {
    const char* k;   // codes of kv head kvh in block 0
    const char* v;
    const char* vs;  // V (scale, zero) pairs of kv head kvh in block 0
    const char* ks;  // K (scale, zero) pairs of kv head kvh in block 0
    uint32_t k_sblk, v_sblk, k_stok, v_stok;
    uint32_t vs_blk, ks_blk;  // bytes per block of the V / K pair tensors
    uint32_t cmask;           // 16-token chunks per page - 1
    uint32_t vmask;           // 16-token chunks per V (scale, zero) group - 1
};

// Buffer resource at a wave-uniform address: stride 0, the full 32-bit range (offsets from
// it stay below 2^31), dword data format.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t block_rsrc(const char* base, int phys,
                                                             uint32_t blk_bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(base + (uint64_t)(uint32_t)phys * blk_bytes), (short)0, -1, 0x00020000);
}

// kvh: the caches' kv head (cache_head); D the head dim.
template <int D>
__device__ __forceinline__ QBase q_base(const DecodeParams& p, int kvh) {
    const int hkv = p.kv_heads / p.kv_rep;  // the caches' kv heads
    QBase B;
    B.k = (const char*)p.k + (int64_t)kvh * p.k_sh;
    B.v = (const char*)p.v + (int64_t)kvh * p.v_sh;
    B.vs = (const char*)p.v_scale + ((int64_t)kvh * 4 << p.vg_shift);
    B.ks = (const char*)p.k_scale + (int64_t)kvh * 4 * D;
    B.k_sblk = (uint32_t)p.k_sblk;
    B.v_sblk = (uint32_t)p.v_sblk;
    B.k_stok = (uint32_t)p.k_stok;
    B.v_stok = (uint32_t)p.v_stok;
    B.vs_blk = (uint32_t)(hkv * 4) << p.vg_shift;
    B.ks_blk = (uint32_t)(hkv * 4 * D);
    B.cmask = (1u << p.cpp_shift) - 1;
    B.vmask = (1u << (p.vg_shift - 4)) - 1;
    return B;
}

// Cache policy of the loads that stream the cache once (codes, V scale/zero): nt, the
// streaming hint; measured on MI355X it lifts a plain streaming read from about 6.3 to
// 7.0 TB/s. The K group scales, which every chunk of the group reloads, keep the default
// policy.
constexpr int kNT = 2;

// 16 bytes per lane, or 8 (INT4 rows at D = 64) in the low half of the vector.
template <bool HALF>
__device__ __forceinline__ u4v load_codes(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                          uint32_t soff) {
    if constexpr (HALF) {
        const u2 x = __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, kNT));
        return __builtin_shufflevector(x, x, 0, 1, 0, 1);
    } else {
        return __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kNT);
    }
}

// WITH_K: also load the K group's (scale, zero) pairs (ch.ksz), stored with the group's
// first page `lead`. VS: the V (scale, zero) pairs ch.vsz brings, from the chunk's V group
// in its first page `vlead`: 1 the chunk's own; 2 those of the chunk pair c, c + 1 (c even,
// both in one V group: lane l takes chunk c + ((l >> 2) & 1)); 3 the same with chunk
// c + ((l >> 3) & 1); 0 none.
template <int FMT, int D, bool WITH_K = true, int VS = 1>
__device__ __forceinline__ void load_chunk_q(const QBase& B, int c, const QLaneOff& lo, int phys,
                                             int lead, int vlead, ChunkQ<FMT, D>& ch) {
    typedef QFmt<FMT, D> Q;
    constexpr bool HALF = FMT == KVQ_KV_INT4 && D == 64;
    const uint32_t slot = ((uint32_t)c & B.cmask) << 4;
    const auto rk = block_rsrc(B.k, phys, B.k_sblk);
    const auto rv = block_rsrc(B.v, phys, B.v_sblk);
#pragma unroll
    for (int j = 0; j < Q::KLOADS; ++j) ch.k[j] = load_codes<HALF>(rk, lo.k[j], slot * B.k_stok);
#pragma unroll
    for (int j = 0; j < Q::VLOADS; ++j) ch.vr[j] = load_codes<HALF>(rv, lo.v[j], slot * B.v_stok);
    // V (scale, zero) pair of token 4g + (l & 3) of the chunk (slots past the sequence
    // hold garbage and are masked by selects, never multiplied); the chunk's 16 pairs sit
    // at 64 (c & vmask) bytes in its V group
    if constexpr (VS != 0)
        ch.vsz = __builtin_amdgcn_raw_buffer_load_b32(block_rsrc(B.vs, vlead, B.vs_blk),
                                                      VS == 2 ? lo.vs2 : VS == 3 ? lo.vs3 : lo.vs,
                                                      64 * ((uint32_t)c & B.vmask & ~(VS >= 2 ? 1u : 0u)),
                                                      kNT);
    if constexpr (WITH_K) {
        const auto rs = block_rsrc(B.ks, lead, B.ks_blk);
        if constexpr (Q::CPL == 1) {
            ch.ksz[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, lo.ks, 0, 0);
        } else if constexpr (Q::CPL == 2) {
            const u2 x = __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(rs, lo.ks, 0, 0));
            ch.ksz[0] = x[0];
            ch.ksz[1] = x[1];
        } else {
            const u4v x = __builtin_amdgcn_raw_buffer_load_b128(rs, lo.ks, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) ch.ksz[i] = x[i];
        }
    }
}

// Half-row rotation: lane l reads lane (l & ~15) | ((l + 8) & 15), i.e. column n of a
// 16-lane row meets column n ^ 8 (DPP row_ror:8).
__device__ __forceinline__ float ror8(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf,
                                                      false));
}

// INT8 / FP8 K rows (16 rows of D bytes, loaded RPL whole rows per instruction) to the
// k-operand layout (lane (tok = l%16, g) holds bytes [64j + 16g, +16) of row tok, j < D/64)
// through the wave's LDS tile of 16 D bytes. 16-byte piece j of row r sits at slot
// j ^ ((r >> 1) % PCS). At D = 128 the row writes (16 lanes = 2 rows x 8 pieces) and the
// operand reads (16 lanes = 16 rows, one piece) each touch 16 distinct 16-byte slots
// modulo 256 bytes - no bank conflicts.
template <int D>
__device__ __forceinline__ void kstage_q(const u4v* rows, char* kst, int g, u4v* kr) {
    constexpr int PCS = D / 16, RPL = 64 / PCS;
    const int lane = __lane_id();
#pragma unroll
    for (int j = 0; j < D / 64; ++j) {
        const int row = RPL * j + lane / PCS;
        *(u4v*)(kst + row * D + 16 * ((lane % PCS) ^ ((row >> 1) & (PCS - 1)))) = rows[j];
    }
    const int tok = lane & 15;
#pragma unroll
    for (int j = 0; j < D / 64; ++j)
        kr[j] = *(const u4v*)(kst + tok * D + 16 * ((4 * j + g) ^ ((tok >> 1) & (PCS - 1))));
}

// The chunk's K codes in k-operand order.
template <int FMT, int D>
__device__ __forceinline__ void k_operand(const ChunkQ<FMT, D>& ch, char* kst, int g,
                                          u4v* kr) {
    if constexpr (FMT != KVQ_KV_INT4) {
        kstage_q<D>(ch.k, kst, g, kr);
    } else {
#pragma unroll
        for (int j = 0; j < QFmt<FMT, D>::KLOADS; ++j) kr[j] = ch.k[j];
    }
}

// INT4 V rows (16 rows of D/2 bytes, RS = D/8 dwords each) to the PV operand's grouping
// (lane (i16, g) needs bytes [D/32 i16, +D/32) of rows 4g .. 4g + 3) through the wave's LDS
// tile. Dword c of row R sits at 5 RS (R / 4) + RS (R % 4) + c. At D = 128 (lane l holding
// row l/4, dwords [4(l%4), +4)) the 16-byte row writes and the 4-byte reads (rows 4g + r,
// column i16: 80g + 16r + i16) each hit distinct banks, so neither conflicts.
template <int D>
__device__ __forceinline__ void vstage_i4(const u4v* vr, char* vst, int i16, int g,
                                          uint32_t (*v)[(D / 32 + 3) / 4]) {
    constexpr int RS = D / 8, GS = 5 * RS;
    const int lane = __lane_id();
    uint32_t* t = (uint32_t*)vst;
    if constexpr (D == 64) {  // rows of 32 bytes: lane l row l/4, dwords [2(l%4), +2)
        const int row = lane >> 2;
        *(u2*)(t + GS * (row >> 2) + RS * (row & 3) + 2 * (lane & 3)) = u2{vr[0][0], vr[0][1]};
#pragma unroll
        for (int r = 0; r < 4; ++r)
            v[r][0] = ((const uint16_t*)(t + GS * g + RS * r))[i16];
    } else if constexpr (D == 128) {
        const int row = lane >> 2;
        *(u4v*)(t + GS * (row >> 2) + RS * (row & 3) + 4 * (lane & 3)) = vr[0];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r][0] = t[GS * g + RS * r + i16];
    } else {  // rows of 128 bytes: load j lane l row 8j + l/8, dwords [4(l%8), +4)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int row = 8 * j + (lane >> 3);
            *(u4v*)(t + GS * (row >> 2) + RS * (row & 3) + 4 * (lane & 7)) = vr[j];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const u2 x = *(const u2*)(t + GS * g + RS * r + 2 * i16);
            v[r][0] = x[0];
            v[r][1] = x[1];
        }
    }
}

// INT8 / FP8 V rows (16 rows of D bytes, RS = D/4 dwords each; load j: lane l holds row
// RPL j + l/PCS, dwords [4(l%PCS), +4)) to the PV grouping (lane (i16, g) needs dwords
// [VW i16, +VW), VW = D/64, of rows 4g .. 4g + 3) through the wave's V tile (20 D bytes).
// Dword c of row R sits at 5 RS (R / 4) + RS (R % 4) + c. At D = 128 the 8-byte reads of
// lanes with g and g + 1 fall in opposite halves of 64 banks, the 16-byte writes of 8 lanes
// cover 32 distinct banks.
template <int D>
__device__ __forceinline__ void vstage_i8(const u4v* vr, char* vst, int i16, int g,
                                          uint32_t (*v)[D / 64]) {
    constexpr int RS = D / 4, GS = 5 * RS, PCS = D / 16, RPL = 64 / PCS, VW = D / 64;
    const int lane = __lane_id();
    uint32_t* t = (uint32_t*)vst;
#pragma unroll
    for (int j = 0; j < D / 64; ++j) {
        const int row = RPL * j + lane / PCS;
        *(u4v*)(t + GS * (row >> 2) + RS * (row & 3) + 4 * (lane % PCS)) = vr[j];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t* src = t + GS * g + RS * r + VW * i16;
        if constexpr (VW == 1) {
            v[r][0] = src[0];
        } else if constexpr (VW == 2) {
            const u2 x = *(const u2*)src;
            v[r][0] = x[0];
            v[r][1] = x[1];
        } else {
            const u4v x = *(const u4v*)src;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[r][e] = x[e];
        }
    }
}

// The chunk's V codes grouped by token row as vtiles takes them. The V tile follows the
// wave's K tile (16 D bytes) for INT8 / FP8 and takes its place for INT4 (no K staging).
template <int FMT, int D>
__device__ __forceinline__ void v_rows(const ChunkQ<FMT, D>& ch, char* kst, int i16, int g,
                                       uint32_t (*v)[vrow_dwords<FMT, D>()]) {
    if constexpr (FMT == KVQ_KV_INT4) {
        vstage_i4<D>(ch.vr, kst, i16, g, v);
    } else {
        vstage_i8<D>(ch.vr, kst + 16 * D, i16, g, v);
    }
}

// q'' = q * s / w of the K group whose scales lane l holds for channels CPL l .. CPL l +
// CPL - 1 (ksz), as hi + lo fp16 parts: hi = fp16(q s') (v_pk_mul_f16), lo = fma(q, s', -hi)
// rounded once (v_pk_fma_f16: q s' - hi is exact), s' = s / w. For INT4 the odd channels'
// s / 16 is exact unless it falls below the fp16 normal range, where its error stays under
// 2^-25 - at most 16 * 15 * 2^-25 |q| (about 7e-6 |q|) in the score. One fp16 rounding of
// q s alone would move logits by ~1e-3 on outlier channels. The lane keeps the part
// `lo_part` selects for the head whose q `qsh` points at (q in k-operand order in LDS, 64
// h8 apart per k-step). The scales pass through the wave's LDS slot `stage` (4 D bytes) to
// reach every lane in k-operand order (INT4: written there in the permuted order). Returns
// C = sum_d q_d z_d of that head (all D channels).
template <int FMT, int D>
__device__ __forceinline__ float make_qprime(const uint32_t* ksz, uint32_t* stage, int g,
                                             const h8* qsh, bool lo_part, h8* val) {
    typedef QFmt<FMT, D> Q;
    constexpr int CPL = Q::CPL;
    const int lane = __lane_id();
    _Float16* ss = (_Float16*)stage;
    _Float16* zz = (_Float16*)(stage + D / 2);
    if constexpr (Q::permuted()) {
        // channel c (even: w = 1, odd: w = 16) of block c / 8 sits at k-order position
        // 2 (c % 4) + (c % 8) / 4 of that block: {0, 4, 1, 5, 2, 6, 3, 7}
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = CPL * lane + i, e = c & 7;
            const int pos = (c & ~7) + 2 * (e & 3) + (e >> 2);
            const h2 sz = __builtin_bit_cast(h2, ksz[i]);
            ss[pos] = (e & 1) ? sz[0] * (_Float16)0.0625f : sz[0];
            zz[pos] = sz[1];
        }
    } else if constexpr (CPL == 1) {
        const h2 sz = __builtin_bit_cast(h2, ksz[0]);
        ss[lane] = sz[0];
        zz[lane] = sz[1];
    } else {
        // (s, z) pairs of two channels -> their two scales and their two zeros
#pragma unroll
        for (int i = 0; i < CPL; i += 2) {
            stage[CPL / 2 * lane + i / 2] = perm(ksz[i + 1], ksz[i], 0x05040100u);
            stage[D / 2 + CPL / 2 * lane + i / 2] = perm(ksz[i + 1], ksz[i], 0x07060302u);
        }
    }
    float qz = 0.f;
#pragma unroll
    for (int st = 0; st < Q::NST; ++st) {
        const h8 sv = *(const h8*)(ss + Q::chan_base(st, g));
        const h8 zv = *(const h8*)(zz + Q::chan_base(st, g));
        const h8 qv = qsh[64 * st];
        const h8 hi = qv * sv;
        const h8 lo = __builtin_elementwise_fma(qv, sv, -hi);
        val[st] = lo_part ? lo : hi;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const h2 qa = {qv[e], qv[e + 1]};
            const h2 za = {zv[e], zv[e + 1]};
            qz = __builtin_amdgcn_fdot2(qa, za, qz, false);
        }
    }
    return rows_sum(qz);
}

// Online-softmax update of one lane for its N = 4 or 8 scores s2 (log2 domain, masked
// scores -inf): rescales the state when a score passes the lazy reference max, returns
// p = 2^(s2 - m).
// PAIRED: lanes l and l ^ 8 hold different scores of one stream and keep one reference
// max (their maxima are combined through DPP row_ror:8).
template <int D, int N = 4, bool PAIRED = false>
__device__ __forceinline__ void softmax_step(float* s2, SoftmaxState<D>& st, float& corr,
                                             float* pr) {
    static_assert(N == 4 || N == 8, "4 or 8 scores per lane");
    float lm = fmaxf(fmaxf(s2[0], s2[1]), fmaxf(s2[2], s2[3]));
    if constexpr (N == 8) lm = fmaxf(lm, fmaxf(fmaxf(s2[4], s2[5]), fmaxf(s2[6], s2[7])));
    if constexpr (PAIRED) lm = fmaxf(lm, ror8(lm));
    if (__builtin_amdgcn_ballot_w64(lm > st.m + kLazyMax) != 0) {  // rare: the max moved
        const float mn = fmaxf(st.m, rows_max(lm));
        const float alpha = fast_exp2(st.m - mn);
        st.m = mn;
        st.l *= alpha;
        corr *= alpha;
#pragma unroll
        for (int t = 0; t < D / 16; ++t) st.acc[t] *= alpha;
    }
#pragma unroll
    for (int r = 0; r < N; ++r) pr[r] = fast_exp2(s2[r] - st.m);
    if constexpr (N == 4)
        st.l += (pr[0] + pr[1]) + (pr[2] + pr[3]);
    else
        st.l += ((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7]));
}

// p s_t as hi + lo fp16 parts, hi = fp16(p s_t) (fma with +0 is the product: p, s >= 0;
// v_fma_mix on the fp16 scale) and lo = fp16(p s_t - hi): one fp16 rounding of p s_t
// would be an error of up to 2^-11 (V - z) when one token dominates. corr accumulates
// p z_t in fp32. Rows r with !ok (past the sequence: garbage scales) give 0.
// vsz: lane r of each quad holds the pair of token 4g + r (ChunkQ::vsz); a DPP quad
// broadcast (quad_perm [r, r, r, r]) hands it to the quad's other lanes. The quad's lanes
// must all pass the same chunk's vsz.
template <int R>
__device__ __forceinline__ uint32_t quad_bcast(uint32_t x) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x55 * R, 0xf, 0xf, false);
}

template <bool MASK>
__device__ __forceinline__ void pv_weights(const float* pr, uint32_t vsz, int valid, int g,
                                           h4& phi, h4& plo, float& corr) {
    const uint32_t pairs[4] = {quad_bcast<0>(vsz), quad_bcast<1>(vsz), quad_bcast<2>(vsz),
                               quad_bcast<3>(vsz)};
    float cadd = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const bool ok = !MASK || 4 * g + r < valid;
        const uint32_t pair = pairs[r];
        const h2 sz = __builtin_bit_cast(h2, pair);
        const float sv = (float)sz[0];
        const _Float16 hi = (_Float16)__builtin_fmaf(pr[r], sv, 0.f);
        phi[r] = ok ? hi : (_Float16)0.f;
        plo[r] = ok ? (_Float16)__builtin_fmaf(pr[r], sv, -(float)hi) : (_Float16)0.f;
        cadd = __builtin_fmaf(pr[r], ok ? (float)sz[1] : 0.f, cadd);
    }
    corr += cadd;
}

// One chunk, 5 to 16 q heads per kv head (decode_q_kernel). SPLIT (at most 8 heads): the
// MFMA's 16 columns hold hi in column h and lo in column h + 8, so one QK^T chain gives
// both parts (summed across the half rows after the MFMAs) and one PV chain takes p''
// hi / lo the same way. Otherwise hi and lo run in two chains over columns [0, G).
template <int FMT, int D, bool MASK, bool SPLIT>
__device__ __forceinline__ void chunk_q(const ChunkQ<FMT, D>& ch, const h8* qhi, const h8* qlo,
                                        float csl, float sl2f, int valid, int g, char* kst,
                                        SoftmaxState<D>& st, float& corr) {
    typedef QFmt<FMT, D> Q;
    // V regrouped first (INT4: through LDS), so that its latency overlaps the QK product
    uint32_t vrows[4][vrow_dwords<FMT, D>()];
    v_rows<FMT, D>(ch, kst, __lane_id() & 15, g, vrows);
    u4v kr[Q::KLOADS];
    k_operand<FMT, D>(ch, kst, g, kr);
    float s2[4];
    if constexpr (SPLIT) {
        f4 sc = (f4)0.f;
#pragma unroll
        for (int k = 0; k < Q::NST; ++k)
            sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(Q::kop(kr, k), qhi[k], sc, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) s2[r] = __builtin_fmaf(sc[r] + ror8(sc[r]), sl2f, csl);
    } else {
        // hi and lo parts in two independent MFMA chains (half the dependent-chain latency)
        f4 sh = (f4)0.f, sl = (f4)0.f;
#pragma unroll
        for (int k = 0; k < Q::NST; ++k) {
            const h8 kh = Q::kop(kr, k);
            sh = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qhi[k], sh, 0, 0, 0);
            sl = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qlo[k], sl, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) s2[r] = __builtin_fmaf(sh[r] + sl[r], sl2f, csl);
    }
    if (MASK) {
#pragma unroll
        for (int r = 0; r < 4; ++r) s2[r] = 4 * g + r < valid ? s2[r] : -INFINITY;
    }
    float pr[4];
    softmax_step(s2, st, corr, pr);
    h4 phi, plo;
    pv_weights<MASK>(pr, ch.vsz, valid, g, phi, plo, corr);
    uint32_t a01[Q::DV], a23[Q::DV];
    Q::vtiles(vrows, a01, a23);
    if constexpr (SPLIT) {
        // column h takes p hi, column h + 8 p lo (the lanes of a pair hold the same p)
        const h4 pop = (__lane_id() & 8) ? plo : phi;
#pragma unroll
        for (int t = 0; t < Q::DV; ++t) {
            u2 w = {a01[t], a23[t]};
            st.acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h4, w), pop,
                                                               st.acc[t], 0, 0, 0);
        }
    } else {
#pragma unroll
        for (int t = 0; t < Q::DV; ++t) {
            u2 w = {a01[t], a23[t]};
            st.acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h4, w), phi,
                                                               st.acc[t], 0, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < Q::DV; ++t) {
            u2 w = {a01[t], a23[t]};
            st.acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h4, w), plo,
                                                               st.acc[t], 0, 0, 0);
        }
    }
}

// A chunk pair (chunks a, b) of one K group, 1 to 4 q heads per kv head
// (decode_q2_kernel). `slot` = the lane column's chunk (0: a, 1: b). Both chunks' QK
// products run against the same q'' operand (column j: head j & 3, part j >> 3) into two
// accumulators; each column keeps its own chunk's. csl = C * scale * log2 e of the group.
// MASK: tokens at or past valid_a / valid_b of their chunk are masked (valid_b = 0: no
// second chunk).
template <int FMT, int D, bool MASK>
__device__ __forceinline__ void chunk_pair(const ChunkQ<FMT, D>& ca, const ChunkQ<FMT, D>& cb,
                                           const h8* qv, float csl, float sl2f, int valid_a,
                                           int valid_b, int g, int slot, bool lo_part,
                                           char* kst, SoftmaxState<D>& st, float& corr) {
    typedef QFmt<FMT, D> Q;
    // V regrouped first (INT4: through LDS), so that its latency overlaps the QK products
    uint32_t va[4][vrow_dwords<FMT, D>()], vb[4][vrow_dwords<FMT, D>()];
    v_rows<FMT, D>(ca, kst, __lane_id() & 15, g, va);
    v_rows<FMT, D>(cb, kst, __lane_id() & 15, g, vb);
    f4 sa = (f4)0.f, sb = (f4)0.f;
    {
        u4v kr[Q::KLOADS];
        k_operand<FMT, D>(ca, kst, g, kr);
#pragma unroll
        for (int k = 0; k < Q::NST; ++k)
            sa = __builtin_amdgcn_mfma_f32_16x16x32_f16(Q::kop(kr, k), qv[k], sa, 0, 0, 0);
        k_operand<FMT, D>(cb, kst, g, kr);
#pragma unroll
        for (int k = 0; k < Q::NST; ++k)
            sb = __builtin_amdgcn_mfma_f32_16x16x32_f16(Q::kop(kr, k), qv[k], sb, 0, 0, 0);
    }
    float s2[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float x = slot ? sb[r] : sa[r];
        s2[r] = __builtin_fmaf(x + ror8(x), sl2f, csl);
    }
    const int valid = slot ? valid_b : valid_a;
    if (MASK) {
#pragma unroll
        for (int r = 0; r < 4; ++r) s2[r] = 4 * g + r < valid ? s2[r] : -INFINITY;
    }
    float pr[4];
    softmax_step(s2, st, corr, pr);
    const uint32_t vsz = ca.vsz;  // the pairs of the lane's own chunk (load_chunk_q VS 2)
    h4 phi, plo;
    pv_weights<MASK>(pr, vsz, valid, g, phi, plo, corr);
    // B operand: k-slots 8g + r (chunk a's token 4g + r) and 8g + 4 + r (chunk b's); the
    // lane's p in its chunk's half, zeros in the other
    const u2 pw = __builtin_bit_cast(u2, lo_part ? plo : phi);
    u4v pbw;
    pbw[0] = slot ? 0u : pw[0];
    pbw[1] = slot ? 0u : pw[1];
    pbw[2] = slot ? pw[0] : 0u;
    pbw[3] = slot ? pw[1] : 0u;
    const h8 pb = __builtin_bit_cast(h8, pbw);
    uint32_t a01[Q::DV], a23[Q::DV], b01[Q::DV], b23[Q::DV];
    Q::vtiles(va, a01, a23);
    Q::vtiles(vb, b01, b23);
#pragma unroll
    for (int t = 0; t < Q::DV; ++t) {
        const u4v w = {a01[t], a23[t], b01[t], b23[t]};
        st.acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, w), pb,
                                                           st.acc[t], 0, 0, 0);
    }
}

// A chunk pair (chunks a, b) of one K group, 5 to 8 q heads per kv head (decode_q2_kernel
// with SPLIT): the 16 columns hold {hi, lo} x 8 heads (column j: head j & 7, part j >> 3),
// as in chunk_q, and every column takes both chunks. Two QK accumulators (one per chunk)
// against the same q''. The hi lane (column j < 8) of a head runs the softmax and the PV
// weights of chunk a's rows, its lo lane (j + 8) those of chunk b: the two share one
// reference max (softmax_step PAIRED) and swap the parts the other column needs through
// DPP row_ror:8, so no lane repeats its partner's work; their l and corr are summed at the
// end. The PV product contracts both chunks in one 16x16x32 MFMA per tile (k-slots 8g + r:
// chunk a's token 4g + r, 8g + 4 + r: chunk b's). The V pairs come as load_chunk_q's VS 3
// (lane l: chunk (l >> 3) & 1, the lane's own); a single chunk loaded with VS 1 passes
// itself as b with valid_b = 0.
template <int FMT, int D, bool MASK>
__device__ __forceinline__ void chunk_pair_wide(const ChunkQ<FMT, D>& ca,
                                                const ChunkQ<FMT, D>& cb, const h8* qv,
                                                float csl, float sl2f, int valid_a, int valid_b,
                                                int g, bool lo_part, char* kst,
                                                SoftmaxState<D>& st, float& corr) {
    typedef QFmt<FMT, D> Q;
    const int lane = __lane_id();
    uint32_t va[4][vrow_dwords<FMT, D>()], vb[4][vrow_dwords<FMT, D>()];
    v_rows<FMT, D>(ca, kst, lane & 15, g, va);
    v_rows<FMT, D>(cb, kst, lane & 15, g, vb);
    f4 sa = (f4)0.f, sb = (f4)0.f;
    {
        u4v kr[Q::KLOADS];
        k_operand<FMT, D>(ca, kst, g, kr);
#pragma unroll
        for (int k = 0; k < Q::NST; ++k)
            sa = __builtin_amdgcn_mfma_f32_16x16x32_f16(Q::kop(kr, k), qv[k], sa, 0, 0, 0);
        k_operand<FMT, D>(cb, kst, g, kr);
#pragma unroll
        for (int k = 0; k < Q::NST; ++k)
            sb = __builtin_amdgcn_mfma_f32_16x16x32_f16(Q::kop(kr, k), qv[k], sb, 0, 0, 0);
    }
    // the lane's own chunk's scores, hi + lo: the hi lane sums chunk a's columns j and
    // j + 8, the lo lane chunk b's
    const int valid = lo_part ? valid_b : valid_a;
    float s2[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float x = lo_part ? sb[r] : sa[r], y = lo_part ? sa[r] : sb[r];
        s2[r] = __builtin_fmaf(x + ror8(y), sl2f, csl);
    }
    if (MASK) {
#pragma unroll
        for (int r = 0; r < 4; ++r) s2[r] = 4 * g + r < valid ? s2[r] : -INFINITY;
    }
    float pr[4];
    softmax_step<D, 4, true>(s2, st, corr, pr);
    h4 ph, pl;
    pv_weights<MASK>(pr, ca.vsz, valid, g, ph, pl, corr);
    // hi lane: chunk a's hi parts and (from the lo lane) chunk b's; lo lane: chunk a's lo
    // parts (from the hi lane) and chunk b's
    const u2 keep = __builtin_bit_cast(u2, lo_part ? pl : ph);
    const u2 send = __builtin_bit_cast(u2, lo_part ? ph : pl);
    u2 recv;
    recv[0] = (uint32_t)__float_as_int(ror8(__int_as_float((int)send[0])));
    recv[1] = (uint32_t)__float_as_int(ror8(__int_as_float((int)send[1])));
    u4v pbw;
    pbw[0] = lo_part ? recv[0] : keep[0];
    pbw[1] = lo_part ? recv[1] : keep[1];
    pbw[2] = lo_part ? keep[0] : recv[0];
    pbw[3] = lo_part ? keep[1] : recv[1];
    const h8 pb = __builtin_bit_cast(h8, pbw);
    uint32_t a01[Q::DV], a23[Q::DV], b01[Q::DV], b23[Q::DV];
    Q::vtiles(va, a01, a23);
    Q::vtiles(vb, b01, b23);
#pragma unroll
    for (int t = 0; t < Q::DV; ++t) {
        const u4v w = {a01[t], a23[t], b01[t], b23[t]};
        st.acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, w), pb,
                                                           st.acc[t], 0, 0, 0);
    }
}

// INT4 V tiles: tile 2k sums p'' (c_2k + 16 c_2k+1), tile 2k + 1 sums p'' 16 c_2k+1 (both in
// units of 2^-24). Code 2k's sum is their difference and code 2k + 1's a sixteenth of the
// second. The difference cancels at most 255 / 15 of the magnitude: the fp32 accumulators'
// rounding stays below 2^-24 * 255 * sum p'', about 1.5e-5 of the largest V value.
template <int FMT, int D>
__device__ __forceinline__ void tile_weights(SoftmaxState<D>& st) {
    if constexpr (FMT == KVQ_KV_INT4) {
#pragma unroll
        for (int t = 0; t < D / 16; t += 2) {
            st.acc[t] -= st.acc[t + 1];
            st.acc[t + 1] *= 0.0625f;
        }
    }
}

// Writes q in this format's k-operand order (zero for heads >= G) to LDS for the
// once-per-K-group q'' products: [4 k-steps][64 lanes] h8, lane (g, head i16).
template <int FMT, int D>
__device__ __forceinline__ void stage_q(const DecodeParams& p, int b, int kvh, int i16, int g,
                                        h8* qsh) {
    typedef QFmt<FMT, D> Q;
    const int G = p.group;
    const bool head_ok = i16 < G;
    const _Float16* qrow = (const _Float16*)p.q + (int64_t)b * p.q_sb +
                           (int64_t)(kvh * G + (head_ok ? i16 : 0)) * p.q_sh;
#pragma unroll
    for (int st = 0; st < Q::NST; ++st) {
        h8 x = *(const h8*)(qrow + Q::chan_base(st, g));
        if constexpr (Q::permuted()) x = __builtin_shufflevector(x, x, 0, 4, 1, 5, 2, 6, 3, 7);
        qsh[64 * st + __lane_id()] = head_ok ? x : (h8)(_Float16)0;
    }
}

// P-deep register ring: chunk c + P is loaded while chunk c computes, the block-table
// entries of chunks c + 2P .. c + 3P - 1 meanwhile. Every chunk carries its own K group's
// scales, so any group size works with any P. 5 to 16 q heads per kv head.
//
// q_range runs one wave's chunk range [w_lo, w_hi) of sequence b (of length seq_len) for
// kv head kvh and stores the workgroup's result (partial rows part_base + h * part_stride,
// or the output row for FINAL).
template <int FMT, int D, int W, bool FINAL, int P, bool SPLIT>
__device__ __forceinline__ void q_range(const DecodeParams& p, int kvh, int b, int seq_len,
                                        int w_lo, int w_hi, int wave, int64_t part_base,
                                        int64_t part_stride) {
    typedef QFmt<FMT, D> Q;
    constexpr int DV = D / 16, NST = D / 32;
    const int lane = threadIdx.x & 63;
    const int i16 = lane & 15, g = lane >> 4;
    const int G = p.group;
    const int c_full = seq_len >> 4;  // chunks below this index are fully valid
    const int kgs = p.k_group_shift;  // log2 of 16-token chunks per K group
    const int vgs = p.vg_shift - 4;   // log2 of 16-token chunks per V (scale, zero) group
    const QBase base = q_base<D>(p, cache_head(p, kvh));

    // LDS: [region 0][K-scale slots, 4 D bytes per wave][q, 32 D bytes] (launch_q). Region 0 holds
    // the cross-wave combine after the chunk loop and, before it, the waves' staging tiles
    // (Q::TILE bytes each: INT8 / FP8 K and V rows, INT4 V rows).
    extern __shared__ __attribute__((aligned(16))) float smem[];
    const int r0 = quant_lds_region0(W, G, FMT, D);
    char* kst = (char*)smem + wave * Q::TILE;
    h8* qsh = (h8*)(smem + r0 + W * D);
    if (wave == 0) stage_q<FMT, D>(p, b, kvh, i16, g, qsh);
    __syncthreads();
    qsh += SPLIT ? (lane & ~8) : lane;  // SPLIT: columns h and h + 8 read head h

    SoftmaxState<D> st;
#pragma unroll
    for (int t = 0; t < DV; ++t) st.acc[t] = (f4)0.f;
    st.m = kM0;
    st.l = 0.f;
    float corr = 0.f, csl = 0.f;
    const float sl2 = p.scale_log2, sl2f = sl2 * Q::F;
    h8 qhi[NST], qlo[NST];
    const bool upper = SPLIT && (lane & 8);

    uint32_t* stage = (uint32_t*)(smem + r0) + wave * D;
    auto valid_of = [&](int c) { return min(seq_len - (c << 4), 16); };
    // q'' of chunk ch's K group into the operands (hi / lo by column in SPLIT; both chains
    // otherwise) and C * scale * log2 e into csl
    auto new_group = [&](const ChunkQ<FMT, D>& ch) {
        h8 v[NST];
        if constexpr (SPLIT) {
            csl = make_qprime<FMT, D>(ch.ksz, stage, g, qsh, upper, v) * sl2;
#pragma unroll
            for (int k = 0; k < NST; ++k) qhi[k] = v[k];
        } else {
            csl = make_qprime<FMT, D>(ch.ksz, stage, g, qsh, false, qhi) * sl2;
            make_qprime<FMT, D>(ch.ksz, stage, g, qsh, true, qlo);
        }
    };

    // The ring covers the wave's fully valid chunks [w_lo, r_hi); the sequence's partial
    // last chunk (at most one per sequence) is handled once after it. Every load in the
    // ring is issued on every path (chunks past r_hi - 1 re-read chunk r_hi - 1 and are
    // never used), so each wait counts exactly the loads still in flight behind it.
    const int r_hi = min(w_hi, c_full);
    const int gmask = (1 << kgs) - 1;
    if (w_lo < r_hi) {
        const QLaneOff lo = lane_offsets<FMT, D>(p, i16, g, 15);
        const int last = r_hi - 1;
        ChunkQ<FMT, D> ring[P];
        int pg_cur = chunk_pages<P>(p, b, w_lo, last, kgs, vgs);
        int pg_nxt = chunk_pages<P>(p, b, w_lo + P, last, kgs, vgs);
        // Issued slot by slot: a slot's loads moved behind a later slot's would make the
        // ring's waits (vmcnt counts the loads issued after the awaited one) drain it.
#pragma unroll
        for (int i = 0; i < P; ++i) {
            load_chunk_q<FMT, D>(base, min(w_lo + i, last), lo,
                              __builtin_amdgcn_readlane(pg_cur, i),
                              __builtin_amdgcn_readlane(pg_cur, P + i),
                              __builtin_amdgcn_readlane(pg_cur, 2 * P + i), ring[i]);
            __builtin_amdgcn_sched_barrier(0);
        }
        for (int c0 = w_lo; c0 < r_hi; c0 += P) {
            pg_cur = pg_nxt;  // pages of chunks c0 + P .. c0 + 2P - 1
            pg_nxt = chunk_pages<P>(p, b, c0 + 2 * P, last, kgs, vgs);
#pragma unroll
            for (int i = 0; i < P; ++i) {
                const int c = c0 + i;
                if (c < r_hi) {
                    if (c == w_lo || (c & gmask) == 0) new_group(ring[i]);
                    chunk_q<FMT, D, false, SPLIT>(ring[i], qhi, qlo, csl, sl2f, 16, g, kst, st,
                                                  corr);
                }
                load_chunk_q<FMT, D>(base, min(c + P, last), lo,
                                  __builtin_amdgcn_readlane(pg_cur, i),
                                  __builtin_amdgcn_readlane(pg_cur, P + i),
                                  __builtin_amdgcn_readlane(pg_cur, 2 * P + i), ring[i]);
            }
        }
    }
    if (w_lo <= r_hi && r_hi < w_hi) {  // this wave owns the partial last chunk c_full
        const int c = r_hi;
        const int valid = valid_of(c);
        const int pg = chunk_pages<1>(p, b, c, c, kgs, vgs);
        ChunkQ<FMT, D> ch;
        load_chunk_q<FMT, D>(base, c, lane_offsets<FMT, D>(p, i16, g, valid - 1),
                             __builtin_amdgcn_readlane(pg, 0), __builtin_amdgcn_readlane(pg, 1),
                             __builtin_amdgcn_readlane(pg, 2), ch);
        if (c == w_lo || (c & gmask) == 0) new_group(ch);
        chunk_q<FMT, D, true, SPLIT>(ch, qhi, qlo, csl, sl2f, valid, g, kst, st, corr);
    }

    if constexpr (SPLIT) {  // add the lo columns into the hi columns
#pragma unroll
        for (int t = 0; t < DV; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) st.acc[t][r] += ror8(st.acc[t][r]);
    }
    tile_weights<FMT, D>(st);
    __syncthreads();  // every wave is done with its LDS staging tile
    combine_store<D, W, FINAL>(p, st.acc, Q::F, rows_sum(corr), st.m, rows_sum(st.l), wave, i16,
                               g, kvh, b, part_base, part_stride);
}

// Split-KV stage 1 / single pass: workgroup = (kv head, split, sequence), W waves.
template <int FMT, int D, int W, bool FINAL, int P, bool SPLIT>
__global__ __launch_bounds__(W * 64) void decode_q_kernel(const DecodeParams p) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const WgCoord wc = wg_coord(p, FINAL ? 1 : p.num_splits);
    if (!wc.live) return;
    const WaveRange wr = wave_range<W>(p, wc.b, wc.split, wave);
    q_range<FMT, D, W, FINAL, P, SPLIT>(p, wc.kvh, wc.b, wr.seq_len, wr.w_lo, wr.w_hi, wave,
                                        split_part_base(p, wc.b, wc.split), p.num_splits);
}

// Chunk pairs, 1 to 4 q heads per kv head, K groups of at least 2 chunks. Pairs are
// (2i, 2i + 1) in absolute chunk index, so both chunks of a pair share their K group; a
// wave's odd leading chunk, odd trailing full chunk and the sequence's partial last chunk
// run as single-chunk steps. P-deep ring over the pairs (P = 4 or 8 chunks: while a pair
// computes, P - 2 chunks are in flight); the ring depth never changes the arithmetic.
template <int FMT, int D, int W, bool FINAL, int P, bool WIDE>
__device__ __forceinline__ void q2_range(const DecodeParams& p, int kvh, int b, int seq_len,
                                         int w_lo, int w_hi, int wave, int64_t part_base,
                                         int64_t part_stride) {
    static_assert(P == 4 || P == 8, "a pair computes while P - 2 chunks are in flight");
    typedef QFmt<FMT, D> Q;
    constexpr int DV = D / 16, NST = D / 32;
    const int lane = threadIdx.x & 63;
    const int i16 = lane & 15, g = lane >> 4;
    const int G = p.group;
    const int slot = (i16 >> 2) & 1;   // the column's chunk of the pair
    const bool lo_part = i16 >= 8;     // the column holds the lo parts
    const int c_full = seq_len >> 4;
    const int kgs = p.k_group_shift;
    const int vgs = p.vg_shift - 4;
    const QBase base = q_base<D>(p, cache_head(p, kvh));

    // the chunk ranges, and the block-table entries of the pair ring's first two fills,
    // loaded before the q staging so that their round trip overlaps its own (clamped at use)
    const int r_hi = min(w_hi, c_full);  // fully valid chunks [w_lo, r_hi)
    const int c_first = (w_lo & 1) && w_lo < r_hi ? w_lo + 1 : w_lo;
    // pairs [c_first, e_hi); an empty wave or split has r_hi < w_lo and runs nothing
    const int e_hi = c_first + (max(r_hi - c_first, 0) & ~1);
    const int last_pair = max(e_hi - 1, 0);
    const int pg_raw0 = chunk_pages_raw<P>(p, b, min(c_first, last_pair), last_pair, kgs, vgs);
    const int pg_raw1 =
        chunk_pages_raw<P>(p, b, min(c_first + P, last_pair), last_pair, kgs, vgs);

    extern __shared__ __attribute__((aligned(16))) float smem[];
    const int r0 = quant_lds_region0(W, G, FMT, D);
    char* kst = (char*)smem + wave * Q::TILE;
    h8* qsh = (h8*)(smem + r0 + W * D);
    if (wave == 0) stage_q<FMT, D>(p, b, kvh, i16, g, qsh);
    __syncthreads();
    qsh += WIDE ? (lane & ~8) : ((lane & 48) | (lane & 3));  // column j reads head j & 7 / 3
    uint32_t* stage = (uint32_t*)(smem + r0) + wave * D;

    SoftmaxState<D> st;
#pragma unroll
    for (int t = 0; t < DV; ++t) st.acc[t] = (f4)0.f;
    st.m = kM0;
    st.l = 0.f;
    float corr = 0.f, csl = 0.f;
    const float sl2 = p.scale_log2, sl2f = sl2 * Q::F;
    h8 qv[NST];
    int gq = -1;  // the K group whose q'' qv holds

    auto group = [&](const ChunkQ<FMT, D>& ch, int gi) {
        if (gi != gq) {
            csl = make_qprime<FMT, D>(ch.ksz, stage, g, qsh, lo_part, qv) * sl2;
            gq = gi;
        }
    };
    // chunk c alone (in the first chunk's columns), its first `valid` tokens
    auto single = [&](int c, int valid) {
        const int pg = chunk_pages<1>(p, b, c, c, kgs, vgs);
        ChunkQ<FMT, D> ch;
        load_chunk_q<FMT, D>(base, c, lane_offsets<FMT, D>(p, i16, g, valid - 1),
                             __builtin_amdgcn_readlane(pg, 0), __builtin_amdgcn_readlane(pg, 1),
                             __builtin_amdgcn_readlane(pg, 2), ch);
        group(ch, c >> kgs);
        if constexpr (WIDE)
            chunk_pair_wide<FMT, D, true>(ch, ch, qv, csl, sl2f, valid, 0, g, lo_part, kst, st,
                                          corr);
        else
            chunk_pair<FMT, D, true>(ch, ch, qv, csl, sl2f, valid, 0, g, slot, lo_part, kst, st,
                                     corr);
    };

    if (c_first != w_lo) single(w_lo, 16);
    if (c_first < e_hi) {
        const QLaneOff lo = lane_offsets<FMT, D>(p, i16, g, 15);
        const int last = e_hi - 1;
        ChunkQ<FMT, D> ring[P];
        int pg_cur = clamp_page(p, pg_raw0);
        int pg_nxt = clamp_page(p, pg_raw1);
        // Issued slot by slot: a slot's loads moved behind a later slot's would make the
        // ring's waits (vmcnt counts the loads issued after the awaited one) drain it.
        // a pair's K group is its first chunk's: odd slots skip the K pair load
#pragma unroll
        for (int i = 0; i < P; ++i) {
            if (i % 2 == 0)
                load_chunk_q<FMT, D, true, WIDE ? 3 : 2>(
                    base, min(c_first + i, last), lo, __builtin_amdgcn_readlane(pg_cur, i),
                    __builtin_amdgcn_readlane(pg_cur, P + i),
                    __builtin_amdgcn_readlane(pg_cur, 2 * P + i), ring[i]);
            else
                load_chunk_q<FMT, D, false, 0>(base, min(c_first + i, last), lo,
                                               __builtin_amdgcn_readlane(pg_cur, i), 0, 0,
                                               ring[i]);
            __builtin_amdgcn_sched_barrier(0);
        }
        for (int c0 = c_first; c0 < e_hi; c0 += P) {
            pg_cur = pg_nxt;
            pg_nxt = chunk_pages<P>(p, b, c0 + 2 * P, last, kgs, vgs);
#pragma unroll
            for (int i = 0; i < P; i += 2) {
                const int c = c0 + i;
                if (c < e_hi) {
                    group(ring[i], c >> kgs);
                    if constexpr (WIDE)
                        chunk_pair_wide<FMT, D, false>(ring[i], ring[i + 1], qv, csl, sl2f, 16,
                                                       16, g, lo_part, kst, st, corr);
                    else
                        chunk_pair<FMT, D, false>(ring[i], ring[i + 1], qv, csl, sl2f, 16, 16,
                                                  g, slot, lo_part, kst, st, corr);
                }
                load_chunk_q<FMT, D, true, WIDE ? 3 : 2>(
                    base, min(c0 + i + P, last), lo, __builtin_amdgcn_readlane(pg_cur, i),
                    __builtin_amdgcn_readlane(pg_cur, P + i),
                    __builtin_amdgcn_readlane(pg_cur, 2 * P + i), ring[i]);
                load_chunk_q<FMT, D, false, 0>(base, min(c0 + i + 1 + P, last), lo,
                                               __builtin_amdgcn_readlane(pg_cur, i + 1), 0, 0,
                                               ring[i + 1]);
            }
        }
    }
    if (e_hi < r_hi) single(e_hi, 16);
    if (w_lo <= r_hi && r_hi < w_hi)  // this wave owns the partial last chunk c_full
        single(r_hi, min(seq_len - (r_hi << 4), 16));

    // hi + lo columns, then (up to 4 heads) the two chunk streams of each head (columns j,
    // j ^ 4)
#pragma unroll
    for (int t = 0; t < DV; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) st.acc[t][r] += ror8(st.acc[t][r]);
    if constexpr (!WIDE) {
        const float m_o = __shfl_xor(st.m, 4), l_o = __shfl_xor(st.l, 4);
        const float c_o = __shfl_xor(corr, 4);
        const float M = fmaxf(st.m, m_o);
        const float wa = fast_exp2(st.m - M), wb = fast_exp2(m_o - M);
        st.l = wa * st.l + wb * l_o;
        corr = wa * corr + wb * c_o;
#pragma unroll
        for (int t = 0; t < DV; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                st.acc[t][r] = wa * st.acc[t][r] + wb * __shfl_xor(st.acc[t][r], 4);
        st.m = M;
    } else {  // the hi and lo lanes of a head summed different chunks' l and corr
        st.l += ror8(st.l);
        corr += ror8(corr);
    }
    tile_weights<FMT, D>(st);
    __syncthreads();  // every wave is done with its LDS staging tile
    combine_store<D, W, FINAL>(p, st.acc, Q::F, rows_sum(corr), st.m, rows_sum(st.l), wave, i16,
                               g, kvh, b, part_base, part_stride);
}

template <int FMT, int D, int W, bool FINAL, int P, bool WIDE>
__global__ __launch_bounds__(W * 64) void decode_q2_kernel(const DecodeParams p) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const WgCoord wc = wg_coord(p, FINAL ? 1 : p.num_splits);
    if (!wc.live) return;
    const WaveRange wr = wave_range<W>(p, wc.b, wc.split, wave);
    q2_range<FMT, D, W, FINAL, P, WIDE>(p, wc.kvh, wc.b, wr.seq_len, wr.w_lo, wr.w_hi, wave,
                                        split_part_base(p, wc.b, wc.split), p.num_splits);
}

// Work units (decode_common.h UnitSpace): workgroup = (kv head, unit), W waves running
// one segment per sequence the unit's chunk range overlaps, each wave a contiguous share
// of it; PAIRS selects the chunk-pair kernel (with SPLIT: 5 to 8 heads, chunk_pair_wide).
template <int FMT, int D, int W, int P, bool PAIRS, bool SPLIT>
__global__ __launch_bounds__(W * 64) void decode_q_units_kernel(const DecodeParams p) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    for_unit_segments<W>(p, [&](int kvh, int b, int seq_len, int w_lo, int w_hi, int64_t base,
                                int64_t stride) {
        if constexpr (PAIRS)
            q2_range<FMT, D, W, false, P, SPLIT>(p, kvh, b, seq_len, w_lo, w_hi, wave, base,
                                                 stride);
        else
            q_range<FMT, D, W, false, P, SPLIT>(p, kvh, b, seq_len, w_lo, w_hi, wave, base,
                                                stride);
    });
}

// LDS: region 0 (the cross-wave combine, or the waves' staging tiles), one K-scale slot of
// 4 D bytes per wave, then q in k-operand order (32 D bytes)
template <int FMT, int D, int W>
static size_t q_shmem(const DecodeParams& p) {
    return sizeof(float) * (quant_lds_region0(W, p.group, FMT, D) + W * D) + 32 * D;
}

template <int FMT, int D, int W, bool FINAL, int P, bool SPLIT>
static hipError_t launch_q(const DecodeParams& p, hipStream_t stream) {
    const dim3 grid(decode_grid(p.xcd_group, p.kv_heads, FINAL ? 1 : p.num_splits, p.batch));
    hipLaunchKernelGGL((decode_q_kernel<FMT, D, W, FINAL, P, SPLIT>), grid, dim3(W * 64),
                       (q_shmem<FMT, D, W>(p)), stream, p);
    return hipGetLastError();
}

template <int FMT, int D, int W, bool FINAL, int P, bool WIDE>
static hipError_t launch_q2(const DecodeParams& p, hipStream_t stream) {
    const dim3 grid(decode_grid(p.xcd_group, p.kv_heads, FINAL ? 1 : p.num_splits, p.batch));
    hipLaunchKernelGGL((decode_q2_kernel<FMT, D, W, FINAL, P, WIDE>), grid, dim3(W * 64),
                       (q_shmem<FMT, D, W>(p)), stream, p);
    return hipGetLastError();
}

// The pair kernel for up to 4 heads (chunk_pair) or 5 to 8 (chunk_pair_wide); ring 4 -> 8
// chunks in flight, else 4.
template <int FMT, int D, int W, bool FINAL>
static hipError_t launch_q2_g(const DecodeParams& p, int ring, hipStream_t stream) {
    if (p.group <= 4)
        return ring == 4 ? launch_q2<FMT, D, W, FINAL, 8, false>(p, stream)
                         : launch_q2<FMT, D, W, FINAL, 4, false>(p, stream);
    return ring == 4 ? launch_q2<FMT, D, W, FINAL, 8, true>(p, stream)
                     : launch_q2<FMT, D, W, FINAL, 4, true>(p, stream);
}

// 1 to 8 heads per kv head and K groups of at least 2 chunks: chunk pairs, ring 1 or 2 ->
// 4 chunks, 4 -> 8. Up to 8 heads otherwise (K groups of one chunk): hi / lo parts in the
// two column halves of one MFMA chain, any ring depth. 9 to 16 heads: two chains, ring
// depth 4. Head dim 256:
// the single-chunk kernel only, ring depth 1 or 2 (9 to 16 heads: 2), which keeps its
// twice-as-large chunks and tiles in registers.
template <int FMT, int D, bool FINAL, int W>
static hipError_t launch_q_g(const DecodeParams& p, int ring, hipStream_t stream) {
    if constexpr (D == 256) {
        if (p.group > 8) return launch_q<FMT, D, W, FINAL, 2, false>(p, stream);
        switch (ring) {
            case 1: return launch_q<FMT, D, W, FINAL, 1, true>(p, stream);
            case 2: return launch_q<FMT, D, W, FINAL, 2, true>(p, stream);
            default: return hipErrorInvalidValue;
        }
    } else {
        // pair kernel: ring 4 -> 8 chunks in flight, else 4 (a pair computes while P - 2
        // load); single-chunk kernel: the ring depth as given (two chains above 8 heads: 4)
        if (p.group <= 8 && p.k_group_chunks >= 2)
            return launch_q2_g<FMT, D, W, FINAL>(p, ring, stream);
        if (p.group > 8) return launch_q<FMT, D, W, FINAL, 4, false>(p, stream);
        switch (ring) {
            case 1: return launch_q<FMT, D, W, FINAL, 1, true>(p, stream);
            case 2: return launch_q<FMT, D, W, FINAL, 2, true>(p, stream);
            case 4: return launch_q<FMT, D, W, FINAL, 4, true>(p, stream);
            default: return hipErrorInvalidValue;
        }
    }
}

template <int FMT, int D, bool FINAL>
static hipError_t launch_q_w(const DecodeParams& p, int waves, int ring, hipStream_t stream) {
    if (ring != 1 && ring != 2 && ring != 4) return hipErrorInvalidValue;
    switch (waves) {
        case 1: return launch_q_g<FMT, D, FINAL, 1>(p, ring, stream);
        case 2: return launch_q_g<FMT, D, FINAL, 2>(p, ring, stream);
        case 4: return launch_q_g<FMT, D, FINAL, 4>(p, ring, stream);
        case 8: return launch_q_g<FMT, D, FINAL, 8>(p, ring, stream);
        default: return hipErrorInvalidValue;
    }
}

// Work units: the kernel variant launch_q_g picks, for W-wave workgroups.
template <int FMT, int D, int W, int P, bool PAIRS, bool SPLIT>
static hipError_t launch_qu(const DecodeParams& p, hipStream_t stream) {
    hipLaunchKernelGGL((decode_q_units_kernel<FMT, D, W, P, PAIRS, SPLIT>),
                       dim3((unsigned)(p.kv_heads * p.units)), dim3(W * 64),
                       (q_shmem<FMT, D, W>(p)), stream, p);
    return hipGetLastError();
}

template <int FMT, int D, int W>
static hipError_t launch_q_units_w(const DecodeParams& p, int ring, hipStream_t stream) {
    if constexpr (D == 256) {
        if (p.group > 8) return launch_qu<FMT, D, W, 2, false, false>(p, stream);
        switch (ring) {
            case 1: return launch_qu<FMT, D, W, 1, false, true>(p, stream);
            case 2: return launch_qu<FMT, D, W, 2, false, true>(p, stream);
            default: return hipErrorInvalidValue;
        }
    } else {
        if (p.group <= 4 && p.k_group_chunks >= 2)
            return ring == 4 ? launch_qu<FMT, D, W, 8, true, false>(p, stream)
                             : launch_qu<FMT, D, W, 4, true, false>(p, stream);
        if (p.group <= 8 && p.k_group_chunks >= 2)
            return ring == 4 ? launch_qu<FMT, D, W, 8, true, true>(p, stream)
                             : launch_qu<FMT, D, W, 4, true, true>(p, stream);
        if (p.group > 8) return launch_qu<FMT, D, W, 4, false, false>(p, stream);
        switch (ring) {
            case 1: return launch_qu<FMT, D, W, 1, false, true>(p, stream);
            case 2: return launch_qu<FMT, D, W, 2, false, true>(p, stream);
            case 4: return launch_qu<FMT, D, W, 4, false, true>(p, stream);
            default: return hipErrorInvalidValue;
        }
    }
}

template <int FMT, int D>
static hipError_t launch_q_units(const DecodeParams& p, int waves, int ring,
                                 hipStream_t stream) {
    switch (waves) {
        case 1: return launch_q_units_w<FMT, D, 1>(p, ring, stream);
        case 2: return launch_q_units_w<FMT, D, 2>(p, ring, stream);
        case 4: return launch_q_units_w<FMT, D, 4>(p, ring, stream);
        default: return hipErrorInvalidValue;
    }
}

// The entry points of one head dim (kvq_internal.h launch_decode_q_hd / _units_hd).
template <int D>
static hipError_t launch_decode_q_units_for(const DecodeParams& p, int kv_format, int waves,
                                            int ring, hipStream_t stream) {
    switch (kv_format) {
        case KVQ_KV_INT8: return launch_q_units<KVQ_KV_INT8, D>(p, waves, ring, stream);
        case KVQ_KV_FP8_E4M3: return launch_q_units<KVQ_KV_FP8_E4M3, D>(p, waves, ring, stream);
        case KVQ_KV_INT4: return launch_q_units<KVQ_KV_INT4, D>(p, waves, ring, stream);
        default: return hipErrorInvalidValue;
    }
}

template <int FMT, int D>
static hipError_t launch_q_f(const DecodeParams& p, bool final_out, int waves, int ring,
                             hipStream_t stream) {
    return final_out ? launch_q_w<FMT, D, true>(p, waves, ring, stream)
                     : launch_q_w<FMT, D, false>(p, waves, ring, stream);
}

template <int D>
static hipError_t launch_decode_q_for(const DecodeParams& p, int kv_format, bool final_out,
                                      int waves, int ring, hipStream_t stream) {
    switch (kv_format) {
        case KVQ_KV_INT8: return launch_q_f<KVQ_KV_INT8, D>(p, final_out, waves, ring, stream);
        case KVQ_KV_FP8_E4M3:
            return launch_q_f<KVQ_KV_FP8_E4M3, D>(p, final_out, waves, ring, stream);
        case KVQ_KV_INT4: return launch_q_f<KVQ_KV_INT4, D>(p, final_out, waves, ring, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace kvq
