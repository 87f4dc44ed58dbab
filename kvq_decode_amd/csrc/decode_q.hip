// Paged-KV GQA decode attention over KIVI-quantized KV for gfx950: INT8, FP8-e4m3 (OCP
// e4m3fn) and packed INT4 codes with fp16 scale and zero-point, K per channel over groups
// of k_group tokens, V per token. The reference plans this (README.md:7, :16 "not
// started"); its byte model (src/bpt/roofline.py:6-9, 22-31) fixes the format's costs.
//
// Same workgroup/wave decomposition and MFMA layouts as the fp16 kernel (decode.hip); the
// dequantization is folded into the two products instead of being applied per element:
//
//   code c -> fp16 h exactly, with c = F * (h - B):
//     INT8  h = 1024 + c  (v_perm with 0x64 bytes; F = 1, B = 1024)
//     INT4  h = 1 + c/64  (nibble into mantissa bits 4-7 of 1.0; F = 64, B = 1)
//     FP8   h = f(c)      (v_cvt_scalef32_pk_f16_fp8, exact; F = 1, B = 0)
//   K (x = c * s_d + z_d, per channel d):
//     q.k = sum_d q'_d c_d + sum_d q_d z_d,  q' = q * s = hi + lo (two fp16 parts,
//           recomputed per K group)
//         = F * (sum_d q'_d h_d + C),  C = sum_d q_d z_d / F - B * sum_d q'_d
//     -> MFMA chains on h (with hi, then lo) with C as the accumulator input, then * F.
//   V (x = c * s_t + z_t, per token t):
//     sum_t p_t x_td = F * sum_t p''_t h_td + corr,  p'' = fp16(p * s_t),
//     corr = sum_t (p_t z_t - F * B * p''_t)     (fp32, per head, rescaled with l)
//     -> the PV MFMA takes p'' as its B operand; corr is added once at the end.
// Only head_dim 128 is built for the quantized formats.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "decode_common.h"

namespace kvq {

typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// v_perm_b32: byte k of the result is byte sel.k of {hi:lo} (0-3 = lo, 4-7 = hi, 12 = 0x00).
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

constexpr uint32_t kMagicI8 = 0x64646464u;   // 0x64bb = fp16 1024 + bb
constexpr uint32_t kMagicI4 = 0x3C003C00u;   // fp16 1.0; nibble n at bits 4-7 -> 1 + n/64
constexpr uint32_t kNib = 0x00F000F0u;

// Two int8 codes -> halves (1024 + c): bytes 0,1 (lo) or 2,3 (hi) of x.
__device__ __forceinline__ uint32_t i8_lo(uint32_t x) { return perm(kMagicI8, x, 0x04010400u); }
__device__ __forceinline__ uint32_t i8_hi(uint32_t x) { return perm(kMagicI8, x, 0x04030402u); }

// The nibble mask and the 1.0 pattern, held in registers the compiler cannot see through,
// so (x & mask) | magic becomes one v_and_or_b32 (VOP3 takes no literal constants here)
// instead of a v_and_b32 + v_or_b32 pair with literals.
struct I4Consts {
    uint32_t nib, magic;
};

__device__ __forceinline__ I4Consts i4_consts() {
    I4Consts c{kNib, kMagicI4};
    asm volatile("" : "+v"(c.nib), "+v"(c.magic));
    return c;
}

__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t o) {
    return (x & m) | o;
}

// Nibbles of one dword (byte j = codes 2j (low), 2j+1 (high)) -> 8 halves 1 + c/64 in the
// order codes {0,4, 1,5, 2,6, 3,7}.
__device__ __forceinline__ u4v i4_dword(uint32_t x, I4Consts k) {
    u4v r;
    r[0] = and_or(x << 4, k.nib, k.magic);
    r[1] = and_or(x, k.nib, k.magic);
    r[2] = and_or(x >> 4, k.nib, k.magic);
    r[3] = and_or(x >> 8, k.nib, k.magic);
    return r;
}

template <int FMT>
struct QFmt;

// INT8 / FP8 share the byte layout: K rows of 128 bytes, lane (token l%16, g) loads bytes
// [64j + 16g, +16) for j = 0, 1; k-step st = 2j + u uses dwords 2u, 2u+1, i.e. channels
// 64*(st/2) + 16g + 8*(st%2) + e in order. V: 8 bytes per token row per lane.
template <>
struct QFmt<KVQ_KV_INT8> {
    static constexpr float F = 1.f, B = 1024.f;
    static constexpr int KLOADS = 2, VBYTES = 8;
    __device__ static int chan_base(int st, int g) { return 64 * (st >> 1) + 16 * g + 8 * (st & 1); }
    static constexpr bool permuted() { return false; }
    __device__ static h8 kop(const u4v* kr, int st, I4Consts) {
        const u4v x = kr[st >> 1];
        const uint32_t d0 = x[2 * (st & 1)], d1 = x[2 * (st & 1) + 1];
        u4v o;
        o[0] = i8_lo(d0);
        o[1] = i8_hi(d0);
        o[2] = i8_lo(d1);
        o[3] = i8_hi(d1);
        return __builtin_bit_cast(h8, o);
    }
    // V^T operand halves of tile pairs: tiles 4k..4k+3 of token pair (ra, rb).
    __device__ static void vpair(uint32_t a, uint32_t b, uint32_t* out4) {
        const uint32_t y0 = perm(b, a, 0x05010400u), y1 = perm(b, a, 0x07030602u);
        out4[0] = i8_lo(y0);
        out4[1] = i8_hi(y0);
        out4[2] = i8_lo(y1);
        out4[3] = i8_hi(y1);
    }
};

// FP8: gfx950 converts OCP e4m3fn to fp16 exactly in hardware (two codes per
// v_cvt_scalef32_pk_f16_fp8, scale 1.0), so h = f(c) with F = 1, B = 0.
__device__ __forceinline__ uint32_t f8_lo(uint32_t x) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, 1.0f, false));
}
__device__ __forceinline__ uint32_t f8_hi(uint32_t x) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, 1.0f, true));
}

template <>
struct QFmt<KVQ_KV_FP8_E4M3> {
    static constexpr float F = 1.f, B = 0.f;
    static constexpr int KLOADS = 2, VBYTES = 8;
    __device__ static int chan_base(int st, int g) { return 64 * (st >> 1) + 16 * g + 8 * (st & 1); }
    static constexpr bool permuted() { return false; }
    __device__ static h8 kop(const u4v* kr, int st, I4Consts) {
        const u4v x = kr[st >> 1];
        const uint32_t d0 = x[2 * (st & 1)], d1 = x[2 * (st & 1) + 1];
        u4v o;
        o[0] = f8_lo(d0);
        o[1] = f8_hi(d0);
        o[2] = f8_lo(d1);
        o[3] = f8_hi(d1);
        return __builtin_bit_cast(h8, o);
    }
    __device__ static void vpair(uint32_t a, uint32_t b, uint32_t* out4) {
        const uint32_t y0 = perm(b, a, 0x05010400u), y1 = perm(b, a, 0x07030602u);
        out4[0] = f8_lo(y0);
        out4[1] = f8_hi(y0);
        out4[2] = f8_lo(y1);
        out4[3] = f8_hi(y1);
    }
};

// INT4: K rows of 64 bytes, lane (token, g) loads bytes [16g, +16) (channels [32g, +32));
// k-step st uses dword st, halves in code order {0,4,1,5,2,6,3,7} of channels 32g + 8st.
// V: 4 bytes (8 channels) per token row per lane.
template <>
struct QFmt<KVQ_KV_INT4> {
    static constexpr float F = 64.f, B = 1.f;
    static constexpr int KLOADS = 1, VBYTES = 4;
    __device__ static int chan_base(int st, int g) { return 32 * g + 8 * st; }
    static constexpr bool permuted() { return true; }
    __device__ static h8 kop(const u4v* kr, int st, I4Consts k) {
        return __builtin_bit_cast(h8, i4_dword(kr[0][st], k));
    }
    // Tiles 0..3 (channels 0..3 of the lane's 8) or 4..7 of token pair (ra, rb) from the
    // dwords a, b holding each token's 8 codes.
    __device__ static void vpair_half(uint32_t a, uint32_t b, uint32_t sel, uint32_t* out4,
                                      I4Consts k) {
        const uint32_t y = perm(b, a, sel);  // low 16 bits: ra's 4 codes, high: rb's
        out4[0] = and_or(y << 4, k.nib, k.magic);
        out4[1] = and_or(y, k.nib, k.magic);
        out4[2] = and_or(y >> 4, k.nib, k.magic);
        out4[3] = and_or(y >> 8, k.nib, k.magic);
    }
};

// Raw codes of one 16-token chunk as held by one lane, the 4 tokens' V scale/zero, and
// (lane l) channels 2l, 2l+1 of the scale/zero of the chunk's K group. The group data is
// loaded with every chunk, not only with a group's first one: loads issued on every path
// keep the compiler's wait counts exact, so no chunk waits for loads it does not use.
template <int FMT>
struct ChunkQ {
    u4v k[QFmt<FMT>::KLOADS];
    uint32_t v[4][QFmt<FMT>::VBYTES / 4];
    h4 vs, vz;
    uint32_t ks2, kz2;
};

// Per-lane byte offsets of a chunk's loads inside its page (the page base and the slot
// are wave-uniform): K row min(l%16, last) bytes [16g, +16) (+64 per further load), V rows
// min(4g + r, last) bytes [VBYTES * (l%16), +VBYTES), V scales of tokens 4g..4g+3, and
// channels 2l, 2l+1 of the K group scales. `last` = valid tokens - 1 of the chunk.
struct QLaneOff {
    uint32_t k, v[4], vs, ks;
};

template <int FMT>
__device__ __forceinline__ QLaneOff lane_offsets(const DecodeParams& p, int i16, int g,
                                                 int last) {
    typedef QFmt<FMT> Q;
    QLaneOff o;
    o.k = (uint32_t)(min(i16, last) * (int)p.k_stok + 16 * g);
#pragma unroll
    for (int r = 0; r < 4; ++r)
        o.v[r] = (uint32_t)(min(4 * g + r, last) * (int)p.v_stok + Q::VBYTES * i16);
    o.vs = 8 * g;
    o.ks = 4 * __lane_id();
    return o;
}

// Cache policy of the loads that stream the cache once (codes, V scale/zero): NT, the
// streaming hint (buffer_load ... nt); measured on MI355X it lifts a plain streaming read
// from about 6.3 to 7.0 TB/s. The K group scales, which every chunk of the group reloads,
// keep the default policy.
constexpr int kNT = 2;

template <int FMT>
__device__ __forceinline__ void load_chunk_q(const DecodeParams& p, int kvh, int c,
                                             const QLaneOff& lo, int phys, int lead,
                                             ChunkQ<FMT>& ch) {
    typedef QFmt<FMT> Q;
    const int slot = (c & ((1 << p.cpp_shift) - 1)) << 4;
    const char* kpage = (const char*)p.k + block_offset(phys, p.k_sblk) +
                        ((int64_t)slot * p.k_stok + (int64_t)kvh * p.k_sh);
    const char* vpage = (const char*)p.v + block_offset(phys, p.v_sblk) +
                        ((int64_t)slot * p.v_stok + (int64_t)kvh * p.v_sh);
    const auto rk = page_rsrc(kpage), rv = page_rsrc(vpage);
#pragma unroll
    for (int j = 0; j < Q::KLOADS; ++j)
        ch.k[j] = __builtin_amdgcn_raw_buffer_load_b128(rk, lo.k + 64 * j, 0, kNT);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        if constexpr (Q::VBYTES == 8) {
            const u2 x = __builtin_amdgcn_raw_buffer_load_b64(rv, lo.v[r], 0, kNT);
            ch.v[r][0] = x[0];
            ch.v[r][Q::VBYTES / 4 - 1] = x[1];
        } else {
            ch.v[r][0] = __builtin_amdgcn_raw_buffer_load_b32(rv, lo.v[r], 0, kNT);
        }
    }
    // V scale/zero of tokens slot + 4g .. +3 (4 consecutive halves; slots past the
    // sequence hold garbage and are masked in chunk_q).
    const uint64_t vrow = ((uint64_t)(uint32_t)phys * (uint32_t)p.kv_heads + kvh) *
                          (uint32_t)(2 * p.block_size);
    const auto rvs = page_rsrc((const char*)p.v_scale + vrow);
    const auto rvz = page_rsrc((const char*)p.v_zero + vrow);
    ch.vs = __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(rvs, lo.vs, 2 * slot, kNT));
    ch.vz = __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(rvz, lo.vs, 2 * slot, kNT));
    // K group scale/zero, stored with the group's first page `lead`
    const uint64_t krow = ((uint64_t)(uint32_t)lead * (uint32_t)p.kv_heads + kvh) * 256u;
    const auto rks = page_rsrc((const char*)p.k_scale + krow);
    const auto rkz = page_rsrc((const char*)p.k_zero + krow);
    ch.ks2 = __builtin_amdgcn_raw_buffer_load_b32(rks, lo.ks, 0, 0);
    ch.kz2 = __builtin_amdgcn_raw_buffer_load_b32(rkz, lo.ks, 0, 0);
}

// Half-row rotation: lane l reads lane (l & ~15) | ((l + 8) & 15), i.e. column n of a
// 16-lane row meets column n ^ 8 (DPP row_ror:8).
__device__ __forceinline__ float ror8(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf,
                                                      false));
}

// q' = q * s would lose 2^-12 relative per channel in fp16 - enough to move logits by
// ~1e-3 on outlier channels - so it is kept as hi + lo: hi = fp16(q s) (v_pk_mul_f16),
// lo = fma(q, s, -hi) rounded once (v_pk_fma_f16: q s - hi is exact).
// C = sum q z / F - B * sum (hi + lo) (v_dot2_f32_f16).
// SPLIT (at most 8 heads per kv head): the MFMA's 16 columns hold hi in column h and lo
// in column h + 8, so one QK^T chain gives both parts (summed across the half rows
// after the MFMAs); lanes of columns >= 8 take C = 0. Otherwise hi and lo run in two
// chains over columns [0, G).
// The group's scales (lane l holds channels 2l, 2l+1) pass through the wave's 512-byte
// LDS slot `stage` to reach every lane in k-operand order; `qsh` points at the lane's
// q in k-operand order (head l % 8 when SPLIT) in LDS, 64 h8 apart per k-step.
template <int FMT, bool SPLIT>
__device__ __forceinline__ float make_qprime(uint32_t s2, uint32_t z2, uint32_t* stage, int g,
                                             const h8* qsh, h8* qhi, h8* qlo) {
    typedef QFmt<FMT> Q;
    const int lane = __lane_id();
    const bool upper = SPLIT && (lane & 8);
    stage[lane] = s2;
    stage[64 + lane] = z2;
    const _Float16* ss = (const _Float16*)stage;
    const _Float16* zz = (const _Float16*)(stage + 64);
    float qz = 0.f, qs = 0.f;
    const h2 one = {(_Float16)1.f, (_Float16)1.f};
#pragma unroll
    for (int st = 0; st < 4; ++st) {
        h8 sv = *(const h8*)(ss + Q::chan_base(st, g));
        h8 zv = *(const h8*)(zz + Q::chan_base(st, g));
        if constexpr (Q::permuted()) {
            sv = __builtin_shufflevector(sv, sv, 0, 4, 1, 5, 2, 6, 3, 7);
            zv = __builtin_shufflevector(zv, zv, 0, 4, 1, 5, 2, 6, 3, 7);
        }
        const h8 qv = qsh[64 * st];
        const h8 hi = qv * sv;
        const h8 lo = __builtin_elementwise_fma(qv, sv, -hi);
        if constexpr (SPLIT) {
            qhi[st] = upper ? lo : hi;
        } else {
            qhi[st] = hi;
            qlo[st] = lo;
        }
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const h2 qa = {qv[e], qv[e + 1]};
            const h2 za = {zv[e], zv[e + 1]};
            const h2 ha = {hi[e], hi[e + 1]};
            const h2 la = {lo[e], lo[e + 1]};
            qz = __builtin_amdgcn_fdot2(qa, za, qz, false);
            qs = __builtin_amdgcn_fdot2(ha, one, qs, false);
            qs = __builtin_amdgcn_fdot2(la, one, qs, false);
        }
    }
    qz = rows_sum(qz);
    qs = rows_sum(qs);
    return upper ? 0.f : qz * (1.f / Q::F) - Q::B * qs;
}

template <int FMT, bool MASK, bool SPLIT>
__device__ __forceinline__ void chunk_q(const ChunkQ<FMT>& ch, const h8* qhi, const h8* qlo,
                                        float cinit, float sl2f, int valid, int g,
                                        SoftmaxState<128>& st, float& corr, I4Consts k4) {
    typedef QFmt<FMT> Q;
    float s2[4];
    if constexpr (SPLIT) {
        // one chain; column h + 8 holds the lo part of head h: s = C[h] + C[h + 8] in
        // both lanes of the pair
        f4 sc = (f4)cinit;
#pragma unroll
        for (int k = 0; k < 4; ++k)
            sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(Q::kop(ch.k, k, k4), qhi[k], sc, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) s2[r] = (sc[r] + ror8(sc[r])) * sl2f;
    } else {
        // hi and lo parts in two independent MFMA chains (half the dependent-chain latency)
        f4 sh = (f4)cinit, sl = (f4)0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const h8 kh = Q::kop(ch.k, k, k4);
            sh = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qhi[k], sh, 0, 0, 0);
            sl = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qlo[k], sl, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) s2[r] = (sh[r] + sl[r]) * sl2f;
    }
    if (MASK) {
#pragma unroll
        for (int r = 0; r < 4; ++r) s2[r] = 4 * g + r < valid ? s2[r] : -INFINITY;
    }
    const float lm = fmaxf(fmaxf(s2[0], s2[1]), fmaxf(s2[2], s2[3]));
    if (__builtin_amdgcn_ballot_w64(lm > st.m + kLazyMax) != 0) {  // rare: the max moved
        const float mn = fmaxf(st.m, rows_max(lm));
        const float alpha = fast_exp2(st.m - mn);
        st.m = mn;
        st.l *= alpha;
        corr *= alpha;
#pragma unroll
        for (int t = 0; t < 8; ++t) st.acc[t] *= alpha;
    }
    float pr[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) pr[r] = fast_exp2(s2[r] - st.m);
    st.l += (pr[0] + pr[1]) + (pr[2] + pr[3]);
    // p s_t feeds the MFMA as two fp16 parts, hi = fp16(p s_t) (fma with +0 is the
    // product: p, s >= 0; v_fma_mix_f32 on the fp16 scale) and lo = fp16(p s_t - hi): one
    // fp16 rounding of p s_t would be an error of up to 2^-11 (V - z) when one token
    // dominates. corr accumulates p z (v_fma_mix_f32) and -F B (hi + lo) (exact
    // products, v_dot2_f32_f16) in fp32.
    h4 phi, plo;
    float cadd = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const bool ok = !MASK || 4 * g + r < valid;
        const float sv = (float)ch.vs[r];
        const _Float16 hi = (_Float16)__builtin_fmaf(pr[r], sv, 0.f);
        phi[r] = ok ? hi : (_Float16)0.f;
        plo[r] = ok ? (_Float16)__builtin_fmaf(pr[r], sv, -(float)hi) : (_Float16)0.f;
        cadd = __builtin_fmaf(pr[r], ok ? (float)ch.vz[r] : 0.f, cadd);
    }
    if constexpr (Q::B != 0.f) {
        const h2 fb = {(_Float16)(-Q::F * Q::B), (_Float16)(-Q::F * Q::B)};
        cadd = __builtin_amdgcn_fdot2(__builtin_shufflevector(phi, phi, 0, 1), fb, cadd, false);
        cadd = __builtin_amdgcn_fdot2(__builtin_shufflevector(phi, phi, 2, 3), fb, cadd, false);
        cadd = __builtin_amdgcn_fdot2(__builtin_shufflevector(plo, plo, 0, 1), fb, cadd, false);
        cadd = __builtin_amdgcn_fdot2(__builtin_shufflevector(plo, plo, 2, 3), fb, cadd, false);
    }
    corr += cadd;
    // V^T operands: tiles t of token pairs (0,1) and (2,3).
    uint32_t a01[8], a23[8];
    if constexpr (FMT == KVQ_KV_INT4) {
        QFmt<KVQ_KV_INT4>::vpair_half(ch.v[0][0], ch.v[1][0], 0x05040100u, a01, k4);
        QFmt<KVQ_KV_INT4>::vpair_half(ch.v[0][0], ch.v[1][0], 0x07060302u, a01 + 4, k4);
        QFmt<KVQ_KV_INT4>::vpair_half(ch.v[2][0], ch.v[3][0], 0x05040100u, a23, k4);
        QFmt<KVQ_KV_INT4>::vpair_half(ch.v[2][0], ch.v[3][0], 0x07060302u, a23 + 4, k4);
    } else {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            Q::vpair(ch.v[0][k], ch.v[1][k], a01 + 4 * k);
            Q::vpair(ch.v[2][k], ch.v[3][k], a23 + 4 * k);
        }
    }
    if constexpr (SPLIT) {
        // column h takes p hi, column h + 8 p lo (the lanes of a pair hold the same p)
        const h4 pop = (__lane_id() & 8) ? plo : phi;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            u2 w = {a01[t], a23[t]};
            const h4 a = __builtin_bit_cast(h4, w);
            st.acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, pop, st.acc[t], 0, 0, 0);
        }
    } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            u2 w = {a01[t], a23[t]};
            const h4 a = __builtin_bit_cast(h4, w);
            st.acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, phi, st.acc[t], 0, 0, 0);
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            u2 w = {a01[t], a23[t]};
            const h4 a = __builtin_bit_cast(h4, w);
            st.acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, plo, st.acc[t], 0, 0, 0);
        }
    }
}

// P-deep register ring: chunk c + P is loaded while chunk c computes, the block-table
// entries of chunks c + 2P .. c + 3P - 1 meanwhile. Every chunk carries its own K group's
// scales, so any group size works with any P.
template <int FMT, int W, bool FINAL, int P, bool SPLIT>
__global__ __launch_bounds__(W * 64) void decode_q_kernel(const DecodeParams p) {
    typedef QFmt<FMT> Q;
    constexpr int D = 128, DV = 8;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kvh = blockIdx.x, split = blockIdx.y, b = blockIdx.z;
    const int i16 = lane & 15, g = lane >> 4;
    const int G = p.group;
    const bool head_ok = i16 < G;
    const WaveRange wr = wave_range<W>(p, b, split, wave);
    const int seq_len = wr.seq_len, w_lo = wr.w_lo, w_hi = wr.w_hi;
    const int kgs = p.k_group_shift;  // log2 of 16-token chunks per K group
    const I4Consts k4 = i4_consts();

    // q in this format's k-operand order (zero for padded heads), kept in LDS for the
    // once-per-K-group q' products: [4 k-steps][64 lanes] h8, written by wave 0.
    extern __shared__ float smem[];
    h8* qsh = (h8*)(smem + W * G * D + 2 * W * 16 + W * 128);
    if (wave == 0) {
        const _Float16* qrow = (const _Float16*)p.q + (int64_t)b * p.q_sb +
                               (int64_t)(kvh * G + (head_ok ? i16 : 0)) * p.q_sh;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            h8 x = *(const h8*)(qrow + Q::chan_base(st, g));
            if constexpr (Q::permuted()) x = __builtin_shufflevector(x, x, 0, 4, 1, 5, 2, 6, 3, 7);
            qsh[64 * st + lane] = head_ok ? x : (h8)(_Float16)0;
        }
    }
    __syncthreads();
    qsh += SPLIT ? (lane & ~8) : lane;  // SPLIT: columns h and h + 8 read head h

    SoftmaxState<D> st;
#pragma unroll
    for (int t = 0; t < DV; ++t) st.acc[t] = (f4)0.f;
    st.m = -INFINITY;
    st.l = 0.f;
    float corr = 0.f, cinit = 0.f;
    const float sl2f = p.scale_log2 * Q::F;
    h8 qhi[4], qlo[SPLIT ? 1 : 4];

    auto valid_of = [&](int c) { return min(seq_len - (c << 4), 16); };

    uint32_t* stage = (uint32_t*)(smem + W * G * D + 2 * W * 16) + wave * 128;
    // The ring covers the wave's fully valid chunks [w_lo, r_hi); the sequence's partial
    // last chunk (at most one per sequence) is handled once after it. Every load in the
    // ring is issued on every path (chunks past r_hi - 1 re-read chunk r_hi - 1 and are
    // never used), so each wait counts exactly the loads still in flight behind it.
    const int r_hi = min(w_hi, wr.c_full);
    const int gmask = (1 << kgs) - 1;
    if (w_lo < r_hi) {
        const QLaneOff lo = lane_offsets<FMT>(p, i16, g, 15);
        const int last = r_hi - 1;
        ChunkQ<FMT> ring[P];
        int pg_cur = chunk_pages<P>(p, b, w_lo, last, kgs);
        int pg_nxt = chunk_pages<P>(p, b, w_lo + P, last, kgs);
        // Issued slot by slot: a slot's loads moved behind a later slot's would make the
        // ring's waits (vmcnt counts the loads issued after the awaited one) drain it.
#pragma unroll
        for (int i = 0; i < P; ++i) {
            load_chunk_q<FMT>(p, kvh, min(w_lo + i, last), lo,
                              __builtin_amdgcn_readlane(pg_cur, i),
                              __builtin_amdgcn_readlane(pg_cur, P + i), ring[i]);
            __builtin_amdgcn_sched_barrier(0);
        }
        for (int c0 = w_lo; c0 < r_hi; c0 += P) {
            pg_cur = pg_nxt;  // pages of chunks c0 + P .. c0 + 2P - 1
            pg_nxt = chunk_pages<P>(p, b, c0 + 2 * P, last, kgs);
#pragma unroll
            for (int i = 0; i < P; ++i) {
                const int c = c0 + i;
                if (c < r_hi) {
                    if (c == w_lo || (c & gmask) == 0)
                        cinit = make_qprime<FMT, SPLIT>(ring[i].ks2, ring[i].kz2, stage, g, qsh, qhi, qlo);
                    chunk_q<FMT, false, SPLIT>(ring[i], qhi, qlo, cinit, sl2f, 16, g, st, corr, k4);
                }
                load_chunk_q<FMT>(p, kvh, min(c + P, last), lo,
                                  __builtin_amdgcn_readlane(pg_cur, i),
                                  __builtin_amdgcn_readlane(pg_cur, P + i), ring[i]);
            }
        }
    }
    if (w_lo <= r_hi && r_hi < w_hi) {  // this wave owns the partial last chunk c_full
        const int c = r_hi;
        const int valid = valid_of(c);
        const int pg = chunk_pages<1>(p, b, c, c, kgs);
        ChunkQ<FMT> ch;
        load_chunk_q<FMT>(p, kvh, c, lane_offsets<FMT>(p, i16, g, valid - 1),
                          __builtin_amdgcn_readlane(pg, 0), __builtin_amdgcn_readlane(pg, 1), ch);
        if (c == w_lo || (c & gmask) == 0)
            cinit = make_qprime<FMT, SPLIT>(ch.ks2, ch.kz2, stage, g, qsh, qhi, qlo);
        chunk_q<FMT, true, SPLIT>(ch, qhi, qlo, cinit, sl2f, valid, g, st, corr, k4);
    }

    if constexpr (SPLIT) {  // add the lo columns into the hi columns
#pragma unroll
        for (int t = 0; t < DV; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) st.acc[t][r] += ror8(st.acc[t][r]);
    }
    combine_store<D, W, FINAL>(p, st.acc, Q::F, rows_sum(corr), st.m, rows_sum(st.l), wave, i16,
                               g, kvh, split, b);
}

template <int FMT, int W, bool FINAL, int P, bool SPLIT>
static hipError_t launch_q(const DecodeParams& p, hipStream_t stream) {
    const dim3 grid(p.kv_heads, FINAL ? 1 : p.num_splits, p.batch);
    // cross-wave combine ([W][G][128] + [W][16] m, l), one 512-byte K-scale slot per wave,
    // then q in k-operand order (4 KB)
    const size_t shmem = sizeof(float) * (W * p.group * 128 + 2 * W * 16 + W * 128) + 4096;
    hipLaunchKernelGGL((decode_q_kernel<FMT, W, FINAL, P, SPLIT>), grid, dim3(W * 64), shmem,
                       stream, p);
    return hipGetLastError();
}

// Up to 8 heads per kv head: hi / lo parts in the two column halves of one MFMA chain,
// any ring depth. 9 to 16 heads: two chains, ring depth 4.
template <int FMT, bool FINAL, int P>
static hipError_t launch_q_w(const DecodeParams& p, int waves, hipStream_t stream) {
    if (p.group > 8) {
        switch (waves) {
            case 1: return launch_q<FMT, 1, FINAL, 4, false>(p, stream);
            case 2: return launch_q<FMT, 2, FINAL, 4, false>(p, stream);
            case 4: return launch_q<FMT, 4, FINAL, 4, false>(p, stream);
            case 8: return launch_q<FMT, 8, FINAL, 4, false>(p, stream);
            default: return hipErrorInvalidValue;
        }
    }
    switch (waves) {
        case 1: return launch_q<FMT, 1, FINAL, P, true>(p, stream);
        case 2: return launch_q<FMT, 2, FINAL, P, true>(p, stream);
        case 4: return launch_q<FMT, 4, FINAL, P, true>(p, stream);
        case 8: return launch_q<FMT, 8, FINAL, P, true>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

template <int FMT, bool FINAL>
static hipError_t launch_q_p(const DecodeParams& p, int waves, int ring, hipStream_t stream) {
    switch (ring) {
        case 1: return launch_q_w<FMT, FINAL, 1>(p, waves, stream);
        case 2: return launch_q_w<FMT, FINAL, 2>(p, waves, stream);
        case 4: return launch_q_w<FMT, FINAL, 4>(p, waves, stream);
        default: return hipErrorInvalidValue;
    }
}

template <int FMT>
static hipError_t launch_q_f(const DecodeParams& p, bool final_out, int waves, int ring,
                             hipStream_t stream) {
    return final_out ? launch_q_p<FMT, true>(p, waves, ring, stream)
                     : launch_q_p<FMT, false>(p, waves, ring, stream);
}

hipError_t launch_decode_q(const DecodeParams& p, int kv_format, int head_dim, bool final_out,
                           int waves, int ring, hipStream_t stream) {
    if (head_dim != 128) return hipErrorInvalidValue;
    switch (kv_format) {
        case KVQ_KV_INT8: return launch_q_f<KVQ_KV_INT8>(p, final_out, waves, ring, stream);
        case KVQ_KV_FP8_E4M3:
            return launch_q_f<KVQ_KV_FP8_E4M3>(p, final_out, waves, ring, stream);
        case KVQ_KV_INT4: return launch_q_f<KVQ_KV_INT4>(p, final_out, waves, ring, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace kvq
