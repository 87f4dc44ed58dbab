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
//     FP8   h = f(c)/256  (e4m3 sign/exponent/mantissa re-based into fp16; F = 256, B = 0)
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

// e4m3fn bytes placed at bits 8-15 / 24-31 (sign at 15 / 31) -> fp16 f(c) / 256:
// sign stays, exponent+mantissa (7 bits) move to fp16 bits 7-13.
__device__ __forceinline__ uint32_t f8_fix(uint32_t y) {
    return (y & 0x80008000u) | ((y >> 1) & 0x3F803F80u);
}

// Nibbles of one dword (byte j = codes 2j (low), 2j+1 (high)) -> 8 halves 1 + c/64 in the
// order codes {0,4, 1,5, 2,6, 3,7}.
__device__ __forceinline__ u4v i4_dword(uint32_t x) {
    u4v r;
    r[0] = ((x << 4) & kNib) | kMagicI4;
    r[1] = (x & kNib) | kMagicI4;
    r[2] = ((x >> 4) & kNib) | kMagicI4;
    r[3] = ((x >> 8) & kNib) | kMagicI4;
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
    __device__ static h8 kop(const u4v* kr, int st) {
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

template <>
struct QFmt<KVQ_KV_FP8_E4M3> {
    static constexpr float F = 256.f, B = 0.f;
    static constexpr int KLOADS = 2, VBYTES = 8;
    __device__ static int chan_base(int st, int g) { return 64 * (st >> 1) + 16 * g + 8 * (st & 1); }
    static constexpr bool permuted() { return false; }
    __device__ static h8 kop(const u4v* kr, int st) {
        const u4v x = kr[st >> 1];
        const uint32_t d0 = x[2 * (st & 1)], d1 = x[2 * (st & 1) + 1];
        u4v o;
        o[0] = f8_fix(perm(0u, d0, 0x010C000Cu));
        o[1] = f8_fix(perm(0u, d0, 0x030C020Cu));
        o[2] = f8_fix(perm(0u, d1, 0x010C000Cu));
        o[3] = f8_fix(perm(0u, d1, 0x030C020Cu));
        return __builtin_bit_cast(h8, o);
    }
    __device__ static void vpair(uint32_t a, uint32_t b, uint32_t* out4) {
        out4[0] = f8_fix(perm(b, a, 0x040C000Cu));
        out4[1] = f8_fix(perm(b, a, 0x050C010Cu));
        out4[2] = f8_fix(perm(b, a, 0x060C020Cu));
        out4[3] = f8_fix(perm(b, a, 0x070C030Cu));
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
    __device__ static h8 kop(const u4v* kr, int st) {
        return __builtin_bit_cast(h8, i4_dword(kr[0][st]));
    }
    // Tiles 0..3 (channels 0..3 of the lane's 8) or 4..7 of token pair (ra, rb) from the
    // dwords a, b holding each token's 8 codes.
    __device__ static void vpair_half(uint32_t a, uint32_t b, uint32_t sel, uint32_t* out4) {
        const uint32_t y = perm(b, a, sel);  // low 16 bits: ra's 4 codes, high: rb's
        out4[0] = ((y << 4) & kNib) | kMagicI4;
        out4[1] = (y & kNib) | kMagicI4;
        out4[2] = ((y >> 4) & kNib) | kMagicI4;
        out4[3] = ((y >> 8) & kNib) | kMagicI4;
    }
};

// Raw codes of one 16-token chunk as held by one lane, plus the 4 tokens' V scale/zero.
template <int FMT>
struct ChunkQ {
    u4v k[QFmt<FMT>::KLOADS];
    uint32_t v[4][QFmt<FMT>::VBYTES / 4];
    h4 vs, vz;
};

template <int FMT>
__device__ __forceinline__ void load_chunk_q(const DecodeParams& p, int b, int kvh, int c,
                                             int valid, int i16, int g, int n_pages,
                                             PageWindow& win, ChunkQ<FMT>& ch) {
    typedef QFmt<FMT> Q;
    const int page = c >> p.cpp_shift;
    const int slot = (c - (page << p.cpp_shift)) << 4;
    const int phys = window_phys(p, b, page, n_pages, win);
    const char* kb = (const char*)p.k + (int64_t)phys * p.k_sblk + (int64_t)slot * p.k_stok +
                     (int64_t)kvh * p.k_sh;
    const char* vb = (const char*)p.v + (int64_t)phys * p.v_sblk + (int64_t)slot * p.v_stok +
                     (int64_t)kvh * p.v_sh;
    const int last = valid - 1;
    const uint32_t koff = (uint32_t)(min(i16, last) * (int)p.k_stok + 16 * g);
#pragma unroll
    for (int j = 0; j < Q::KLOADS; ++j) ch.k[j] = *(const u4v*)(kb + koff + 64 * j);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t voff = (uint32_t)(min(4 * g + r, last) * (int)p.v_stok + Q::VBYTES * i16);
        if constexpr (Q::VBYTES == 8) {
            const u2 x = *(const u2*)(vb + voff);
            ch.v[r][0] = x[0];
            ch.v[r][Q::VBYTES / 4 - 1] = x[1];
        } else {
            ch.v[r][0] = *(const uint32_t*)(vb + voff);
        }
    }
    // V scale/zero of tokens slot + 4g .. +3 (4 consecutive halves; slots past the
    // sequence hold garbage and are masked in chunk_q).
    const int64_t vsz = ((int64_t)phys * p.kv_heads + kvh) * p.block_size + slot + 4 * g;
    ch.vs = *(const h4*)(p.v_scale + vsz);
    ch.vz = *(const h4*)(p.v_zero + vsz);
}

// Per-wave state of the quantized kernel beyond the softmax state: the q' operand of the
// current K group and its MFMA accumulator input.
struct KGroupState {
    int group;     // K scale group the operands belong to (-1 = none yet)
    float cinit;   // sum_d q z / F - B * sum_d q' of this lane's head column
};

// q' = q * s in fp16 would lose 2^-12 relative per channel - enough to move logits by
// ~1e-3 on outlier channels - so q' is kept as an unevaluated sum hi + lo of two fp16
// operands (hi = fp16(q s), lo = fp16(q s - hi); q s is exact in fp32), and the QK^T
// MFMA chain runs once per part. C uses the same hi + lo sums.
template <int FMT>
__device__ __forceinline__ void load_kgroup(const DecodeParams& p, int b, int kvh, int grp,
                                            int g, const h8* qop, h8* qhi, h8* qlo,
                                            KGroupState& ks) {
    typedef QFmt<FMT> Q;
    const int lead_page = grp * p.k_group_pages;
    int phys = p.bt[(int64_t)b * p.bt_sb + lead_page];
    phys = min(max(phys, 0), p.num_blocks - 1);
    const int64_t row = ((int64_t)phys * p.kv_heads + kvh) * 128;
    float qz = 0.f, qs = 0.f;
#pragma unroll
    for (int st = 0; st < 4; ++st) {
        h8 s = *(const h8*)(p.k_scale + row + Q::chan_base(st, g));
        h8 z = *(const h8*)(p.k_zero + row + Q::chan_base(st, g));
        if constexpr (Q::permuted()) {
            s = __builtin_shufflevector(s, s, 0, 4, 1, 5, 2, 6, 3, 7);
            z = __builtin_shufflevector(z, z, 0, 4, 1, 5, 2, 6, 3, 7);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float qe = (float)qop[st][e];
            const float prod = qe * (float)s[e];  // exact: 11-bit x 11-bit mantissas
            const _Float16 hi = (_Float16)prod;
            const _Float16 lo = (_Float16)(prod - (float)hi);
            qhi[st][e] = hi;
            qlo[st][e] = lo;
            qz += qe * (float)z[e];
            qs += (float)hi + (float)lo;
        }
    }
    qz = rows_sum(qz);
    qs = rows_sum(qs);
    ks.cinit = qz * (1.f / Q::F) - Q::B * qs;
    ks.group = grp;
}

template <int FMT, bool MASK>
__device__ __forceinline__ void chunk_q(const ChunkQ<FMT>& ch, const h8* qhi, const h8* qlo,
                                        float cinit, float sl2f, int valid, int g,
                                        SoftmaxState<128>& st, float& corr) {
    typedef QFmt<FMT> Q;
    f4 s = (f4)cinit;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const h8 kh = Q::kop(ch.k, k);
        s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qhi[k], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qlo[k], s, 0, 0, 0);
    }
    float s2[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) s2[r] = s[r] * sl2f;
    if (MASK) {
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
    // p'' = fp16(p * s_t) feeds the MFMA; corr accumulates p z - F B p'' in fp32.
    h4 pop;
    float cadd = 0.f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const bool ok = !MASK || 4 * g + r < valid;
        const _Float16 pp = ok ? (_Float16)(pr[r] * (float)ch.vs[r]) : (_Float16)0.f;
        pop[r] = pp;
        const float zt = ok ? (float)ch.vz[r] : 0.f;
        cadd += pr[r] * zt - (Q::F * Q::B) * (float)pp;
    }
    corr = corr * alpha + cadd;
    // V^T operands: tiles t of token pairs (0,1) and (2,3).
    uint32_t a01[8], a23[8];
    if constexpr (FMT == KVQ_KV_INT4) {
        QFmt<KVQ_KV_INT4>::vpair_half(ch.v[0][0], ch.v[1][0], 0x05040100u, a01);
        QFmt<KVQ_KV_INT4>::vpair_half(ch.v[0][0], ch.v[1][0], 0x07060302u, a01 + 4);
        QFmt<KVQ_KV_INT4>::vpair_half(ch.v[2][0], ch.v[3][0], 0x05040100u, a23);
        QFmt<KVQ_KV_INT4>::vpair_half(ch.v[2][0], ch.v[3][0], 0x07060302u, a23 + 4);
    } else {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            Q::vpair(ch.v[0][k], ch.v[1][k], a01 + 4 * k);
            Q::vpair(ch.v[2][k], ch.v[3][k], a23 + 4 * k);
        }
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
        u2 w = {a01[t], a23[t]};
        const h4 a = __builtin_bit_cast(h4, w);
        st.acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, pop, st.acc[t] * alpha, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    }
}

template <int FMT, int W, bool FINAL>
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
    const int seq_len = wr.seq_len, n_pages = wr.n_pages, w_lo = wr.w_lo, w_hi = wr.w_hi;

    // q in this format's k-operand order (zero for padded heads).
    h8 qop[4];
    {
        const _Float16* qrow = (const _Float16*)p.q + (int64_t)b * p.q_sb +
                               (int64_t)(kvh * G + (head_ok ? i16 : 0)) * p.q_sh;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            h8 x = *(const h8*)(qrow + Q::chan_base(st, g));
            if constexpr (Q::permuted()) x = __builtin_shufflevector(x, x, 0, 4, 1, 5, 2, 6, 3, 7);
            qop[st] = head_ok ? x : (h8)(_Float16)0;
        }
    }

    SoftmaxState<D> st;
#pragma unroll
    for (int t = 0; t < DV; ++t) st.acc[t] = (f4)0.f;
    st.m = -INFINITY;
    st.l = 0.f;
    float corr = 0.f;
    const float sl2f = p.scale_log2 * Q::F;
    KGroupState ks;
    ks.group = -1;
    ks.cinit = 0.f;
    h8 qhi[4], qlo[4];

    PageWindow win;
    window_load(p, b, w_lo >> p.cpp_shift, n_pages, win);
    for (int c = w_lo; c < w_hi; ++c) {
        const int grp = c / p.k_group_chunks;
        if (grp != ks.group) load_kgroup<FMT>(p, b, kvh, grp, g, qop, qhi, qlo, ks);
        const int valid = min(seq_len - (c << 4), 16);
        ChunkQ<FMT> ch;
        load_chunk_q<FMT>(p, b, kvh, c, valid, i16, g, n_pages, win, ch);
        if (valid == 16) chunk_q<FMT, false>(ch, qhi, qlo, ks.cinit, sl2f, 16, g, st, corr);
        else chunk_q<FMT, true>(ch, qhi, qlo, ks.cinit, sl2f, valid, g, st, corr);
    }

    combine_store<D, W, FINAL>(p, st.acc, Q::F, rows_sum(corr), st.m, rows_sum(st.l), wave, i16,
                               g, kvh, split, b);
}

template <int FMT, int W, bool FINAL>
static hipError_t launch_q(const DecodeParams& p, hipStream_t stream) {
    const dim3 grid(p.kv_heads, FINAL ? 1 : p.num_splits, p.batch);
    const size_t shmem = sizeof(float) * (W * p.group * 128 + 2 * W * 16);
    hipLaunchKernelGGL((decode_q_kernel<FMT, W, FINAL>), grid, dim3(W * 64), shmem, stream, p);
    return hipGetLastError();
}

template <int FMT, bool FINAL>
static hipError_t launch_q_w(const DecodeParams& p, int waves, hipStream_t stream) {
    switch (waves) {
        case 1: return launch_q<FMT, 1, FINAL>(p, stream);
        case 2: return launch_q<FMT, 2, FINAL>(p, stream);
        case 4: return launch_q<FMT, 4, FINAL>(p, stream);
        case 8: return launch_q<FMT, 8, FINAL>(p, stream);
        case 16: return launch_q<FMT, 16, FINAL>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

template <int FMT>
static hipError_t launch_q_f(const DecodeParams& p, bool final_out, int waves,
                             hipStream_t stream) {
    return final_out ? launch_q_w<FMT, true>(p, waves, stream)
                     : launch_q_w<FMT, false>(p, waves, stream);
}

hipError_t launch_decode_q(const DecodeParams& p, int kv_format, int head_dim, bool final_out,
                           int waves, hipStream_t stream) {
    if (head_dim != 128) return hipErrorInvalidValue;
    switch (kv_format) {
        case KVQ_KV_INT8: return launch_q_f<KVQ_KV_INT8>(p, final_out, waves, stream);
        case KVQ_KV_FP8_E4M3: return launch_q_f<KVQ_KV_FP8_E4M3>(p, final_out, waves, stream);
        case KVQ_KV_INT4: return launch_q_f<KVQ_KV_INT4>(p, final_out, waves, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace kvq
