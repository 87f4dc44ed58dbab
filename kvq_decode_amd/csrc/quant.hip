// KIVI quantization of the paged KV cache for gfx950: bulk (prefill) and on-append
// (decode). No reference code exists for this (README.md:16 "not started"); the format
// follows the reference's byte model (src/bpt/roofline.py:6-9): asymmetric fp16 scale and
// zero, K per channel over groups of k_group tokens, V per token. Every code must be
// bit-exact with the float32 specification, so the arithmetic below is spelled out one
// IEEE operation at a time, in the spec's order:
//   integer b bits, R = 2^b - 1: s = fp16((max - min) / R), z = fp16(min),
//       c = s == 0 ? 0 : clamp(rint((x - z) / s), 0, R)
//   fp8 e4m3fn, E = 448: z = fp16((max + min) * 0.5), s = fp16((max - min) / (2E)),
//       c = s == 0 ? 0x00 : e4m3fn_rne(clamp((x - z) / s, -E, E))
// rint rounds half to even; division is IEEE (correctly rounded, computed as in
// quotient()); no contraction.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "kvq_internal.h"

#pragma clang fp contract(off)

namespace kvq {

namespace {

constexpr float kFp8Max = 448.f;

__device__ __forceinline__ int clampi(int v, int lo, int hi) { return min(max(v, lo), hi); }

typedef short s2q __attribute__((ext_vector_type(2)));

// float32 -> OCP e4m3fn bits, round to nearest even, for |t| <= 448 (callers clamp
// first): the hardware conversion at scale 1. It equals the spec's software encode
// (mantissa rounded half to even at 2^(e-3), subnormals at 2^-9) on every fp32 value of
// [-448, 448], checked exhaustively on MI355X (tests/gpu_checks/fp8_encode_check.hip).
__device__ __forceinline__ uint32_t e4m3fn_rne(float t) {
    const s2q r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(s2q{0, 0}, t, 0.f, 1.0f, false);
    return __builtin_bit_cast(uint32_t, r) & 0xFFu;
}

struct ScaleZero {
    float s, z;  // fp16 values held in fp32
    float r;     // RN(1 / s), 0 when s == 0
};

template <int FMT>
__device__ __forceinline__ ScaleZero make_params(float mn, float mx) {
    ScaleZero r;
    if (FMT == KVQ_KV_FP8_E4M3) {
        const float mid = (mx + mn) * 0.5f;
        r.z = (float)(_Float16)mid;
        r.s = (float)(_Float16)__fdiv_rn(mx - mn, 2.f * kFp8Max);
    } else {
        const float R = FMT == KVQ_KV_INT4 ? 15.f : 255.f;
        r.s = (float)(_Float16)__fdiv_rn(mx - mn, R);
        r.z = (float)(_Float16)mn;
    }
    r.r = r.s == 0.f ? 0.f : __fdiv_rn(1.f, r.s);
    return r;
}

// RN(d / s) for d = fl(x - z) of fp16 x, z (0 or |d| >= 2^-24) and a positive fp16 s, from
// the correctly rounded reciprocal r: q = RN(d r), the exact remainder d - s q by fma, and
// one fma correction (Markstein's theorem; its exceptions need a divisor significand of 24
// ones, and s has 11 significant bits). Checked bit-identical to IEEE division on every
// finite fp16 s against random and near-multiple d.
__device__ __forceinline__ float quotient(float d, ScaleZero p) {
    const float q = d * p.r;
    const float rem = __builtin_fmaf(-q, p.s, d);
    return __builtin_fmaf(rem, p.r, q);
}

template <int FMT>
__device__ __forceinline__ uint32_t encode(float x, ScaleZero p) {
    if (p.s == 0.f) return 0u;
    const float t = quotient(x - p.z, p);
    if (FMT == KVQ_KV_FP8_E4M3) return e4m3fn_rne(fminf(fmaxf(t, -kFp8Max), kFp8Max));
    const float R = FMT == KVQ_KV_INT4 ? 15.f : 255.f;
    return (uint32_t)__builtin_rintf(fminf(fmaxf(t, 0.f), R));
}

// Physical block of page `page` of sequence b, or -1 when the block-table entry lies
// outside [0, num_blocks). The write paths neither read nor write a row whose page is
// outside the pool (the fp16 append skips such slots the same way), so a bad table entry
// cannot redirect codes or pairs into another sequence's block.
__device__ __forceinline__ int phys_of(const QuantParams& p, int b, int page) {
    const int e = p.bt[(int64_t)b * p.bt_sb + page];
    return (e >= 0 && e < p.num_blocks) ? e : -1;
}

// Tokens of sequence b the bulk quantizer covers: seq_lens[b], limited to the slots its
// block-table row addresses.
__device__ __forceinline__ int seq_len_of(const QuantParams& p, int b) {
    return clampi(p.seq_lens[b], 0, p.max_blocks * p.block_size);
}

// The append's sequence length: seq_lens[b] counts the new token, at position
// seq_lens[b] - 1. A length below 1 or past the block table's last slot has no slot for
// that token; the append then writes nothing for the sequence (-1).
__device__ __forceinline__ int append_len_of(const QuantParams& p, int b) {
    const int n = p.seq_lens[b];
    return (n >= 1 && n <= p.max_blocks * p.block_size) ? n : -1;
}

typedef _Float16 h8q __attribute__((ext_vector_type(8)));
typedef _Float16 h4q __attribute__((ext_vector_type(4)));
typedef _Float16 h2q __attribute__((ext_vector_type(2)));

// A lane's 8 channels of one row, converted to float.
__device__ __forceinline__ void to_float8(h8q v, float* x) {
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (float)v[e];
}

// Codes of 8 consecutive channels 8c .. 8c + 7 of one token row, in one store: INT4 4
// bytes (low nibble = even channel), INT8 / FP8 8 bytes. The row's code offset 8c (INT4:
// 4c) is 4-byte (8-byte) aligned because code rows are 16-byte aligned.
template <int FMT>
__device__ __forceinline__ void store8(uint8_t* row, int c, const uint32_t* code) {
    if (FMT == KVQ_KV_INT4) {
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) w |= code[e] << (4 * e);
        *(uint32_t*)(row + 4 * c) = w;
    } else {
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            lo |= code[e] << (8 * e);
            hi |= code[4 + e] << (8 * e);
        }
        typedef uint32_t u2q __attribute__((ext_vector_type(2)));
        *(u2q*)(row + 8 * c) = u2q{lo, hi};
    }
}

// Codes of one row's 8 channels 8c .. 8c + 7 under (scale, zero) q, into the row's page
// slot (phys: its block).
template <int FMT>
__device__ __forceinline__ void emit_k_row(const QuantParams& p, int kvh, int c, int t,
                                           int phys, h8q v, const ScaleZero* q) {
    float x[8];
    to_float8(v, x);
    uint32_t code[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) code[e] = encode<FMT>(x[e], q[e]);
    store8<FMT>(p.k_codes + (int64_t)phys * p.k_sblk + (int64_t)(t & (p.block_size - 1)) * p.k_stok +
                    (int64_t)kvh * p.k_sh,
                c, code);
}

// Min / max over aligned lane groups without LDS (exact operations, so the order of the
// combination does not change the result): within a 16-lane row by DPP - quad_perm xor 1
// and xor 2; row_half_mirror, where each quad already holds its own result, so lane i
// meeting lane 7 - i combines the two quads of a half; row_ror:8 - and across rows by
// v_permlane16_swap / v_permlane32_swap (xor 16 / xor 32), whose two results are the lane's
// own value and its partner's.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
template <int O>  // xor lane offset 1, 2, 4 (within 8-lane halves), 8, 16 or 32
__device__ __forceinline__ void minmax_xor(float& mn, float& mx) {
    if constexpr (O == 16 || O == 32) {
        const auto a = O == 16 ? __builtin_amdgcn_permlane16_swap(__float_as_uint(mn), __float_as_uint(mn), false, false)
                               : __builtin_amdgcn_permlane32_swap(__float_as_uint(mn), __float_as_uint(mn), false, false);
        const auto b = O == 16 ? __builtin_amdgcn_permlane16_swap(__float_as_uint(mx), __float_as_uint(mx), false, false)
                               : __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
        mn = fminf(__uint_as_float(a[0]), __uint_as_float(a[1]));
        mx = fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
    } else {
        constexpr int CTRL = O == 1 ? 0xB1 : O == 2 ? 0x4E : O == 4 ? 0x141 : 0x128;
        mn = fminf(mn, dpp<CTRL>(mn));
        mx = fmaxf(mx, dpp<CTRL>(mx));
    }
}

// K, bulk: one wave per (kv head, group, sequence), four groups per 256-thread workgroup.
// Lane l owns channels 8c .. 8c + 7 (c = l % PC, PC = D/8 lanes per row: 16-byte loads) of
// rows t0 + RPI j + l / PC (RPI = 64/PC rows per load instruction). Min / max run over the
// lane's rows in registers, then across the RPI row groups of a channel by lane exchanges:
// no LDS and no barrier. The lane's first KC rows stay in registers between the min / max
// pass and the encode pass (every row of a 128-token group at head dims up to 128); longer
// groups re-read the rest. Codes go to each token's page slot, the pairs to the group's
// first block. Rows whose page lies outside the pool are neither read nor written, so they
// do not enter the group's min / max; a group whose first page lies outside the pool
// writes nothing.
template <int FMT, int D>
__device__ __forceinline__ void quant_k_group(const QuantParams& p, int kvh, int grp, int b) {
    constexpr int PC = D / 8, RPI = 64 / PC, KC = D == 256 ? 16 : 32;
    const int lane = threadIdx.x & 63, c = lane % PC, ri = lane / PC;
    const int n = seq_len_of(p, b);
    const int t0 = grp * p.k_group, t1 = min(t0 + p.k_group, n);
    if (t0 >= t1) return;  // uniform over the wave
    // the group's (scale, zero) pairs live in its first page: without it the group's codes
    // could not be read back, so a group whose first page is outside the pool writes nothing
    const int lead = phys_of(p, b, t0 >> p.bs_shift);
    if (lead < 0) return;
    // row t of the group, from the page `phys` holding it
    auto load = [&](int t, int phys) -> h8q {
        return *(const h8q*)(p.k_src + (int64_t)phys * p.s_sblk +
                             (int64_t)(t & (p.block_size - 1)) * p.s_stok + (int64_t)kvh * p.s_sh +
                             8 * c);
    };
    float mn[8], mx[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        mn[e] = INFINITY;
        mx[e] = -INFINITY;
    }
    auto reduce = [&](h8q v) {
        float x[8];
        to_float8(v, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            mn[e] = fminf(mn[e], x[e]);
            mx[e] = fmaxf(mx[e], x[e]);
        }
    };
    h8q cache[KC];
    int cphys[KC];  // the cached rows' pages (-1: outside the pool or past the group)
#pragma unroll
    for (int i = 0; i < KC; ++i) {  // every load issued, at rows inside the pool
        const int t = t0 + ri + i * RPI;
        const int ph = phys_of(p, b, min(t, t1 - 1) >> p.bs_shift);
        cphys[i] = t < t1 ? ph : -1;
        cache[i] = load(min(t, t1 - 1), ph >= 0 ? ph : lead);
    }
#pragma unroll
    for (int i = 0; i < KC; ++i)
        if (cphys[i] >= 0) reduce(cache[i]);
    for (int t = t0 + ri + KC * RPI; t < t1; t += RPI) {
        const int phys = phys_of(p, b, t >> p.bs_shift);
        if (phys >= 0) reduce(load(t, phys));
    }
    // the channel's RPI row groups: lanes c, c + PC, c + 2 PC, ...
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        if constexpr (PC <= 8) minmax_xor<8>(mn[e], mx[e]);
        if constexpr (PC <= 16) minmax_xor<16>(mn[e], mx[e]);
        minmax_xor<32>(mn[e], mx[e]);
    }
    ScaleZero q[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) q[e] = make_params<FMT>(mn[e], mx[e]);
    if (ri == 0) {
        // (scale, zero) pairs of channels 8c .. 8c + 7: two 16-byte stores into the lead
        // page, which also holds row t0, so min / max saw at least that row
        h8q pairs[2];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            pairs[e / 4][2 * (e % 4)] = (_Float16)q[e].s;
            pairs[e / 4][2 * (e % 4) + 1] = (_Float16)q[e].z;
        }
        const int64_t sz = ((int64_t)lead * p.kv_heads + kvh) * D + 8 * c;
        *(h8q*)(p.k_scale + 2 * sz) = pairs[0];
        *(h8q*)(p.k_scale + 2 * sz + 8) = pairs[1];
    }
#pragma unroll
    for (int i = 0; i < KC; ++i)
        if (cphys[i] >= 0) emit_k_row<FMT>(p, kvh, c, t0 + ri + i * RPI, cphys[i], cache[i], q);
    for (int t = t0 + ri + KC * RPI; t < t1; t += RPI) {
        const int phys = phys_of(p, b, t >> p.bs_shift);
        if (phys >= 0) emit_k_row<FMT>(p, kvh, c, t, phys, load(t, phys), q);
    }
}

// V: one token row (D channels of one kv head) per D/8 lanes, each lane 8 channels (one
// 16-byte load, one 4- or 8-byte code store). Bulk: workgroup = kVRows token rows of one
// (kv head, sequence), 256 threads; append: the newest token, on the first D/8 lanes of
// the append kernel's V workgroup. The codes go to the token's page slot, its (scale,
// zero) pair to index t % VG of its V group's first page (VG = 2^vg_shift tokens); a row
// is written only when both pages lie in the pool.
constexpr int kVRows = 64;

template <int FMT, int D, bool APPEND>
__device__ __forceinline__ void quant_v_rows(const QuantParams& p, int kvh, int tile, int b) {
    constexpr int LPR = D / 8, RPP = 256 / LPR;  // lanes per row, rows per pass
    constexpr int PASSES = APPEND ? 1 : kVRows / RPP;
    const int c = threadIdx.x % LPR;
    const int n = APPEND ? append_len_of(p, b) : seq_len_of(p, b);
    // every pass's row is loaded first, so the workgroup waits on memory once. A row past
    // the sequence or in a page outside the pool is neither read nor written (tok = -1).
    int tok[PASSES], phys[PASSES], vlead[PASSES];
    h8q row[PASSES];
#pragma unroll
    for (int i = 0; i < PASSES; ++i) {
        tok[i] = APPEND ? n - 1 : tile * kVRows + i * RPP + threadIdx.x / LPR;
        if (tok[i] < 0 || tok[i] >= n) {  // whole rows (LPR-lane groups) skip together
            tok[i] = -1;
            continue;
        }
        phys[i] = phys_of(p, b, tok[i] >> p.bs_shift);
        vlead[i] = phys_of(p, b, (tok[i] >> p.vg_shift) << (p.vg_shift - p.bs_shift));
        if (phys[i] < 0 || vlead[i] < 0) {
            tok[i] = -1;
            continue;
        }
        const _Float16* src =
            APPEND ? p.v_new + ((int64_t)b * p.kv_heads + kvh) * D + 8 * c
                   : p.v_src + (int64_t)phys[i] * p.s_sblk + (int64_t)(tok[i] & (p.block_size - 1)) * p.s_stok +
                         (int64_t)kvh * p.s_sh + 8 * c;
        row[i] = *(const h8q*)src;
    }
#pragma unroll
    for (int i = 0; i < PASSES; ++i) {
        if (tok[i] < 0) continue;
        const int slot = tok[i] & (p.block_size - 1);
        float x[8];
        to_float8(row[i], x);
        float mn = x[0], mx = x[0];
#pragma unroll
        for (int e = 1; e < 8; ++e) {
            mn = fminf(mn, x[e]);
            mx = fmaxf(mx, x[e]);
        }
        // min / max over the row's LPR lanes (aligned lane groups of one wave)
        minmax_xor<1>(mn, mx);
        minmax_xor<2>(mn, mx);
        minmax_xor<4>(mn, mx);
        if constexpr (LPR >= 16) minmax_xor<8>(mn, mx);
        if constexpr (LPR >= 32) minmax_xor<16>(mn, mx);
        const ScaleZero q = make_params<FMT>(mn, mx);
        uint32_t code[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) code[e] = encode<FMT>(x[e], q);
        store8<FMT>(p.v_codes + (int64_t)phys[i] * p.v_sblk + (int64_t)slot * p.v_stok +
                        (int64_t)kvh * p.v_sh,
                    c, code);
        if (c == 0) {
            const int64_t sz = (((int64_t)vlead[i] * p.kv_heads + kvh) << p.vg_shift) +
                               (tok[i] & ((1 << p.vg_shift) - 1));
            *(h2q*)(p.v_scale + 2 * sz) = h2q{(_Float16)q.s, (_Float16)q.z};
        }
    }
}

// Append, K: the group holding the newest token (position n - 1, row r = (n - 1) % k_group
// of the group that starts at t0). The residual [B][Hkv][k_group + 2][D] keeps the
// group's fp16 rows and, in rows k_group and k_group + 1, their running per-channel min
// and max (exact in fp16: min / max of fp16 values). Lane (c, slice) of the 256-thread
// workgroup owns channels 8c .. 8c + 7; every lane loads the new row and its channels'
// stored min / max together with the sequence length (none of them depends on it), so
// the group's new (scale, zero) pairs are known one memory round trip in (r == 0 starts the
// group from the new row alone). The new row is encoded with them. The group's earlier
// rows are re-encoded only in the 8-channel slices whose min or max moved (a code depends
// on its row and its channel's pair only), by the slice's 2048 / D lanes; in a full
// 128-token group a new token moves about 2 of 128 channels' ranges. The slice's first lane
// writes the pairs (when they moved), the min / max rows and the new residual row. A group
// whose first page lies outside the pool writes nothing; rows whose page lies outside are
// not written. Appends are sequential: the residual holds rows 0 .. r - 1 of the group and
// their min / max (from the appends of positions t0 .. n - 2, or from init_k_residual).
template <int FMT, int D>
__device__ __forceinline__ void quant_k_append(const QuantParams& p, int kvh, int b) {
    constexpr int LPR = D / 8, RS = 256 / LPR, CACHE = 8;
    const int c = threadIdx.x % LPR, rs = threadIdx.x / LPR;
    const int64_t head = (int64_t)b * p.kv_heads + kvh;
    _Float16* res = p.k_resid + head * (p.k_group + 2) * D + 8 * c;  // row 0, this lane's channels
    const h8q kn = *(const h8q*)(p.k_new + head * D + 8 * c);
    const h8q smn = *(const h8q*)(res + (int64_t)p.k_group * D);
    const h8q smx = *(const h8q*)(res + (int64_t)(p.k_group + 1) * D);
    const int n = append_len_of(p, b);
    if (n < 1) return;
    const int t0 = ((n - 1) / p.k_group) * p.k_group, r = n - 1 - t0;
    const int lead = phys_of(p, b, t0 >> p.bs_shift);
    if (lead < 0) return;  // uniform over the workgroup
    const int phys_new = phys_of(p, b, (n - 1) >> p.bs_shift);
    float x[8], mn[8], mx[8];
    to_float8(kn, x);
    bool moved = r == 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float omn = r == 0 ? INFINITY : (float)smn[e];
        const float omx = r == 0 ? -INFINITY : (float)smx[e];
        mn[e] = fminf(omn, x[e]);
        mx[e] = fmaxf(omx, x[e]);
        moved = moved || mn[e] != omn || mx[e] != omx;
    }
    ScaleZero q[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) q[e] = make_params<FMT>(mn[e], mx[e]);
    if (moved) {  // re-encode rows 0 .. r - 1 of these channels: lane slice rs takes rows rs + k RS
        for (int base = 0; base < r; base += RS * CACHE) {
            h8q rows[CACHE];
            int ph[CACHE];
#pragma unroll
            for (int i = 0; i < CACHE; ++i) {  // loads first, at clamped rows (r >= 1 here)
                const int t = min(base + rs + i * RS, r - 1);
                ph[i] = phys_of(p, b, (t0 + t) >> p.bs_shift);
                rows[i] = *(const h8q*)(res + (int64_t)t * D);
            }
#pragma unroll
            for (int i = 0; i < CACHE; ++i) {
                const int t = base + rs + i * RS;
                if (t < r && ph[i] >= 0) emit_k_row<FMT>(p, kvh, c, t0 + t, ph[i], rows[i], q);
            }
        }
    }
    if (rs == 0) {
        if (phys_new >= 0) emit_k_row<FMT>(p, kvh, c, n - 1, phys_new, kn, q);
        h8q nmn, nmx;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            nmn[e] = (_Float16)mn[e];
            nmx[e] = (_Float16)mx[e];
        }
        *(h8q*)(res + (int64_t)r * D) = kn;
        *(h8q*)(res + (int64_t)p.k_group * D) = nmn;
        *(h8q*)(res + (int64_t)(p.k_group + 1) * D) = nmx;
        if (moved) {  // (scale, zero) pairs of channels 8c .. 8c + 7, in the group's first page
            h8q pairs[2];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                pairs[e / 4][2 * (e % 4)] = (_Float16)q[e].s;
                pairs[e / 4][2 * (e % 4) + 1] = (_Float16)q[e].z;
            }
            const int64_t sz = ((int64_t)lead * p.kv_heads + kvh) * D + 8 * c;
            *(h8q*)(p.k_scale + 2 * sz) = pairs[0];
            *(h8q*)(p.k_scale + 2 * sz + 8) = pairs[1];
        }
    }
}

template <int FMT, int D>
__global__ __launch_bounds__(256) void quant_k_kernel(const QuantParams p) {
    // grid (kv_heads * cdiv(groups, 4), batch): the groups of a sequence need no 16-bit grid
    // axis; wave w takes group 4 x + w (groups past the sequence return at once)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    quant_k_group<FMT, D>(p, blockIdx.x % p.kv_heads, 4 * (blockIdx.x / p.kv_heads) + wave,
                          blockIdx.y);
}

template <int FMT, int D>
__global__ __launch_bounds__(256) void quant_v_kernel(const QuantParams p) {
    // grid (kv_heads * row tiles, batch)
    quant_v_rows<FMT, D, false>(p, blockIdx.x % p.kv_heads, blockIdx.x / p.kv_heads,
                                blockIdx.y);
}

// Append in one launch: workgroup (kv head, role, sequence), role 0 re-quantizes the K
// group holding the newest token, role 1 (its first D/8 lanes) quantizes the newest V row.
// The two roles write disjoint memory (K codes, pairs and residual; V codes and pairs).
template <int FMT, int D>
__global__ __launch_bounds__(256) void quant_append_kernel(const QuantParams p) {
    if (blockIdx.y == 0) {
        quant_k_append<FMT, D>(p, blockIdx.x, blockIdx.z);
    } else if (threadIdx.x < D / 8) {
        quant_v_rows<FMT, D, true>(p, blockIdx.x, 0, blockIdx.z);
    }
}

template <int FMT, int D, bool APPEND>
hipError_t launch_fmt_d(const QuantParams& p, hipStream_t stream) {
    if (APPEND) {
        hipLaunchKernelGGL((quant_append_kernel<FMT, D>), dim3(p.kv_heads, 2, p.batch),
                           dim3(256), 0, stream, p);
        return hipGetLastError();
    }
    hipLaunchKernelGGL((quant_k_kernel<FMT, D>),
                       dim3(p.kv_heads * ((p.max_groups + 3) / 4), p.batch), dim3(256), 0,
                       stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int tiles = (int)(((int64_t)p.max_blocks * p.block_size + kVRows - 1) / kVRows);
    hipLaunchKernelGGL((quant_v_kernel<FMT, D>), dim3(p.kv_heads * tiles, p.batch), dim3(256),
                       0, stream, p);
    return hipGetLastError();
}

template <int FMT, bool APPEND>
hipError_t launch_fmt(const QuantParams& p, hipStream_t stream) {
    switch (p.head_dim) {  // the quantized formats' head dims (decode reads these)
        case 64: return launch_fmt_d<FMT, 64, APPEND>(p, stream);
        case 128: return launch_fmt_d<FMT, 128, APPEND>(p, stream);
        case 256: return launch_fmt_d<FMT, 256, APPEND>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

template <bool APPEND>
hipError_t launch_any(const QuantParams& p, int kv_format, hipStream_t stream) {
    switch (kv_format) {
        case KVQ_KV_INT8: return launch_fmt<KVQ_KV_INT8, APPEND>(p, stream);
        case KVQ_KV_FP8_E4M3: return launch_fmt<KVQ_KV_FP8_E4M3, APPEND>(p, stream);
        case KVQ_KV_INT4: return launch_fmt<KVQ_KV_INT4, APPEND>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_quantize_cache(const QuantParams& p, int kv_format, hipStream_t stream) {
    return launch_any<false>(p, kv_format, stream);
}

hipError_t launch_quantize_append(const QuantParams& p, int kv_format, hipStream_t stream) {
    return launch_any<true>(p, kv_format, stream);
}

}  // namespace kvq
