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
// rint rounds half to even; division is IEEE (correctly rounded); no contraction.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "kvq_internal.h"

#pragma clang fp contract(off)

namespace kvq {

namespace {

constexpr float kFp8Max = 448.f;

__device__ __forceinline__ int clampi(int v, int lo, int hi) { return min(max(v, lo), hi); }

// float32 -> e4m3fn bits, round to nearest even, |t| <= 448 (callers clamp first).
__device__ __forceinline__ uint32_t e4m3fn_rne(float t) {
    const uint32_t sign = (__float_as_uint(t) >> 31) << 7;
    const float a = fabsf(t);
    uint32_t bits;
    if (a < 0.015625f) {  // below 2^-6: subnormal m * 2^-9, m = 8 carries to 2^-6
        bits = (uint32_t)__builtin_rintf(a * 512.f);
    } else {
        int e = (int)((__float_as_uint(a) >> 23) & 0xFF) - 127;
        const float frac = a * __uint_as_float((uint32_t)(127 - e) << 23) - 1.f;  // [0, 1)
        int m = (int)__builtin_rintf(frac * 8.f);
        if (m == 8) {
            m = 0;
            ++e;
        }
        bits = ((uint32_t)(e + 7) << 3) | (uint32_t)m;
    }
    return bits | sign;
}

struct ScaleZero {
    float s, z;  // fp16 values held in fp32
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
    return r;
}

template <int FMT>
__device__ __forceinline__ uint32_t encode(float x, ScaleZero p) {
    if (p.s == 0.f) return 0u;
    const float t = __fdiv_rn(x - p.z, p.s);
    if (FMT == KVQ_KV_FP8_E4M3) return e4m3fn_rne(fminf(fmaxf(t, -kFp8Max), kFp8Max));
    const float R = FMT == KVQ_KV_INT4 ? 15.f : 255.f;
    return (uint32_t)__builtin_rintf(fminf(fmaxf(t, 0.f), R));
}

__device__ __forceinline__ int phys_of(const QuantParams& p, int b, int page) {
    return clampi(p.bt[(int64_t)b * p.bt_sb + page], 0, p.num_blocks - 1);
}

__device__ __forceinline__ int seq_len_of(const QuantParams& p, int b) {
    return clampi(p.seq_lens[b], 0, p.max_blocks * p.block_size);
}

// Codes of two adjacent channels (2j, 2j+1) of one token row.
template <int FMT>
__device__ __forceinline__ void store_pair(uint8_t* row, int j, uint32_t c0, uint32_t c1) {
    if (FMT == KVQ_KV_INT4) {
        row[j] = (uint8_t)(c0 | (c1 << 4));
    } else {
        *(uint16_t*)(row + 2 * j) = (uint16_t)(c0 | (c1 << 8));
    }
}

// K: per (kv head, group, sequence), 256 threads: thread (j, ts) owns channels 2j, 2j+1
// (j < D/2) of the group's rows t0 + ts, t0 + ts + TS, ... (TS = 512 / D row slices).
// Pass 1 reduces min / max over each slice, then across the slices through LDS; pass 2
// encodes the slice's rows with the group's (scale, zero). Codes go to each token's page
// slot, the pairs to the group's first block. Append: the group holding the newest token,
// read from the fp16 residual except the new row itself (from k_new), which also joins
// the residual for later appends.
template <int FMT, bool APPEND>
__global__ __launch_bounds__(256) void quant_k_kernel(const QuantParams p) {
    const int kvh = blockIdx.x, grp = blockIdx.y, b = blockIdx.z;
    const int D = p.head_dim;
    const int TS = 512 / D;                // row slices
    const int j = threadIdx.x % (D / 2), ts = threadIdx.x / (D / 2);
    const int n = seq_len_of(p, b);
    int t0 = grp * p.k_group, t1 = min(t0 + p.k_group, n);
    if (APPEND) {  // only the group holding the newest token, rows 0..(n-1) % k_group
        if (n < 1) return;
        t0 = ((n - 1) / p.k_group) * p.k_group;
        t1 = n;
    }
    if (t0 >= t1) return;  // uniform over the workgroup
    const int64_t resid = ((int64_t)b * p.kv_heads + kvh) * p.k_group * D;
    const _Float16* kn = p.k_new + ((int64_t)b * p.kv_heads + kvh) * D + 2 * j;
    if (APPEND && ts == 0) {  // the new token's K joins the fp16 residual of its group
        _Float16* dst = p.k_resid + resid + (int64_t)(t1 - 1 - t0) * D + 2 * j;
        dst[0] = kn[0];
        dst[1] = kn[1];
    }
    auto load = [&](int t, float& x0, float& x1) {
        const _Float16* src;
        if (APPEND) {
            src = t == t1 - 1 ? kn : p.k_resid + resid + (int64_t)(t - t0) * D + 2 * j;
        } else {
            const int phys = phys_of(p, b, t / p.block_size);
            src = p.k_src + (int64_t)phys * p.s_sblk + (int64_t)(t % p.block_size) * p.s_stok +
                  (int64_t)kvh * p.s_sh + 2 * j;
        }
        x0 = (float)src[0];
        x1 = (float)src[1];
    };
    float mn0 = INFINITY, mx0 = -INFINITY, mn1 = INFINITY, mx1 = -INFINITY;
#pragma unroll 8
    for (int t = t0 + ts; t < t1; t += TS) {
        float x0, x1;
        load(t, x0, x1);
        mn0 = fminf(mn0, x0);
        mx0 = fmaxf(mx0, x0);
        mn1 = fminf(mn1, x1);
        mx1 = fmaxf(mx1, x1);
    }
    __shared__ float4 part[256];       // per thread: (mn0, mx0, mn1, mx1)
    __shared__ float4 params[128];     // per channel pair: (s0, z0, s1, z1)
    part[threadIdx.x] = make_float4(mn0, mx0, mn1, mx1);
    __syncthreads();
    if (ts == 0) {
        for (int k = 1; k < TS; ++k) {
            const float4 o = part[k * (D / 2) + j];
            mn0 = fminf(mn0, o.x);
            mx0 = fmaxf(mx0, o.y);
            mn1 = fminf(mn1, o.z);
            mx1 = fmaxf(mx1, o.w);
        }
        const ScaleZero q0 = make_params<FMT>(mn0, mx0), q1 = make_params<FMT>(mn1, mx1);
        params[j] = make_float4(q0.s, q0.z, q1.s, q1.z);
        // (scale, zero) pairs of channels 2j, 2j + 1: one 8-byte store
        const int lead = phys_of(p, b, t0 / p.block_size);
        const int64_t sz = ((int64_t)lead * p.kv_heads + kvh) * D + 2 * j;
        typedef _Float16 h4q __attribute__((ext_vector_type(4)));
        const h4q pairs = {(_Float16)q0.s, (_Float16)q0.z, (_Float16)q1.s, (_Float16)q1.z};
        *(h4q*)(p.k_scale + 2 * sz) = pairs;
    }
    __syncthreads();
    const float4 pr = params[j];
    const ScaleZero q0 = {pr.x, pr.y}, q1 = {pr.z, pr.w};
#pragma unroll 8
    for (int t = t0 + ts; t < t1; t += TS) {
        float x0, x1;
        load(t, x0, x1);
        const int phys = phys_of(p, b, t / p.block_size);
        uint8_t* row = p.k_codes + (int64_t)phys * p.k_sblk +
                       (int64_t)(t % p.block_size) * p.k_stok + (int64_t)kvh * p.k_sh;
        store_pair<FMT>(row, j, encode<FMT>(x0, q0), encode<FMT>(x1, q1));
    }
}

// V: one token row (D channels of one kv head) per 16 lanes, each lane D/16 channels.
// Bulk: workgroup = 16 token rows of one (kv head, sequence); append: the newest token.
template <int FMT, int D, bool APPEND>
__global__ __launch_bounds__(256) void quant_v_kernel(const QuantParams p) {
    constexpr int PER = D / 16;
    const int kvh = blockIdx.x, b = blockIdx.z;
    const int lane16 = threadIdx.x & 15;
    const int n = seq_len_of(p, b);
    int t = blockIdx.y * 16 + (threadIdx.x >> 4);
    if (APPEND) t = threadIdx.x < 16 ? n - 1 : -1;
    if (t < 0 || t >= n) return;
    const int phys = phys_of(p, b, t / p.block_size);
    const int slot = t % p.block_size;
    const _Float16* src =
        APPEND ? p.v_new + ((int64_t)b * p.kv_heads + kvh) * D
               : p.v_src + (int64_t)phys * p.s_sblk + (int64_t)slot * p.s_stok + (int64_t)kvh * p.s_sh;
    float x[PER];
    float mn = INFINITY, mx = -INFINITY;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        x[e] = (float)src[lane16 * PER + e];
        mn = fminf(mn, x[e]);
        mx = fmaxf(mx, x[e]);
    }
    // min / max over the row's 16 lanes (lanes of a row are contiguous within the wave)
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
        mn = fminf(mn, __shfl_xor(mn, o, 16));
        mx = fmaxf(mx, __shfl_xor(mx, o, 16));
    }
    const ScaleZero q = make_params<FMT>(mn, mx);
    uint8_t* row = p.v_codes + (int64_t)phys * p.v_sblk + (int64_t)slot * p.v_stok +
                   (int64_t)kvh * p.v_sh;
#pragma unroll
    for (int e = 0; e < PER; e += 2)
        store_pair<FMT>(row, (lane16 * PER + e) / 2, encode<FMT>(x[e], q), encode<FMT>(x[e + 1], q));
    if (lane16 == 0) {
        const int64_t sz = ((int64_t)phys * p.kv_heads + kvh) * p.block_size + slot;
        typedef _Float16 h2q __attribute__((ext_vector_type(2)));
        *(h2q*)(p.v_scale + 2 * sz) = h2q{(_Float16)q.s, (_Float16)q.z};
    }
}

template <int FMT, bool APPEND>
hipError_t launch_fmt(const QuantParams& p, hipStream_t stream) {
    const int groups = APPEND ? 1 : p.max_groups;
    hipLaunchKernelGGL((quant_k_kernel<FMT, APPEND>), dim3(p.kv_heads, groups, p.batch),
                       dim3(256), 0, stream, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int tok_wgs = APPEND ? 1 : (p.max_blocks * p.block_size + 15) / 16;
    const dim3 vgrid(p.kv_heads, tok_wgs, p.batch);
    const dim3 vblock(APPEND ? 16 : 256);
    switch (p.head_dim) {
        case 32: hipLaunchKernelGGL((quant_v_kernel<FMT, 32, APPEND>), vgrid, vblock, 0, stream, p); break;
        case 64: hipLaunchKernelGGL((quant_v_kernel<FMT, 64, APPEND>), vgrid, vblock, 0, stream, p); break;
        case 128: hipLaunchKernelGGL((quant_v_kernel<FMT, 128, APPEND>), vgrid, vblock, 0, stream, p); break;
        case 256: hipLaunchKernelGGL((quant_v_kernel<FMT, 256, APPEND>), vgrid, vblock, 0, stream, p); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
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
