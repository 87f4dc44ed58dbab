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
//         A = K: lane (tok = l%16, g = l/16) holds K[tok][32*st + 8*g + 0..7] - one 16-byte
//         load per k-step, 64 contiguous bytes per token row per instruction;
//         B = Q^T: the same k-mapping, heads >= group are zero padding.
//     online softmax on the C layout: lane holds S^T[4g + r][head l%16], r = 0..3;
//     O^T[D x 16 heads] += V^T[D x 16 tok] . P^T[16 tok x 16 heads]  D/16 x mfma 16x16x16
//         B = P^T is exactly the QK C layout (no data movement);
//         A = V^T: lane (i = l%16, g) needs V[4g + r][d] for one d per tile - it loads the
//         D/16 contiguous halves V[4g + r][(D/16)*i ...] of 4 token rows (16 lanes cover one
//         full 256-byte row) and transposes them in registers; tile t then holds
//         d = (D/16)*i + t, so the accumulator lane (head l%16, g) ends with
//         O[head][(D/16)*(4g + r) + t].
//   No LDS in the chunk loop. The running max is lazy (see kLazyMax), so the common chunk
//   has no cross-lane traffic at all; a max update uses two v_permlane swaps.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "decode_common.h"

namespace kvq {

// One 16-token chunk of one kv head, fp16 cache, as held by one lane.
template <int D>
struct ChunkF16 {
    static constexpr int NST = D / 32;
    static constexpr int DV = D / 16;
    typedef typename HalfVec<DV>::type vrow;
    h8 k[NST];
    vrow v[4];
};

// Loads chunk c (16 tokens of kv head kvh). `valid` = tokens of the chunk inside the
// sequence (16 except for its last chunk): rows past it are redirected to the last valid
// row, so unused page slots (whatever they hold) are never read; their scores are masked
// to -inf in chunk_f16. Addresses are a wave-uniform block base plus 32-bit lane offsets.
template <int D>
__device__ __forceinline__ void load_chunk_f16(const DecodeParams& p, int b, int kvh, int c,
                                               int valid, int i16, int g, int n_pages,
                                               PageWindow& win, ChunkF16<D>& ch) {
    constexpr int DV = D / 16;
    typedef typename ChunkF16<D>::vrow vrow;
    const int page = c >> p.cpp_shift;
    const int slot = (c - (page << p.cpp_shift)) << 4;
    const int phys = window_phys(p, b, page, n_pages, win);
    const char* kb = (const char*)p.k +
                     2 * ((int64_t)phys * p.k_sblk + (int64_t)slot * p.k_stok + (int64_t)kvh * p.k_sh);
    const char* vb = (const char*)p.v +
                     2 * ((int64_t)phys * p.v_sblk + (int64_t)slot * p.v_stok + (int64_t)kvh * p.v_sh);
    const int last = valid - 1;
    const uint32_t koff = (uint32_t)(min(i16, last) * (int)p.k_stok + 8 * g) * 2u;
#pragma unroll
    for (int st = 0; st < D / 32; ++st) ch.k[st] = *(const h8*)(kb + koff + 64 * st);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint32_t voff = (uint32_t)(min(4 * g + r, last) * (int)p.v_stok + DV * i16) * 2u;
        ch.v[r] = *(const vrow*)(vb + voff);
    }
}

// One chunk: QK^T, softmax update, PV. MASK handles the sequence's partial last chunk.
template <int D, bool MASK>
__device__ __forceinline__ void chunk_f16(const ChunkF16<D>& ch, const h8* qop, float sl2,
                                          int valid, int g, SoftmaxState<D>& st) {
    constexpr int NST = D / 32;
    constexpr int DV = D / 16;
    typedef typename ChunkF16<D>::vrow vrow;
    f4 s = (f4)0.f;
#pragma unroll
    for (int k = 0; k < NST; ++k)
        s = __builtin_amdgcn_mfma_f32_16x16x32_f16(ch.k[k], qop[k], s, 0, 0, 0);
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
        h4 a;
        a[0] = ch.v[0][t];
        a[1] = ch.v[1][t];
        a[2] = ch.v[2][t];
        a[3] = ch.v[3][t];
        st.acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, pop, st.acc[t] * alpha, 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    }
}

// PIPE = 2 keeps the next chunk's loads in flight while the current one computes (two
// chunks of registers, lower occupancy); PIPE = 1 relies on occupancy alone.
template <int D, int W, bool FINAL, int PIPE>
__global__ __launch_bounds__(W * 64)
void decode_f16_kernel(const DecodeParams p) {
    constexpr int NST = D / 32;
    constexpr int DV = D / 16;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kvh = blockIdx.x, split = blockIdx.y, b = blockIdx.z;
    const int i16 = lane & 15, g = lane >> 4;
    const int G = p.group;
    const bool head_ok = i16 < G;
    const WaveRange wr = wave_range<W>(p, b, split, wave);
    const int seq_len = wr.seq_len, n_pages = wr.n_pages, w_lo = wr.w_lo, w_hi = wr.w_hi;
    const int c_full = wr.c_full;

    // Q^T operand: lane (head i16, g) holds Q[head][32*k + 8*g + 0..7]; padded heads = 0.
    h8 qop[NST];
    {
        const _Float16* qrow = (const _Float16*)p.q + (int64_t)b * p.q_sb +
                               (int64_t)(kvh * G + (head_ok ? i16 : 0)) * p.q_sh + 8 * g;
#pragma unroll
        for (int k = 0; k < NST; ++k) {
            h8 x = *(const h8*)(qrow + 32 * k);
            qop[k] = head_ok ? x : (h8)(_Float16)0;
        }
    }

    SoftmaxState<D> st;
#pragma unroll
    for (int t = 0; t < DV; ++t) st.acc[t] = (f4)0.f;
    st.m = -INFINITY;
    st.l = 0.f;
    const float sl2 = p.scale_log2;

    PageWindow win;
    window_load(p, b, w_lo >> p.cpp_shift, n_pages, win);
    auto valid_of = [&](int c) { return min(seq_len - (c << 4), 16); };

    if (PIPE == 2) {
        // Two-deep register pipeline: chunk c+1's loads are in flight while c computes.
        ChunkF16<D> ca, cb;
        int c = w_lo;
        if (c < w_hi) load_chunk_f16<D>(p, b, kvh, c, valid_of(c), i16, g, n_pages, win, ca);
        while (c < w_hi) {
            if (c + 1 < w_hi)
                load_chunk_f16<D>(p, b, kvh, c + 1, valid_of(c + 1), i16, g, n_pages, win, cb);
            if (c < c_full) chunk_f16<D, false>(ca, qop, sl2, 16, g, st);
            else chunk_f16<D, true>(ca, qop, sl2, seq_len - (c << 4), g, st);
            if (++c >= w_hi) break;
            if (c + 1 < w_hi)
                load_chunk_f16<D>(p, b, kvh, c + 1, valid_of(c + 1), i16, g, n_pages, win, ca);
            if (c < c_full) chunk_f16<D, false>(cb, qop, sl2, 16, g, st);
            else chunk_f16<D, true>(cb, qop, sl2, seq_len - (c << 4), g, st);
            ++c;
        }
    } else {
        for (int c = w_lo; c < w_hi; ++c) {
            ChunkF16<D> ch;
            load_chunk_f16<D>(p, b, kvh, c, valid_of(c), i16, g, n_pages, win, ch);
            if (c < c_full) chunk_f16<D, false>(ch, qop, sl2, 16, g, st);
            else chunk_f16<D, true>(ch, qop, sl2, seq_len - (c << 4), g, st);
        }
    }

    combine_store<D, W, FINAL>(p, st.acc, 1.f, 0.f, st.m, rows_sum(st.l), wave, i16, g, kvh,
                               split, b);
}

// Stage 2 (reference _merge_kernel, triton_fp16.py:147-163): one workgroup of 256 threads
// per (q head, sequence) = 8 groups of 32 threads; a thread owns D/32 consecutive columns
// and its group folds splits g, g+8, ... First the global max of lse (every thread scans
// all splits: S floats, cache-resident), so the weighted sum needs no rescaling and its
// loads are independent; then the 8 groups are summed through LDS.
template <int D>
__global__ __launch_bounds__(256) void merge_kernel(const float* __restrict__ o_part,
                                                    const float* __restrict__ lse,
                                                    _Float16* __restrict__ out, int64_t o_sb,
                                                    int64_t o_sh, int q_heads, int S) {
    constexpr int PER = D / 32;  // columns per thread (1..8)
    const int hq = blockIdx.x, b = blockIdx.y;
    const int t = threadIdx.x, lane32 = t & 31, grp = t >> 5;
    const int64_t row0 = ((int64_t)b * q_heads + hq) * S;
    const float* L = lse + row0;
    float M = -INFINITY;
    for (int s = 0; s < S; ++s) M = fmaxf(M, L[s]);
    float wsum = 0.f;
    float acc[PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) acc[e] = 0.f;
    if (M > -INFINITY) {
#pragma unroll 4
        for (int s = grp; s < S; s += 8) {
            const float w = fast_exp2((L[s] - M) * kLog2e);
            const float* src = o_part + (row0 + s) * D + lane32 * PER;
            wsum += w;
#pragma unroll
            for (int e = 0; e < PER; ++e) acc[e] += w * src[e];
        }
    }
    __shared__ float sm_acc[8][D];
    __shared__ float sm_w[8];
#pragma unroll
    for (int e = 0; e < PER; ++e) sm_acc[grp][lane32 * PER + e] = acc[e];
    if (lane32 == 0) sm_w[grp] = wsum;
    __syncthreads();
    for (int d = t; d < D; d += 256) {
        float o = 0.f, W = 0.f;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            o += sm_acc[g][d];
            W += sm_w[g];
        }
        out[(int64_t)b * o_sb + (int64_t)hq * o_sh + d] = (_Float16)(W > 0.f ? o / W : 0.f);
    }
}

template <int D, int W, bool FINAL, int PIPE>
static hipError_t launch_f16(const DecodeParams& p, hipStream_t stream) {
    const dim3 grid(p.kv_heads, FINAL ? 1 : p.num_splits, p.batch);
    const size_t shmem = sizeof(float) * (W * p.group * D + 2 * W * 16);
    hipLaunchKernelGGL((decode_f16_kernel<D, W, FINAL, PIPE>), grid, dim3(W * 64), shmem, stream,
                       p);
    return hipGetLastError();
}

template <int D, bool FINAL, int PIPE>
static hipError_t launch_f16_w(const DecodeParams& p, int waves, hipStream_t stream) {
    switch (waves) {
        case 1: return launch_f16<D, 1, FINAL, PIPE>(p, stream);
        case 2: return launch_f16<D, 2, FINAL, PIPE>(p, stream);
        case 4: return launch_f16<D, 4, FINAL, PIPE>(p, stream);
        case 8: return launch_f16<D, 8, FINAL, PIPE>(p, stream);
        case 16: return launch_f16<D, 16, FINAL, PIPE>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

template <int D>
static hipError_t launch_f16_d(const DecodeParams& p, bool final_out, int waves, int pipe,
                               hipStream_t stream) {
    if (pipe == 2)
        return final_out ? launch_f16_w<D, true, 2>(p, waves, stream)
                         : launch_f16_w<D, false, 2>(p, waves, stream);
    return final_out ? launch_f16_w<D, true, 1>(p, waves, stream)
                     : launch_f16_w<D, false, 1>(p, waves, stream);
}

hipError_t launch_decode(const DecodeParams& p, int kv_format, int head_dim, bool final_out,
                         int waves, int pipe, hipStream_t stream) {
    if (kv_format != KVQ_KV_F16)
        return launch_decode_q(p, kv_format, head_dim, final_out, waves, pipe, stream);
    switch (head_dim) {
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
