// Device helpers shared by the fp16 and the quantized decode kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "kvq_internal.h"

namespace kvq {

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

template <int N>
struct HalfVec {
    typedef _Float16 type __attribute__((ext_vector_type(N)));
};

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

__device__ __forceinline__ int cdiv(int a, int b) { return (a + b - 1) / b; }

// Reductions across the four 16-lane rows of a wave64 without LDS: gfx950's
// v_permlane{16,32}_swap exchange rows between two registers; combining both halves of
// the swap gives every lane the reduction over the row pair.
__device__ __forceinline__ float rows_max(float v) {
    const unsigned u = __float_as_uint(v);
    auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const unsigned w = __float_as_uint(v);
    auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float rows_sum(float v) {
    const unsigned u = __float_as_uint(v);
    auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const unsigned w = __float_as_uint(v);
    auto b = __builtin_amdgcn_permlane32_swap(w, w, false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Lazy running max: the exponent reference m of a head column moves only when a score
// exceeds it by more than kLazyMax (log2 units), so p = 2^(s - m) <= 2^kLazyMax (256,
// exact in fp16 up to its usual rounding). Numerator and denominator share m, so the
// result is unchanged; the common chunk needs no cross-lane max and no rescale.
constexpr float kLazyMax = 8.0f;

// Physical blocks of the P chunks c .. c + P - 1 (lane j < P), of the first pages of
// their K groups (lane P + j, groups of 2^gshift chunks) and of the first pages of their
// V (scale, zero) groups (lane 2P + j, 2^vshift chunks), chunks clamped to `last` so the
// load is issued on every path. Used one ring ahead: the compiler's wait for this
// register then counts the chunk loads issued since, and never drains the loads in flight.
//
// chunk_pages_raw is the block-table load alone (c >= 0 and last >= 0 keep it inside the
// sequence's table row), clamp_page the clamp of an entry into the pool; a caller that
// issues the load ahead of its use applies the clamp at the use.
template <int P>
__device__ __forceinline__ int chunk_pages_raw(const DecodeParams& p, int b, int c, int last,
                                               int gshift, int vshift) {
    static_assert(4 * P <= 64, "three lane regions of P chunks in one wave");
    const int j = __lane_id() & (4 * P - 1);
    int cj = min(c + (j & (P - 1)), last);
    if (j >= 2 * P) {
        cj = (cj >> vshift) << vshift;
    } else if (j >= P) {
        cj = (cj >> gshift) << gshift;
    }
    return p.bt[(int64_t)b * p.bt_sb + (cj >> p.cpp_shift)];
}

__device__ __forceinline__ int clamp_page(const DecodeParams& p, int phys) {
    return min(max(phys, 0), p.num_blocks - 1);
}

template <int P>
__device__ __forceinline__ int chunk_pages(const DecodeParams& p, int b, int c, int last,
                                           int gshift, int vshift) {
    return clamp_page(p, chunk_pages_raw<P>(p, b, c, last, gshift, vshift));
}

// Buffer resource for raw (untyped) loads at a wave-uniform base: stride 0, no range
// limit that matters (2^31 bytes), dword data format. Loads through it take a 32-bit lane
// offset in a VGPR and a wave-uniform offset in an SGPR, so a page's address needs no
// per-lane 64-bit arithmetic.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rsrc(const void* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff,
                                             0x00020000);
}

// byte offset of physical block `phys` for a block stride below 2^32 bytes (checked on the
// host): one 32 x 32 -> 64-bit scalar multiply
__device__ __forceinline__ uint64_t block_offset(int phys, int64_t stride) {
    return (uint64_t)(uint32_t)phys * (uint32_t)stride;
}

// The caches' kv head that the kernels' kv head `kvh` reads (DecodeParams::kv_rep).
__device__ __forceinline__ int cache_head(const DecodeParams& p, int kvh) {
    return p.kv_rep == 1 ? kvh : kvh / p.kv_rep;
}

// XCD-aware workgroup order. MI355X dispatches the workgroups of a launch to its 8 XCDs
// round-robin by linear id, and each XCD has its own L2. The decode kernels run a 1-D grid
// and map its ids to (kv head, split, sequence) units (U = splits * batch of them) in one
// of two orders, chosen by the host (DecodeParams::xcd_group):
//   plain:   id = kvh + kv_heads * u, the kv heads of a unit spread over the XCDs (fp16
//            at head dims of 64 and more, whose heads share no cache lines);
//   grouped: every kv head of a unit on one XCD, back to back, so that a line they share
//            (fp16 at head dims 16 and 32, whose token-major rows put 4 or 2 heads in one
//            128-byte line; the quantized caches) is fetched by one L2. With a split count
//            that is a multiple of 8, split s of sequence b runs on
//            XCD (s + b) % 8 - a sequence's early splits, the ones short sequences have,
//            land on different XCDs for different sequences; otherwise unit u runs on XCD
//            u % 8 (U rounded up to a multiple of 8; workgroups past the last unit exit).
// Fewer than 8 units always take the plain order, which spreads them over all XCDs.
constexpr int kXcds = 8;

struct WgCoord {
    int kvh, split, b;
    bool live;
};

__device__ __forceinline__ WgCoord wg_coord(const DecodeParams& p, int splits) {
    const int i = blockIdx.x;
    WgCoord c;
    if (!p.xcd_group || splits * p.batch < kXcds) {
        c.kvh = i % p.kv_heads;
        const int u = i / p.kv_heads;
        c.split = u % splits;
        c.b = u / splits;
    } else {
        const int x = i % kXcds, q = i / kXcds;
        c.kvh = q % p.kv_heads;
        const int j = q / p.kv_heads;
        if (splits % kXcds == 0) {
            const int per = splits / kXcds;
            c.b = j / per;
            c.split = ((x - c.b) & (kXcds - 1)) + kXcds * (j % per);
        } else {
            const int u = j * kXcds + x;
            c.split = u % splits;
            c.b = u / splits;
        }
    }
    c.live = c.b < p.batch;
    return c;
}

// Workgroups of the 1-D decode grid (see wg_coord).
inline unsigned decode_grid(bool xcd_group, int kv_heads, int splits, int batch) {
    const long u = (long)splits * batch;
    const long units = (!xcd_group || u < kXcds) ? u : (u + kXcds - 1) / kXcds * kXcds;
    return (unsigned)(units * kv_heads);
}

// Online-softmax state of one wave: running reference max m and partial sum l of its
// lane (head l%16, tokens 4g..4g+3 of every chunk), and O^T accumulator tiles.
template <int D>
struct SoftmaxState {
    f4 acc[D / 16];
    float m, l;
};

// Combines the W waves of a workgroup through LDS and writes the split's result.
// Each wave passes its O^T tiles (lane = head l%16, rows 4g..4g+3 of every tile), which
// hold acc_scale * acc + corr after the per-format correction, its column's reference max
// m and its column sum l. LDS: [W][G][D] accumulators then [W][16] m and l.
// FINAL writes o / l in fp16 to p.out (single pass); otherwise the normalized partial to
// o_part and its natural-log LSE to lse (stage 1, reference triton_fp16.py:138-143),
// with o = 0, lse = -inf for an empty split. The partial of q head h goes to row
// part_base + h * part_stride of [rows][D] o_part / [rows] lse (split-KV: part_base =
// b * q_heads * num_splits + split, part_stride = num_splits; units: see UnitSpace).
template <int D, int W, bool FINAL>
__device__ __forceinline__ void combine_store(const DecodeParams& p, const f4* acc,
                                              float acc_scale, float corr, float m, float l,
                                              int wave, int i16, int g, int kvh, int b,
                                              int64_t part_base, int64_t part_stride) {
    constexpr int DV = D / 16;
    const int G = p.group;
    extern __shared__ __attribute__((aligned(16))) float smem[];
    float* sm_acc = smem;
    float* sm_m = smem + W * G * D;
    float* sm_l = sm_m + W * 16;
    if (i16 < G) {
        float* dst = sm_acc + (wave * G + i16) * D;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
            for (int t = 0; t < DV; ++t) dst[DV * (4 * g + r) + t] = acc_scale * acc[t][r] + corr;
        }
        if (g == 0) {
            sm_m[wave * 16 + i16] = m;
            sm_l[wave * 16 + i16] = l;
        }
    }
    __syncthreads();

    const int hq0 = kvh * G;
    for (int idx = threadIdx.x; idx < G * D; idx += W * 64) {
        const int hh = idx / D, d = idx - hh * D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < W; ++w) M = fmaxf(M, sm_m[w * 16 + hh]);
        float L = 0.f, O = 0.f;
        if (M > -INFINITY) {
#pragma unroll
            for (int w = 0; w < W; ++w) {
                const float e = fast_exp2(sm_m[w * 16 + hh] - M);
                L += e * sm_l[w * 16 + hh];
                O += e * sm_acc[(w * G + hh) * D + d];
            }
        }
        const float o = L > 0.f ? O / L : 0.f;
        if (FINAL) {
            _Float16* out = (_Float16*)p.out + (int64_t)b * p.o_sb + (int64_t)(hq0 + hh) * p.o_sh;
            out[d] = (_Float16)o;
        } else {
            const int64_t row = part_base + (int64_t)(hq0 + hh) * part_stride;
            p.o_part[row * D + d] = o;
            if (d == 0) p.lse[row] = L > 0.f ? (M + __builtin_amdgcn_logf(L)) * kLn2 : -INFINITY;
        }
    }
}

// Partial rows of split `split` of sequence b in the split-KV layout [B][Hq][S][D].
__device__ __forceinline__ int64_t split_part_base(const DecodeParams& p, int b, int split) {
    return (int64_t)b * p.q_heads * p.num_splits + split;
}

// Work units (DecodeParams::units > 0). The 16-token chunks of one kv head, flattened
// over the batch, are cut into NU equal ranges: sequence b holds chunks [P_b, P_b + n_b)
// (n_b = cdiv(len_b, 16), P_b = n_0 + ... + n_(b-1), N = P_B) and unit u covers
// [floor(u N / NU), floor((u + 1) N / NU)), NU = min(units, N), so no unit is empty. A
// unit's workgroup takes the sequences its range overlaps, one segment each, whatever the
// lengths are: ragged batches balance as well as uniform ones. The partial of segment
// (u, b) is row u + b of its q head: a sequence's segments lie in consecutive units, so
// its rows are consecutive, and rows of different sequences never collide (a later
// sequence's first unit is at least the earlier one's last). Per q head there are at most
// NU + B - 1 rows; o_part is [Hq][units + B][D] and lse [Hq][units + B]. B is at most
// kUnitMaxBatch (checked on the host).
struct UnitSpace {
    int N, NU;
};

// First chunk of unit u, and the unit holding chunk x (the largest u with lo(u) <= x).
// The products take 64 bits, but they fit in 32 for all but the largest partitions (u N <
// 2^32), and the 32-bit quotient (a short float-reciprocal sequence) is taken then: the
// 64-bit one is a long software routine that the kernels' start would wait on. The
// branch is uniform (u, x and the partition are the same for the whole workgroup).
__device__ __forceinline__ int unit_lo(UnitSpace us, int u) {
    const uint64_t n = (uint64_t)(uint32_t)u * (uint32_t)us.N;
    if ((n >> 32) == 0) return (int)((uint32_t)n / (uint32_t)us.NU);
    return (int)(n / (uint32_t)us.NU);
}
__device__ __forceinline__ int unit_of(UnitSpace us, int64_t x) {
    const uint64_t n = (uint64_t)(x + 1) * (uint32_t)us.NU + (uint32_t)(us.N - 1);
    if ((n >> 32) == 0) return (int)((uint32_t)n / (uint32_t)us.N) - 1;
    return (int)(n / (uint32_t)us.N) - 1;
}

__device__ __forceinline__ int wave_sum(int x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
    return x;
}

// LDS of the work-unit driver: the chunk prefix P_0 .. P_B and the clamped lengths. Its
// size is a multiple of 16 bytes, so the dynamic LDS after it stays aligned for the
// 128-bit accesses of the staging tiles.
struct __attribute__((aligned(16))) UnitLds {
    int pref[kUnitMaxBatch + 4];
    int len[kUnitMaxBatch];
};

// The chunk prefix of the batch, lane t of one wave taking sequences per * t .. + per - 1
// (per <= PER) whose seq_lens are raw[0 .. per - 1]: pref[b] = P_b, pref[B] = N, len[b] =
// the clamped length.
template <int PER>
__device__ __forceinline__ void unit_prefix_scan(const DecodeParams& p, const int* raw,
                                                 int* pref, int* len_out, int t, int per) {
    const int B = p.batch, cap = p.max_blocks * p.block_size;
    int n[PER], local = 0;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        const int b = per * t + e;
        const bool mine = e < per && b < B;
        const int len = mine ? min(max(raw[e], 0), cap) : 0;
        if (mine) len_out[b] = len;
        n[e] = cdiv(len, 16);
        local += n[e];
    }
    int incl = local;  // inclusive scan over the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o);
        if (t >= o) incl += y;
    }
    int run = incl - local;
#pragma unroll
    for (int e = 0; e < PER; ++e) {
        const int b = per * t + e;
        if (e < per && b < B) pref[b] = run;
        run += n[e];
    }
    if (t == 63) pref[B] = incl;
}

// The same, loading the seq_lens first: all PER loads before any use (clamped indices,
// no branch between a load and the next).
template <int PER>
__device__ __forceinline__ void unit_prefix(const DecodeParams& p, int* pref, int* len_out,
                                            int t, int per) {
    int raw[PER];
#pragma unroll
    for (int e = 0; e < PER; ++e) raw[e] = p.seq_lens[min(per * t + e, p.batch - 1)];
    unit_prefix_scan<PER>(p, raw, pref, len_out, t, per);
}

// The calling wave's share of its unit's first segment in the partition where every
// sequence fills its block-table row (n_b = max_blocks * block_size / 16 for all b, so
// P_b = b * n_b): what for_unit_segments computes from the scanned prefix whenever every
// sequence of the batch has that chunk count. `live` is false for a unit past that
// partition's last (its fields then describe the last unit's share, inside the batch).
struct SegGuess {
    int b, seq_len, w_lo, w_hi;
    bool live;
};

template <int W>
__device__ __forceinline__ SegGuess unit_guess(const DecodeParams& p, int u, int wave) {
    const int cap = p.max_blocks * p.block_size;  // a multiple of 16
    const int ng = cap >> 4;
    UnitSpace ug;
    ug.N = p.batch * ng;  // the host checks batch * cdiv(cap, 16) <= INT32_MAX
    ug.NU = min(p.units, ug.N);
    SegGuess g;
    g.live = u < ug.NU;
    const int uu = min(u, ug.NU - 1);
    const int lo = unit_lo(ug, uu), hi = unit_lo(ug, uu + 1);
    g.b = lo / ng;
    const int p0 = g.b * ng;
    const int c_lo = lo - p0, c_hi = min(hi - p0, ng);
    const int per = cdiv(c_hi - c_lo, W);
    g.w_lo = min(c_lo + wave * per, c_hi);
    g.w_hi = min(g.w_lo + per, c_hi);
    g.seq_len = cap;
    return g;
}

// Makes the kernel arguments the start of a work-unit kernel reads available in SGPRs at
// this point. The compiler otherwise issues each argument load in the block that first
// uses it, and the start then waits on several dependent scalar-load round trips before
// its first memory access; loaded together they take one. (An empty asm statement with
// SGPR inputs: it emits no instruction.)
__device__ __forceinline__ void load_unit_args(const DecodeParams& p) {
    asm volatile("" ::"s"(p.q), "s"(p.q_sb), "s"(p.q_sh), "s"(p.bt), "s"(p.bt_sb),
                 "s"(p.seq_lens));
    asm volatile("" ::"s"(p.batch), "s"(p.kv_heads), "s"(p.group), "s"(p.block_size),
                 "s"(p.max_blocks), "s"(p.xcd_group), "s"(p.units), "s"(p.kv_rep),
                 "s"(p.cpp_shift));
}

// Runs fn(kvh, b, seq_len, w_lo, w_hi, part_base, part_stride, pf, first) for each segment
// of this workgroup's unit (workgroup = (kv head, unit), W waves), in batch order, with a
// barrier between segments (they reuse the LDS of the range functions). [w_lo, w_hi) is
// the calling wave's contiguous share of the segment's chunks.
//
// The segments come from the batch's chunk prefix, and a segment's first loads (q,
// block-table entries) depend on it. Two things keep that off the critical path:
// * every wave first calls pf = pre(kvh, guess) with its unit_guess share, which issues
//   those loads for the segment of the partition where every sequence has the table's
//   chunk count, without using them; fn gets pf and first = true for the unit's first
//   segment, and uses what matches the real one;
// * for batches of up to 256 sequences every wave loads its lanes' seq_lens together with
//   them, and when every sequence has that chunk count (a ballot) the prefix is the closed
//   form P_b = b * n: the wave computes its segments from registers, with no scan, LDS
//   table, barrier or search before its first chunk. Otherwise wave 0 scans the lengths
//   into an LDS prefix table that every wave then searches.
//
// Workgroup order: plain (kv head fastest), or with xcd_group and units a multiple of
// kXcds, grouped so that the kv heads of one unit share an XCD (workgroup i runs on XCD
// i % kXcds) and with it the L2 lines of the V scales, which interleave kv heads.
template <int W, typename Pre, typename Fn>
__device__ __forceinline__ void for_unit_segments(const DecodeParams& p, Pre&& pre, Fn&& fn) {
    load_unit_args(p);
    __shared__ UnitLds s;
    int kvh, u;
    if (p.xcd_group && p.units % kXcds == 0) {
        const int q = blockIdx.x / kXcds;
        kvh = q % p.kv_heads;
        u = (q / p.kv_heads) * kXcds + blockIdx.x % kXcds;
    } else {
        kvh = blockIdx.x % p.kv_heads;
        u = blockIdx.x / p.kv_heads;
    }
    const int t = threadIdx.x, B = p.batch, lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int per = (B + 63) >> 6;
    const int cap = p.max_blocks * p.block_size, ng = cap >> 4;  // cap: a multiple of 16
    // the lengths are loaded before the prefetch, which may wait on its own loads
    int raw[4];
    if (per <= 4) {  // lane t: sequences per * t .. per * t + per - 1
#pragma unroll
        for (int e = 0; e < 4; ++e) raw[e] = p.seq_lens[min(per * lane + e, B - 1)];
    }
    const auto pf = pre(kvh, unit_guess<W>(p, u, wave));
    bool uniform = false;
    if (per <= 4) {
        bool ok = true;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (e < per && per * lane + e < B) ok = ok && cdiv(min(max(raw[e], 0), cap), 16) == ng;
        uniform = __ballot(!ok) == 0;
    }
    // The unit's chunk range [lo, hi) and its first sequence b: from the closed form, or
    // from wave 0's LDS prefix table after a barrier (the branch is uniform over the
    // workgroup: every wave's ballot saw the same lengths). One segment loop serves both,
    // so the range function is inlined once.
    UnitSpace us;
    int b = 0;
    if (uniform) {  // P_b = b * ng, N = B * ng (the host checks B * ng <= INT32_MAX)
        us.N = B * ng;
    } else {
        if (t < 64) {
            if (per <= 4)  // batches up to 256: the short scan, over the lengths loaded above
                unit_prefix_scan<4>(p, raw, s.pref, s.len, t, per);
            else
                unit_prefix<kUnitMaxBatch / 64>(p, s.pref, s.len, t, per);
        }
        __syncthreads();
        us.N = __builtin_amdgcn_readfirstlane(s.pref[B]);
    }
    us.NU = min(p.units, us.N);
    if (u >= us.NU) return;
    const int lo = unit_lo(us, u), hi = unit_lo(us, u + 1);
    if (uniform) {
        b = lo / ng;
    } else {  // the sequence holding chunk lo: the largest b with P_b <= lo (P_B = N > lo)
        int top = B;
        while (top - b > 1) {
            const int mid = (b + top) >> 1;
            if (__builtin_amdgcn_readfirstlane(s.pref[mid]) <= lo) b = mid;
            else top = mid;
        }
    }
    bool first = true;
    for (; b < B; ++b) {
        int p0, p1, len;
        if (uniform) {
            p0 = b * ng;
            p1 = p0 + ng;
            // b's length: element b % per of lane b / per
            const int L = b / per, e = b - L * per;
            int v = raw[0];
            v = e == 1 ? raw[1] : v;
            v = e == 2 ? raw[2] : v;
            v = e == 3 ? raw[3] : v;
            len = min(max(__builtin_amdgcn_readlane(v, L), 0), cap);
        } else {
            p0 = __builtin_amdgcn_readfirstlane(s.pref[b]);
            p1 = __builtin_amdgcn_readfirstlane(s.pref[b + 1]);
            len = __builtin_amdgcn_readfirstlane(s.len[b]);
        }
        if (p0 >= hi) break;
        const int c_lo = max(lo, p0) - p0, c_hi = min(hi, p1) - p0;
        if (c_lo >= c_hi) continue;  // an empty sequence
        const int cnt = cdiv(c_hi - c_lo, W);
        const int w_lo = min(c_lo + wave * cnt, c_hi), w_hi = min(w_lo + cnt, c_hi);
        fn(kvh, b, len, w_lo, w_hi, (int64_t)u + b, (int64_t)p.units + B, pf, first);
        first = false;
        __syncthreads();
    }
}

// Without loads ahead: fn(kvh, b, seq_len, w_lo, w_hi, part_base, part_stride).
struct NoPrefetch {};

template <int W, typename Fn>
__device__ __forceinline__ void for_unit_segments(const DecodeParams& p, Fn&& fn) {
    for_unit_segments<W>(
        p, [](int, const SegGuess&) { return NoPrefetch{}; },
        [&](int kvh, int b, int seq_len, int w_lo, int w_hi, int64_t base, int64_t stride,
            const NoPrefetch&, bool) { fn(kvh, b, seq_len, w_lo, w_hi, base, stride); });
}

// The chunk range [w_lo, w_hi) of one wave: split `split` of the sequence covers pages
// [split * pps, min((split + 1) * pps, cdiv(seq_len, block_size))) (reference
// triton_fp16.py:114-116), cut into 16-token chunks, cut into W contiguous runs.
struct WaveRange {
    int seq_len, w_lo, w_hi;
};

template <int W>
__device__ __forceinline__ WaveRange wave_range(const DecodeParams& p, int b, int split,
                                                int wave) {
    WaveRange r;
    int seq_len = p.seq_lens[b];
    seq_len = min(max(seq_len, 0), p.max_blocks * p.block_size);
    r.seq_len = seq_len;
    const int n_pages = cdiv(seq_len, p.block_size);
    const int pg_lo = split * p.pages_per_split;
    const int pg_hi = min(pg_lo + p.pages_per_split, n_pages);
    const int c_lo = pg_lo << p.cpp_shift;
    const int c_hi = min(pg_hi << p.cpp_shift, cdiv(seq_len, 16));
    const int nch = max(c_hi - c_lo, 0);
    const int per = cdiv(nch, W);
    r.w_lo = c_lo + wave * per;
    r.w_hi = min(r.w_lo + per, c_hi);
    return r;
}

}  // namespace kvq
