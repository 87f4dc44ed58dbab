// Exhaustive check of the quantizers' e4m3fn encode (kvq_decode_amd/csrc/quant.hip
// e4m3fn_rne: the hardware conversion v_cvt_scalef32_pk_fp8_f32 at scale 1) against the
// spec's software encode (oracle/kivi.py: mantissa rounded half to even at 2^(e-3),
// subnormals at 2^-9), for every fp32 bit pattern in [0, 448] and its negation
// (2,277,507,074 values). Prints the count of differences and the first few; exit status 0
// = none. Test infrastructure, built by kvq_decode_amd.build, run by
// tests/test_fp8_encode_gpu.py.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#define CK(x)                                                                            \
    do {                                                                                 \
        hipError_t e = (x);                                                              \
        if (e != hipSuccess) {                                                           \
            printf("HIP error %s at line %d\n", hipGetErrorString(e), __LINE__);         \
            exit(2);                                                                     \
        }                                                                                \
    } while (0)

typedef short s2 __attribute__((ext_vector_type(2)));

// The spec's encode, restated in software.
__device__ uint32_t spec_e4m3fn(float t) {
    const uint32_t sign = (__float_as_uint(t) >> 31) << 7;
    const float a = fabsf(t);
    uint32_t bits;
    if (a < 0.015625f) {  // below 2^-6: subnormal m * 2^-9 (m = 8 is 2^-6)
        bits = (uint32_t)__builtin_rintf(a * 512.f);
    } else {
        int e = (int)((__float_as_uint(a) >> 23) & 0xFF) - 127;
        const float frac = a * __uint_as_float((uint32_t)(127 - e) << 23) - 1.f;
        int m = (int)__builtin_rintf(frac * 8.f);
        if (m == 8) {
            m = 0;
            ++e;
        }
        bits = ((uint32_t)(e + 7) << 3) | (uint32_t)m;
    }
    return bits | sign;
}

// The kernel's encode (quant.hip).
__device__ uint32_t kernel_e4m3fn(float t) {
    const s2 r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(s2{0, 0}, t, 0.f, 1.0f, false);
    return __builtin_bit_cast(uint32_t, r) & 0xFFu;
}

constexpr uint32_t kTop = 0x43E00000u;  // 448.0f

__global__ void check(unsigned long long* bad, uint32_t* rec) {
    const uint64_t n = 2ull * (kTop + 1);  // [0, kTop], then the same values negated
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint32_t u = (uint32_t)(i % (kTop + 1)) | (i > kTop ? 0x80000000u : 0u);
        const float t = __uint_as_float(u);
        const uint32_t want = spec_e4m3fn(t), got = kernel_e4m3fn(t);
        if (want != got) {
            const unsigned long long k = atomicAdd(bad, 1ull);
            if (k < 8) {
                rec[3 * k] = u;
                rec[3 * k + 1] = want;
                rec[3 * k + 2] = got;
            }
        }
    }
}

int main() {
    unsigned long long* bad;
    uint32_t* rec;
    CK(hipMalloc(&bad, sizeof(unsigned long long)));
    CK(hipMalloc(&rec, 24 * sizeof(uint32_t)));
    CK(hipMemset(bad, 0, sizeof(unsigned long long)));
    CK(hipMemset(rec, 0, 24 * sizeof(uint32_t)));
    hipLaunchKernelGGL(check, dim3(65536), dim3(256), 0, 0, bad, rec);
    CK(hipGetLastError());
    CK(hipDeviceSynchronize());
    unsigned long long nbad = 0;
    uint32_t hrec[24];
    CK(hipMemcpy(&nbad, bad, sizeof(nbad), hipMemcpyDeviceToHost));
    CK(hipMemcpy(hrec, rec, sizeof(hrec), hipMemcpyDeviceToHost));
    printf("%llu values, %llu differ\n", 2ull * (kTop + 1), nbad);
    for (unsigned k = 0; k < 8 && k < nbad; ++k)
        printf("  fp32 %08x: spec %02x, kernel %02x\n", hrec[3 * k], hrec[3 * k + 1],
               hrec[3 * k + 2]);
    return nbad != 0;
}
