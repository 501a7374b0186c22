// Synthetic workload generation on the device.
//
// Counter-based splitmix64 (S. Vigna's public-domain mixer): value(seed, i) =
// mix(seed + (i + 1) * 0x9E3779B97F4A7C15). Element i of every stream depends only
// on (seed, i), so a host mirror (leanstream_amd/synth.py) produces the same bytes.
//   bytes:    little-endian bytes of value(seed, i) for word i (uniform INT4 nibbles)
//   uniform:  lo + (hi - lo) * u, u = (value >> 11) * 2^-53, rounded double -> fp16 (RNE)
//   normal:   Box-Muller of u1 = ((value(2i) >> 11) + 1) 2^-53 in (0, 1] and u2 = unit(2i + 1):
//             sqrt(-2 ln u1) cos(2 pi u2) -> fp16 or bf16 (RNE). ln and cos are series in IEEE
//             double +, -, *, / (no library calls, no fused multiply-add), so the host mirror
//             computes the same doubles.
// The double -> fp16 rounding is done in integer arithmetic (no double rounding).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <cerrno>
#include "leanstream_hip.h"

namespace lsamd {

__host__ __device__ inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__host__ __device__ inline uint64_t stream_value(uint64_t seed, uint64_t i) {
    return mix64(seed + (i + 1) * 0x9E3779B97F4A7C15ull);
}
__host__ __device__ inline double stream_unit(uint64_t seed, uint64_t i) {
    return (double)(stream_value(seed, i) >> 11) * 0x1.0p-53;
}

// Round-to-nearest-even conversion of a double to IEEE binary16 bits.
__host__ __device__ inline uint16_t f64_to_f16_bits(double d) {
    const uint64_t b = __builtin_bit_cast(uint64_t, d);
    const uint16_t sign = (uint16_t)((b >> 48) & 0x8000u);
    const int exp = (int)((b >> 52) & 0x7ff);
    const uint64_t mant = b & 0xFFFFFFFFFFFFFull;
    if (exp == 0x7ff) return sign | 0x7c00u | (mant ? 0x200u : 0u);
    const int e = exp - 1023 + 15;
    if (e >= 31) return sign | 0x7c00u;
    if (e <= 0) {
        if (e < -10) return sign;
        const uint64_t m = mant | (1ull << 52);
        const int shift = 42 + (1 - e);
        uint64_t hm = m >> shift;
        const uint64_t rem = m & ((1ull << shift) - 1), half = 1ull << (shift - 1);
        if (rem > half || (rem == half && (hm & 1))) ++hm;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = ((uint32_t)e << 10) | (uint32_t)(mant >> 42);
    const uint64_t rem = mant & ((1ull << 42) - 1), half = 1ull << 41;
    if (rem > half || (rem == half && (h & 1))) ++h;
    return (uint16_t)(sign | h);
}

__global__ void synth_bytes_kernel(uint8_t* dst, uint64_t bytes, uint64_t seed) {
    const uint64_t words = (bytes + 7) / 8;
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < words; i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t v = stream_value(seed, i);
        if (8 * i + 8 <= bytes) {
            reinterpret_cast<uint64_t*>(dst)[i] = v;
        } else {
            for (uint64_t k = 0; 8 * i + k < bytes; ++k) dst[8 * i + k] = (uint8_t)(v >> (8 * k));
        }
    }
}

__global__ void synth_uniform_kernel(uint16_t* dst, uint64_t count, uint64_t seed, double lo, double hi) {
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < count; i += (uint64_t)gridDim.x * blockDim.x)
        dst[i] = f64_to_f16_bits(lo + (hi - lo) * stream_unit(seed, i));
}

// Round-to-nearest-even conversion of a double to bfloat16 bits (finite values of the
// normal generator, |v| < 9; below bf16's normal range maps to signed zero).
__host__ __device__ inline uint16_t f64_to_bf16_bits(double d) {
    const uint64_t b = __builtin_bit_cast(uint64_t, d);
    const uint16_t sign = (uint16_t)((b >> 48) & 0x8000u);
    const int exp = (int)((b >> 52) & 0x7ff);
    if (exp == 0) return sign;
    const uint64_t mant = b & 0xFFFFFFFFFFFFFull;
    int e = exp - 1023 + 127;
    uint32_t m = (uint32_t)(mant >> 45);
    const uint64_t rem = mant & ((1ull << 45) - 1), half = 1ull << 44;
    if (rem > half || (rem == half && (m & 1u))) ++m;
    if (m == 128u) {
        m = 0;
        ++e;
    }
    if (e >= 255) return sign | 0x7f80u;
    if (e <= 0) return sign;
    return sign | (uint16_t)(e << 7) | (uint16_t)m;
}

// ln(u), u in (0, 1]: u = m 2^e with m in [sqrt(1/2), sqrt(2)), ln m = 2 atanh(t),
// t = (m - 1) / (m + 1), series to t^25 in Horner form.
__device__ inline double ln_unit(double u) {
#pragma clang fp contract(off)
    uint64_t b = __builtin_bit_cast(uint64_t, u);
    int e = (int)((b >> 52) & 0x7ff) - 1022;
    double m = __builtin_bit_cast(double, (b & 0x800FFFFFFFFFFFFFull) | (1022ull << 52));
    if (m < 0.7071067811865476) {
        m = m * 2.0;
        e -= 1;
    }
    const double t = (m - 1.0) / (m + 1.0), t2 = t * t;
    double p = 1.0 / 25.0;
    for (int k = 11; k >= 0; --k) p = p * t2 + 1.0 / (double)(2 * k + 1);
    return (double)e * 0.6931471805599453 + 2.0 * t * p;
}

// cos(2 pi v), v in [0, 1): quadrant q = floor(4v), x = (4v - q) pi / 2, Taylor series of
// cos x / sin x to x^22 / x^23, coefficients by the division sequence f = -f / ((k+1)(k+2)).
__device__ inline double cos_turns(double v) {
#pragma clang fp contract(off)
    double cc[12], sc[12], f = 1.0, g = 1.0;
#pragma unroll
    for (int k = 0; k < 12; ++k) {
        cc[k] = f;
        sc[k] = g;
        f = -f / (double)((2 * k + 1) * (2 * k + 2));
        g = -g / (double)((2 * k + 2) * (2 * k + 3));
    }
    const double w = v * 4.0, q = __builtin_floor(w), x = (w - q) * 1.5707963267948966, x2 = x * x;
    double c = cc[11], s = sc[11];
#pragma unroll
    for (int k = 10; k >= 0; --k) {
        c = c * x2 + cc[k];
        s = s * x2 + sc[k];
    }
    s = s * x;
    return q == 0.0 ? c : q == 1.0 ? -s : q == 2.0 ? -c : s;
}

__device__ inline double box_muller(uint64_t seed, uint64_t i) {
#pragma clang fp contract(off)
    const double u1 = (double)((stream_value(seed, 2 * i) >> 11) + 1) * 0x1.0p-53;
    const double u2 = stream_unit(seed, 2 * i + 1);
    return __builtin_sqrt(-2.0 * ln_unit(u1)) * cos_turns(u2);
}

__global__ void synth_normal_bf16_kernel(uint16_t* dst, uint64_t count, uint64_t seed) {
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < count; i += (uint64_t)gridDim.x * blockDim.x)
        dst[i] = f64_to_bf16_bits(box_muller(seed, i));
}

__global__ void synth_normal_kernel(uint16_t* dst, uint64_t count, uint64_t seed) {
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < count; i += (uint64_t)gridDim.x * blockDim.x)
        dst[i] = f64_to_f16_bits(box_muller(seed, i));
}

// One wave holds its stream until the host sets *flag (a host-coherent word) or the bound
// (in ticks of the 100 MHz clock) passes, whichever comes first.
__global__ void hold_kernel(const uint32_t* flag, uint64_t limit) {
    if (threadIdx.x != 0) return;
    const uint64_t start = wall_clock64();
    uint32_t n = 0;
    while (!__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM)) {
        __builtin_amdgcn_s_sleep(8);
        if ((++n & 15u) == 0 && wall_clock64() - start > limit) break;
    }
}

static unsigned grid_for(uint64_t n) {
    uint64_t g = (n + 255) / 256;
    return (unsigned)(g > 65536 ? 65536 : (g ? g : 1));
}

}  // namespace lsamd

extern "C" {

int ls_synth_bytes(void* dst, uint64_t bytes, uint64_t seed, void* stream) {
    if (!dst && bytes) return EINVAL;
    if (!bytes) return 0;
    hipLaunchKernelGGL(lsamd::synth_bytes_kernel, dim3(lsamd::grid_for((bytes + 7) / 8)), dim3(256), 0,
                       (hipStream_t)stream, (uint8_t*)dst, bytes, seed);
    return (int)hipPeekAtLastError();
}

int ls_synth_uniform_f16(void* dst, uint64_t count, uint64_t seed, double lo, double hi, void* stream) {
    if (!dst && count) return EINVAL;
    if (!count) return 0;
    hipLaunchKernelGGL(lsamd::synth_uniform_kernel, dim3(lsamd::grid_for(count)), dim3(256), 0, (hipStream_t)stream,
                       (uint16_t*)dst, count, seed, lo, hi);
    return (int)hipPeekAtLastError();
}

int ls_synth_normal_bf16(void* dst, uint64_t count, uint64_t seed, void* stream) {
    if (!dst && count) return EINVAL;
    if (!count) return 0;
    hipLaunchKernelGGL(lsamd::synth_normal_bf16_kernel, dim3(lsamd::grid_for(count)), dim3(256), 0,
                       (hipStream_t)stream, (uint16_t*)dst, count, seed);
    return (int)hipPeekAtLastError();
}

int ls_synth_normal_f16(void* dst, uint64_t count, uint64_t seed, void* stream) {
    if (!dst && count) return EINVAL;
    if (!count) return 0;
    hipLaunchKernelGGL(lsamd::synth_normal_kernel, dim3(lsamd::grid_for(count)), dim3(256), 0, (hipStream_t)stream,
                       (uint16_t*)dst, count, seed);
    return (int)hipPeekAtLastError();
}

int ls_hold_stream(void* stream, const uint32_t* flag, uint64_t limit_ticks) {
    if (!flag || !limit_ticks) return EINVAL;
    hipLaunchKernelGGL(lsamd::hold_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, flag, limit_ticks);
    return (int)hipPeekAtLastError();
}

}  // extern "C"
