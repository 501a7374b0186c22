/* CPU oracle for the streaming sparse INT4 MLP -- TEST INFRASTRUCTURE ONLY.
 *
 * Used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
 * checker / CPU baseline. Never linked into or called by the product library.
 *
 * Each function restates the reference algorithm it cites (paths relative to the
 * LeanStream repository):
 *   ora_weight        kernels/streaming_mlp.cu:11-15   (nibble decode, fp16_rn(q*scale))
 *   ora_compute       kernels/streaming_mlp.cu:21-43   (gate/up, fp16 rounding points,
 *                     sum256 tree order :16-20, down-projection accumulation :38-41)
 *   ora_reduce        kernels/streaming_mlp.cu:80-84   (fixed slot-order fp32 sum, fp16 out)
 *   ora_rank          predictor/predictor_cpu.cpp:192-201 (score desc, id asc)
 *   ora_publish_hidden backends/triton/reduction.py:20-22 (fp16(fp32 residual + fp32 y16))
 *   ora_rmsnorm       examples/ministral/native/predictor_shared_input.cu:16-34 (per-thread
 *                     strided sum of x^2 over 256 threads, halving tree, inverse =
 *                     1/sqrt(sum/width + eps), fp16(x*inverse) then the fp16 product with
 *                     the weight); the reference's rsqrtf is an approximation, so the
 *                     inverse is restated with IEEE sqrt and division
 *   ora_stream / ora_fill_*  the synthetic workload generator of this repository
 *                     (counter-based splitmix64, Box-Muller normal with its own ln / cos
 *                     series in IEEE double operations, double->fp16 RNE)
 * Rounding to fp16 is this file's own round-to-nearest-even integer implementation;
 * exp is the C library's expf (the reference's expf/tl.exp are only pinned to
 * tolerance by its own tests).
 */
#include "oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------- fp16 <-> fp32 / fp64 ---------------- */
float ora_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1f, mant = h & 0x3ffu, bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else { /* subnormal: mant * 2^-24 */
            float v = (float)mant * (1.0f / 16777216.0f);
            return (h & 0x8000u) ? -v : v;
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 112) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t ora_f32_to_f16(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    int exp = (int)((b >> 23) & 0xff);
    uint32_t mant = b & 0x7fffffu;
    if (exp == 0xff) return sign | 0x7c00u | (mant ? 0x200u : 0u);
    int e = exp - 127 + 15;
    if (e >= 31) return sign | 0x7c00u;
    if (e <= 0) {
        if (e < -10) return sign;
        uint32_t m = mant | 0x800000u;
        int shift = 13 + (1 - e);
        uint32_t hm = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1u))) ++hm;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = ((uint32_t)e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

uint16_t ora_f64_to_f16(double d) {
    uint64_t b;
    memcpy(&b, &d, 8);
    uint16_t sign = (uint16_t)((b >> 48) & 0x8000u);
    int exp = (int)((b >> 52) & 0x7ff);
    uint64_t mant = b & 0xFFFFFFFFFFFFFull;
    if (exp == 0x7ff) return sign | 0x7c00u | (mant ? 0x200u : 0u);
    int e = exp - 1023 + 15;
    if (e >= 31) return sign | 0x7c00u;
    if (e <= 0) {
        if (e < -10) return sign;
        uint64_t m = mant | (1ull << 52);
        int shift = 42 + (1 - e);
        uint64_t hm = m >> shift, rem = m & ((1ull << shift) - 1), half = 1ull << (shift - 1);
        if (rem > half || (rem == half && (hm & 1u))) ++hm;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = ((uint32_t)e << 10) | (uint32_t)(mant >> 42);
    uint64_t rem = mant & ((1ull << 42) - 1), half = 1ull << 41;
    if (rem > half || (rem == half && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

static float round_half(float v) { return ora_f16_to_f32(ora_f32_to_f16(v)); }

/* ---------------- generator ---------------- */
uint64_t ora_stream(uint64_t seed, uint64_t i) {
    uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static double unit(uint64_t seed, uint64_t i) { return (double)(ora_stream(seed, i) >> 11) * (1.0 / 9007199254740992.0); }

void ora_fill_bytes(uint8_t* dst, uint64_t n, uint64_t seed) {
    for (uint64_t i = 0; i < n; ++i) dst[i] = (uint8_t)(ora_stream(seed, i / 8) >> (8 * (i % 8)));
}

void ora_fill_uniform_f16(uint16_t* dst, uint64_t n, uint64_t seed, double lo, double hi) {
    for (uint64_t i = 0; i < n; ++i) dst[i] = ora_f64_to_f16(lo + (hi - lo) * unit(seed, i));
}

/* ln(u), u in (0, 1]: u = m 2^e with m in [sqrt(1/2), sqrt(2)) (exponent bits, exact),
 * ln m = 2 atanh(t), t = (m - 1) / (m + 1), series to t^25 in Horner form. */
static double ln_unit(double u) {
    uint64_t b;
    memcpy(&b, &u, 8);
    int e = (int)((b >> 52) & 0x7ff) - 1022;
    b = (b & 0x800FFFFFFFFFFFFFull) | (1022ull << 52);   /* m in [0.5, 1) */
    double m;
    memcpy(&m, &b, 8);
    if (m < 0.7071067811865476) {
        m = m * 2.0;
        e -= 1;
    }
    const double t = (m - 1.0) / (m + 1.0), t2 = t * t;
    double p = 1.0 / 25.0;
    for (int k = 11; k >= 0; --k) p = p * t2 + 1.0 / (double)(2 * k + 1);
    return (double)e * 0.6931471805599453 + 2.0 * t * p;
}

/* cos(2 pi v), v in [0, 1): quadrant q = floor(4v), x = (4v - q) pi/2, Taylor series of
 * cos x / sin x to x^22 / x^23 (coefficients by the division sequence f = -f / ((k+1)(k+2))). */
static double cos_turns(double v) {
    double cc[12], sc[12], f = 1.0, g = 1.0;
    for (int k = 0; k < 12; ++k) {
        cc[k] = f;
        sc[k] = g;
        f = -f / (double)((2 * k + 1) * (2 * k + 2));
        g = -g / (double)((2 * k + 2) * (2 * k + 3));
    }
    const double w = v * 4.0, q = floor(w), x = (w - q) * 1.5707963267948966, x2 = x * x;
    double c = cc[11], s = sc[11];
    for (int k = 10; k >= 0; --k) {
        c = c * x2 + cc[k];
        s = s * x2 + sc[k];
    }
    s = s * x;
    return q == 0.0 ? c : q == 1.0 ? -s : q == 2.0 ? -c : s;
}

/* Standard normal by Box-Muller: u1 = ((v(2i) >> 11) + 1) 2^-53 in (0, 1], u2 = unit(2i + 1). */
double ora_normal(uint64_t seed, uint64_t i) {
    const double u1 = (double)((ora_stream(seed, 2 * i) >> 11) + 1) * (1.0 / 9007199254740992.0);
    const double u2 = unit(seed, 2 * i + 1);
    return sqrt(-2.0 * ln_unit(u1)) * cos_turns(u2);
}

void ora_fill_normal_f16(uint16_t* dst, uint64_t n, uint64_t seed) {
    for (uint64_t i = 0; i < n; ++i) dst[i] = ora_f64_to_f16(ora_normal(seed, i));
}

/* ---------------- MLP arithmetic ---------------- */
float ora_weight(const uint8_t* row, const uint16_t* scale_row, uint32_t c) {
    int q = (row[c / 2] >> ((c % 2) * 4)) & 15;
    if (q >= 8) q -= 16;
    return round_half((float)q * ora_f16_to_f32(scale_row[c / 128]));
}

/* Per-lane strided accumulation then a 256-lane binary tree (sum256). */
static float tree256(float* lanes) {
    for (int stride = 128; stride; stride /= 2)
        for (int t = 0; t < stride; ++t) lanes[t] += lanes[t + stride];
    return lanes[0];
}

int ora_compute(const ora_desc* d, const uint8_t* cache, const uint8_t* staging, const uint16_t* scales,
                const uint16_t* x, uint32_t width, uint32_t G, float* partial_row, float* h_out) {
    if (!width || width % 256 || !G) return -1;
    const size_t group_bytes = (size_t)G * 3 * width / 2;
    const uint8_t* base = (d->source_kind == 1 ? staging : cache) + (size_t)d->source_slot * group_bytes;
    float gate_lane[256], up_lane[256];
    for (uint32_t c = 0; c < width; ++c) partial_row[c] = 0.0f;
    for (uint32_t n = 0; n < G; ++n) {
        const uint8_t* row = base + (size_t)n * 3 * width / 2;
        const uint16_t* sc = scales + ((size_t)d->physical_group * G + n) * 3 * (width / 128);
        for (int t = 0; t < 256; ++t) {
            float g = 0.0f, u = 0.0f;
            for (uint32_t c = (uint32_t)t; c < width; c += 256) {
                float xv = ora_f16_to_f32(x[c]);
                g += ora_weight(row, sc, c) * xv;
                u += ora_weight(row + width / 2, sc + width / 128, c) * xv;
            }
            gate_lane[t] = g;
            up_lane[t] = u;
        }
        float ga = round_half(tree256(gate_lane));
        float up = round_half(tree256(up_lane));
        float silu = round_half(ga / (1.0f + expf(-ga)));
        float h = round_half(silu * up);
        if (h_out) h_out[n] = h;
        for (uint32_t c = 0; c < width; ++c)
            partial_row[c] = fmaf(h, ora_weight(row + width, sc + 2 * (width / 128), c), partial_row[c]);
    }
    return 0;
}

void ora_reduce(const float* partial, uint32_t rows, uint32_t width, float* y32, uint16_t* y16) {
    for (uint32_t c = 0; c < width; ++c) {
        float s = 0.0f;
        for (uint32_t i = 0; i < rows; ++i) s += partial[(size_t)i * width + c];
        if (y32) y32[c] = s;
        if (y16) y16[c] = ora_f32_to_f16(s);
    }
}

int ora_layer(const ora_desc* descs, uint32_t count, uint32_t rows, const uint8_t* cache, const uint8_t* staging,
              const uint16_t* scales, const uint16_t* x, uint32_t width, uint32_t G, int threads, float* y32,
              uint16_t* y16, float* h_rows, float* partial) {
    int owned = 0, bad = 0;
    if (!partial) {
        partial = (float*)malloc(sizeof(float) * (size_t)rows * width);
        if (!partial) return -2;
        owned = 1;
    }
    memset(partial, 0, sizeof(float) * (size_t)rows * width);
    for (uint32_t i = 0; i < count; ++i)
        if (descs[i].dest_slot >= rows) bad = 1;
    if (!bad) {
#ifdef _OPENMP
        if (threads < 1) threads = 1;
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
#endif
        for (int i = 0; i < (int)count; ++i) {
            const ora_desc* d = descs + i;
            ora_compute(d, cache, staging, scales, x, width, G, partial + (size_t)d->dest_slot * width,
                        h_rows ? h_rows + (size_t)d->dest_slot * G : NULL);
        }
        ora_reduce(partial, rows, width, y32, y16);
    }
    (void)threads;
    if (owned) free(partial);
    return bad ? -1 : 0;
}

/* ---------------- selection ---------------- */
static const float* rank_scores;
static int rank_cmp(const void* pa, const void* pb) {
    int32_t a = *(const int32_t*)pa, b = *(const int32_t*)pb;
    if (rank_scores[a] > rank_scores[b]) return -1;
    if (rank_scores[a] < rank_scores[b]) return 1;
    return (a > b) - (a < b);
}

int ora_rank(const float* scores, uint32_t n, uint32_t k, int32_t* out) {
    if (k > n) return -1;
    for (uint32_t i = 0; i < n; ++i)
        if (!isfinite(scores[i])) return -3;
    int32_t* ids = (int32_t*)malloc(sizeof(int32_t) * (n ? n : 1));
    if (!ids) return -2;
    for (uint32_t i = 0; i < n; ++i) ids[i] = (int32_t)i;
    rank_scores = scores;
    qsort(ids, n, sizeof(int32_t), rank_cmp);
    memcpy(out, ids, sizeof(int32_t) * k);
    free(ids);
    return 0;
}

/* ---------------- epilogue: next-hidden publication and RMSNorm ---------------- */
void ora_publish_hidden(const uint16_t* residual, const uint16_t* y16, uint32_t n, uint16_t* hidden) {
    for (uint32_t c = 0; c < n; ++c)
        hidden[c] = ora_f32_to_f16(ora_f16_to_f32(residual[c]) + ora_f16_to_f32(y16[c]));
}

int ora_rmsnorm(const uint16_t* x, const uint16_t* weight, float eps, uint32_t width, uint16_t* out) {
    float lanes[256];
    if (!width) return -1;
    for (int t = 0; t < 256; ++t) {
        float sum = 0.f;
        for (uint32_t i = (uint32_t)t; i < width; i += 256) {
            const float v = ora_f16_to_f32(x[i]);
            sum += v * v;
        }
        lanes[t] = sum;
    }
    const float total = tree256(lanes);
    const float inverse = 1.0f / sqrtf(total / (float)width + eps);
    for (uint32_t i = 0; i < width; ++i) {
        const float normalized = round_half(ora_f16_to_f32(x[i]) * inverse);
        out[i] = ora_f32_to_f16(ora_f16_to_f32(weight[i]) * normalized);   /* exact product, one rounding */
    }
    return 0;
}
