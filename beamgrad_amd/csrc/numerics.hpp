// SPDX-License-Identifier: MIT
//
// Bit-exact numerics of the beam search, shared by the host code and the
// gfx950 kernels of libdbs_hip. Every function is a fixed sequence of single
// IEEE-rounded operations; the library is compiled with -ffp-contract=off (no
// fused multiply-add) and without denormal flushing, so host and device give
// the reference's bits:
//   * 16-bit rows to float                    (reference src/half.hpp:16-36)
//   * exp(x) for x <= 0, Cephes expf split    (src/logits.hpp:22-73)
//   * ln(x) for x >= 1 and exp(y) for y >= 0 in double (src/penalty.hpp:40-97)
//   * GNMT length penalty                     (src/penalty.hpp:101-122)
//   * logsumexp from (max, lane sum)          (src/logits.hpp:79-81)
// The constants and operation order are the published Cephes expf reduction
// and polynomial and textbook atanh / Taylor series; they must match the
// reference operation for operation to give the same bits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define DBS_HD __host__ __device__ __forceinline__

namespace dbs_hip {

DBS_HD float bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }
DBS_HD uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }

constexpr float kInf = __builtin_inff();

DBS_HD float half_to_f32(uint16_t h) {
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0) {
        const float mag = static_cast<float>(m) * 5.9604644775390625e-8f;  // m * 2^-24, exact
        return sign ? -mag : mag;
    }
    if (e == 31) return bits_f32(sign | 0x7f800000u | (m << 13));
    return bits_f32(sign | ((e + 112u) << 23) | (m << 13));
}

DBS_HD float bf16_to_f32(uint16_t h) { return bits_f32(static_cast<uint32_t>(h) << 16); }

// exp(x) for x <= 0 (0 below -87, for -inf and for NaN).
DBS_HD float exp_nonpositive(float x) {
    if (!(x >= -87.0f)) return 0.0f;
    const float k = __builtin_floorf(x * 1.44269504088896341f + 0.5f);
    const float r = (x - k * 0.693359375f) - k * -2.12194440e-4f;
    const float r2 = r * r;
    float p = 1.9875691500e-4f;
    p = p * r + 1.3981999507e-3f;
    p = p * r + 8.3334519073e-3f;
    p = p * r + 4.1665795894e-2f;
    p = p * r + 1.6666665459e-1f;
    p = p * r + 5.0000001201e-1f;
    p = (p * r2 + r) + 1.0f;
    return p * bits_f32(static_cast<uint32_t>(static_cast<int>(k) + 127) << 23);
}

// exp_nonpositive without branches: the same operations on max(x, -87),
// then 0 below -87 (and for NaN).
DBS_HD float exp_nonpositive_nb(float x) {
    const bool in = x >= -87.0f;
    const float xc = in ? x : -87.0f;
    const float k = __builtin_floorf(xc * 1.44269504088896341f + 0.5f);
    const float r = (xc - k * 0.693359375f) - k * -2.12194440e-4f;
    const float r2 = r * r;
    float p = 1.9875691500e-4f;
    p = p * r + 1.3981999507e-3f;
    p = p * r + 8.3334519073e-3f;
    p = p * r + 4.1665795894e-2f;
    p = p * r + 1.6666665459e-1f;
    p = p * r + 5.0000001201e-1f;
    p = (p * r2 + r) + 1.0f;
    const float e = p * bits_f32(static_cast<uint32_t>(static_cast<int>(k) + 127) << 23);
    return in ? e : 0.0f;
}

// Constants of log_ge1 as given (Plain), or made opaque by an xor with a
// run-time zero (Opaque: a caller inside a persistent loop keeps them from
// being hoisted into registers for the whole loop).
struct PlainConst {
    DBS_HD double operator()(double c) const { return c; }
};
struct OpaqueConst {
    uint64_t zero;
    DBS_HD double operator()(double c) const {
        return __builtin_bit_cast(double, __builtin_bit_cast(uint64_t, c) ^ zero);
    }
};

// ln(x), x >= 1, in double.
template <class K>
DBS_HD double log_ge1_with(double x, K k) {
    int e = 0;
    double m = __builtin_frexp(x, &e);
    if (m < k(0.70710678118654752440)) {
        m = m * k(2.0);
        e -= 1;
    }
    const double one = k(1.0);
    const double s = (m - one) / (m + one);
    const double z = s * s;
    double p = k(1.0 / 23.0);
    p = p * z + k(1.0 / 21.0);
    p = p * z + k(1.0 / 19.0);
    p = p * z + k(1.0 / 17.0);
    p = p * z + k(1.0 / 15.0);
    p = p * z + k(1.0 / 13.0);
    p = p * z + k(1.0 / 11.0);
    p = p * z + k(1.0 / 9.0);
    p = p * z + k(1.0 / 7.0);
    p = p * z + k(1.0 / 5.0);
    p = p * z + k(1.0 / 3.0);
    p = p * z + one;
    const double log_m = (k(2.0) * s) * p;
    const double de = static_cast<double>(e);
    return de * k(6.93147180369123816490e-01) + (de * k(1.90821492927058770002e-10) + log_m);
}
DBS_HD double log_ge1(double x) { return log_ge1_with(x, PlainConst{}); }

// exp(y), y >= 0, in double.
DBS_HD double exp_ge0(double y) {
    if (y > 709.0) return __builtin_huge_val();
    const int k = static_cast<int>(y * 1.44269504088896338700e+00 + 0.5);
    const double dk = static_cast<double>(k);
    const double r = (y - dk * 6.93147180369123816490e-01) - dk * 1.90821492927058770002e-10;
    double p = 1.0 / 1307674368000.0;
    p = p * r + 1.0 / 87178291200.0;
    p = p * r + 1.0 / 6227020800.0;
    p = p * r + 1.0 / 479001600.0;
    p = p * r + 1.0 / 39916800.0;
    p = p * r + 1.0 / 3628800.0;
    p = p * r + 1.0 / 362880.0;
    p = p * r + 1.0 / 40320.0;
    p = p * r + 1.0 / 5040.0;
    p = p * r + 1.0 / 720.0;
    p = p * r + 1.0 / 120.0;
    p = p * r + 1.0 / 24.0;
    p = p * r + 1.0 / 6.0;
    p = p * r + 0.5;
    p = p * r + 1.0;
    p = p * r + 1.0;
    return __builtin_ldexp(p, k);
}

// ((5 + max(length, 1)) / 6)^alpha as float.
DBS_HD float length_penalty(int length, float alpha) {
    if (alpha == 0.0f) return 1.0f;
    const int l = length > 1 ? length : 1;
    const double base = (5.0 + static_cast<double>(l)) / 6.0;
    if (alpha <= 64.0f && alpha == static_cast<float>(static_cast<int>(alpha))) {
        int n = static_cast<int>(alpha);
        double acc = 1.0;
        double sq = base;
        while (n > 0) {
            if (n & 1) acc = acc * sq;
            sq = sq * sq;
            n >>= 1;
        }
        return static_cast<float>(acc);
    }
    return static_cast<float>(exp_ge0(static_cast<double>(alpha) * log_ge1(base)));
}

DBS_HD float logsumexp_from(float max, float lane_sum) {
    return max + static_cast<float>(log_ge1(static_cast<double>(lane_sum)));
}
// The same, its constants opaque (see OpaqueConst).
DBS_HD float logsumexp_from_opaque(float max, float lane_sum, uint64_t zero) {
    return max + static_cast<float>(log_ge1_with(static_cast<double>(lane_sum), OpaqueConst{zero}));
}

// Softmax probability of x in a row with logsumexp lse; 0 for non-finite x.
DBS_HD float softmax_probability(float x, float lse) {
    const bool finite = x < kInf && x > -kInf;
    return finite ? exp_nonpositive(x - lse) : 0.0f;
}

// Total order of candidates (reference src/common.hpp:269-276): score desc,
// raw desc, parent asc, token asc, length asc, from_logprob desc; float
// comparisons, so -0 == +0.
struct Cand {
    float score;
    float raw;
    int32_t parent;
    int32_t token;
    int32_t length;
    int32_t flp;
};

// Branch-free: each level is "strictly before, or equal and the next level
// decides", with non-short-circuit operators so the device code stays
// straight-line.
DBS_HD bool before(const Cand& a, const Cand& b) {
    const bool by_length = (a.length < b.length) | ((a.length == b.length) & (a.flp > b.flp));
    const bool by_token = (a.token < b.token) | ((a.token == b.token) & by_length);
    const bool by_parent = (a.parent < b.parent) | ((a.parent == b.parent) & by_token);
    const bool by_raw = (a.raw > b.raw) | ((a.raw == b.raw) & by_parent);
    return (a.score > b.score) | ((a.score == b.score) & by_raw);
}

DBS_HD Cand dead_cand() { return Cand{-kInf, -kInf, -1, -1, 0, 0}; }

// float -> bfloat16 / binary16 with round-to-nearest-even, NaN kept quiet
// (the conversion torch's Tensor.to() performs).
DBS_HD uint16_t f32_to_bf16_rne(float f) {
    const uint32_t u = f32_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;  // canonical quiet NaN
    const uint32_t lsb = (u >> 16) & 1u;
    return static_cast<uint16_t>((u + 0x7fffu + lsb) >> 16);
}

DBS_HD uint16_t f32_to_f16_rne(float f) {
    const uint32_t u = f32_bits(f);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return static_cast<uint16_t>(sign | 0x7e00u | ((a >> 13) & 0x3ffu));  // NaN
    if (a >= 0x477ff000u) return static_cast<uint16_t>(sign | 0x7c00u);  // rounds to inf (incl. inf)
    if (a < 0x38800000u) {
        // result is subnormal or zero in binary16: round a * 2^24 to an integer (RNE)
        if (a < 0x33000000u) return static_cast<uint16_t>(sign);  // below half of the smallest subnormal
        const uint32_t e = a >> 23;
        const uint32_t m = (a & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - e;  // value = m * 2^(e-150); want m * 2^(e-150+24) = m >> (126-e)
        uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return static_cast<uint16_t>(sign | q);
    }
    // normal: rebias exponent, round 13 dropped bits (carry may bump the exponent)
    uint32_t r = a - 0x38000000u;
    const uint32_t lsb = (r >> 13) & 1u;
    r = (r + 0xfffu + lsb) >> 13;
    return static_cast<uint16_t>(sign | r);
}

}  // namespace dbs_hip
