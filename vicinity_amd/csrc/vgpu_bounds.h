// Error bounds of the approximate scores the kernels rank by, against the
// reference's float32 arithmetic.  Host and device evaluate the same
// formulas: the kernels use them in their proofs, and the library exports
// them to host-side tests that drive adversarial inputs against them.
#pragma once

#include <hip/hip_runtime.h>

namespace vgpu {

// Error bound of the fp32 scores (MFMA GEMM or approx_dot) against the sequential one: both are within
// (d + 2) u sum|q_j c_j| <= (d + 2) u ||q|| ||c|| of the real dot product,
// plus the rounding of 1 - dot; doubled for safety.
__host__ __device__ inline float coarse_tau(int d, float qn, float cmax) {
    const float u = 5.9604645e-08f;
    return 2.0f * ((2.0f * (float)d + 8.0f) * u * qn * cmax + 4.0f * u * (1.0f + qn * cmax)) +
           1e-30f;
}

// Error bound eps of the bf16x3 score against the reference's sequential one
// for ||q|| <= qn, ||c|| <= cmax (u = 2^-24).  bfloat16 keeps 8 significant
// bits, so rounding to it is within 2^-8 relative: |x - hi| <= 2^-8 |x| and
// x = hi + lo + r with |r| <= 2^-8 |x - hi| <= 2^-16 |x|.  The dropped terms
// (ql.cl, qh.rc, rq.ch and smaller) are then within 3.01 * 2^-16 sum|q_j c_j|,
// the fp32
// accumulation of 3d exact products within 3d 2u (accumulation that
// truncates), the sequential dot within d u, and 1 - dot rounds within
// 2u (1 + qn cmax).
__host__ __device__ inline float coarse_eps_bf16(int d, float qn, float cmax) {
    const float u = 5.9604645e-08f;
    const float qc = qn * cmax;
    return (3.01f * 1.5258789e-05f + 7.0f * (float)d * u) * qc + 2.0f * u * (1.0f + qc) + 1e-30f;
}

// Bound on |a - e| for ||q|| <= qn, ||c|| <= cmax, ||x_r|| <= rmax and
// ||q - c||^2 <= t0max (u = 2^-24).  With rr = sqrt(t0max) + rmax >= ||r - x_r||:
//   |e - D| <= (ds + M) u rr^2 + 2u (||q - c|| rr + rr^2)     (reference arithmetic)
//   |a - D| <= (d + M + ds + 4) u (t0max + rmax^2 + 2 (cmax + qn) rmax)
// where D is the real-number distance; both are below
// (d + M + ds + 8) u S with S = 2 (qn + cmax) rmax + 2 rmax^2 + 2 rr^2, which
// is taken with a factor of 4 to spare.
__host__ __device__ inline float fast_tau(int d, int M, int ds, float qn, float cmax, float rmax,
                                          float t0max) {
    const float u = 5.9604645e-08f;
    float rr = sqrtf(t0max) + rmax;
    float S = 2.0f * (qn + cmax) * rmax + 2.0f * rmax * rmax + 2.0f * rr * rr;
    return 4.0f * (float)(d + M + ds + 8) * u * S + 1e-30f;
}

// Bound on |ranking key + ||q||^2 (metric 0) - exact distance| with the
// exact distance l2_distance_squared / 1 - seq_dot in float32
// (u = 2^-24, |q| <= qn, |x| <= xn): the bf16x3 product is within
// (3.01 2^-16 + 7 d u) |q||x| of q.x (as the coarse bound), ||x||^2 within
// d u ||x||^2, one rounding
// of the score, the reference's sum within (d + 1) u (|q| + |x|)^2 (or
// d u |q||x| + 2u (1 + |q||x|) for 1 - dot), taken twice; plus the packing:
// a key is the score with its low ib mantissa bits replaced by a tile index,
// within 2^ib ulps of |score| <= ||x||^2 + 2 |q||x| (or 1 + |q||x|).
__host__ __device__ inline float flat_bf16_tau(int d, int metric, float qn, float xn, int ib) {
    const float u = 5.9604645e-08f;
    const float qx = qn * xn;
    const float dot = (3.01f * 1.5258789e-05f + 7.0f * (float)d * u) * qx;
    const float smax = metric == 1 ? 1.0f + qx : xn * xn + 2.0f * qx;
    const float pack = ((float)(1u << ib) + 1.0f) * 2.0f * u * smax;
    if (metric == 1) return 2.0f * (dot + (float)d * u * qx + 2.0f * u * (1.0f + qx)) + pack + 1e-30f;
    const float s = qn + xn;
    return 2.0f * (2.0f * dot + (float)d * u * xn * xn + u * (xn * xn + 2.0f * qx) +
                   (float)(d + 1) * u * s * s) + pack + 1e-30f;
}

}  // namespace vgpu
