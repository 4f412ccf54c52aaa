// OPQ kernels: the rotation y = R x of many rows, and the Procrustes
// cross-covariance of a training sample.
//
// Reference: OptimizedProductQuantizer src/ivf_pq/opq.rs:29-160 (rotation R,
// row-major, applied before quantize :112-115 and before the ADC table
// :120-123), matrix_vector_multiply :180-191, compute_optimal_rotation
// :232-295; the residual it rotates, search.rs:1242-1255 / :722-729.
#include "vgpu_device.h"
#include "vgpu_launch.h"

namespace vgpu {

constexpr int ROT_RB = 16;  // rows per row group

// out[r][i] = sum_j R[i][j] * x_r[j], j ascending from 0.0, each product and
// each sum rounded (matrix_vector_multiply; this file is built without FMA
// contraction).  x_r = X[r / xdiv] - C[lists[r]] when C is given (a row whose
// list is >= L is zero: a padding slot), else X[r].  A block takes G row
// groups of ROT_RB rows, G = max(1, 256 / d); the rows wait in LDS and a
// thread forms output i of its group's rows, reading row i of R once for all
// of them.  VEC: d % 4 == 0, so R's rows are read as float4.
template <bool VEC>
__global__ __launch_bounds__(256) void rotate_rows_kernel(const float* __restrict__ R,
                                                          const float* __restrict__ X, int xdiv,
                                                          const float* __restrict__ C,
                                                          const uint32_t* __restrict__ lists, int L,
                                                          int n, int d, float* __restrict__ out) {
    extern __shared__ __align__(16) float xs[];
    const int tid = threadIdx.x;
    const int dg = d < 256 ? d : 256;
    const int G = 256 / dg;
    const int rows = ROT_RB * G;
    const size_t r0 = (size_t)blockIdx.x * rows;
    for (int e = tid; e < rows * d; e += 256) {
        const int rr = e / d, j = e - rr * d;
        const size_t r = r0 + rr;
        float v = 0.0f;
        if (r < (size_t)n) {
            const float x = X[(r / (size_t)xdiv) * d + j];
            if (C) {
                const uint32_t l = lists[r];
                if (l < (uint32_t)L) v = x - C[(size_t)l * d + j];
            } else {
                v = x;
            }
        }
        xs[e] = v;
    }
    __syncthreads();
    const int g = tid / dg;
    if (g >= G) return;
    const float* xg = xs + (size_t)g * ROT_RB * d;
    for (int i = tid - g * dg; i < d; i += dg) {
        const float* Ri = R + (size_t)i * d;
        float acc[ROT_RB];
#pragma unroll
        for (int rr = 0; rr < ROT_RB; rr++) acc[rr] = 0.0f;
        if constexpr (VEC) {
            for (int j = 0; j < d; j += 4) {
                const float4 rv = *reinterpret_cast<const float4*>(Ri + j);
#pragma unroll
                for (int rr = 0; rr < ROT_RB; rr++) {
                    const float4 xv = *reinterpret_cast<const float4*>(xg + rr * d + j);
                    acc[rr] += rv.x * xv.x;
                    acc[rr] += rv.y * xv.y;
                    acc[rr] += rv.z * xv.z;
                    acc[rr] += rv.w * xv.w;
                }
            }
        } else {
            for (int j = 0; j < d; j++) {
                const float rij = Ri[j];
#pragma unroll
                for (int rr = 0; rr < ROT_RB; rr++) acc[rr] += rij * xg[rr * d + j];
            }
        }
#pragma unroll
        for (int rr = 0; rr < ROT_RB; rr++) {
            const size_t r = r0 + (size_t)g * ROT_RB + rr;
            if (r < (size_t)n) out[r * d + i] = acc[rr];
        }
    }
}

size_t rotate_rows_lds_bytes(int d) {
    const int dg = d < 256 ? d : 256;
    return (size_t)ROT_RB * (256 / dg) * d * sizeof(float);
}

void launch_rotate_rows(const float* R, const float* X, int xdiv, const float* C,
                        const uint32_t* lists, int L, size_t n, int d, float* out, hipStream_t s) {
    if (n == 0) return;
    const int dg = d < 256 ? d : 256;
    const size_t rows = (size_t)ROT_RB * (256 / dg);
    const size_t lds = rotate_rows_lds_bytes(d);
    const dim3 grid((unsigned)((n + rows - 1) / rows));
    if (d % 4 == 0) {
        ensure_dyn_lds((const void*)rotate_rows_kernel<true>, lds);
        hipLaunchKernelGGL(rotate_rows_kernel<true>, grid, dim3(256), lds, s, R, X, xdiv, C, lists, L,
                           (int)n, d, out);
    } else {
        ensure_dyn_lds((const void*)rotate_rows_kernel<false>, lds);
        hipLaunchKernelGGL(rotate_rows_kernel<false>, grid, dim3(256), lds, s, R, X, xdiv, C, lists,
                           L, (int)n, d, out);
    }
}

// Mx[i][j] = sum over rows k < ns, in order, of rec_k[i] * X[k][j] in float32
// (compute_optimal_rotation's outer-product sum, opq.rs:255-270), where rec_k
// is the reconstruction of codes[k] (pq.rs:284-290): component i is entry
// i % ds of codeword codes[k][i / ds] of codebook i / ds.  One thread per
// element; j is the fastest index, so the reads of X are coalesced.
__global__ __launch_bounds__(256) void procrustes_kernel(const uint8_t* __restrict__ codes,
                                                         const float* __restrict__ cb, int M, int K,
                                                         int ds, const float* __restrict__ X, int ns,
                                                         int d, float* __restrict__ Mx) {
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= (size_t)d * d) return;
    const int i = (int)(t / d), j = (int)(t - (size_t)i * d);
    const int m = i / ds;
    const float* cbm = cb + (size_t)m * K * ds + (i - m * ds);
    float acc = 0.0f;
    for (int k = 0; k < ns; k++) {
        const float rec = cbm[(size_t)codes[(size_t)k * M + m] * ds];
        acc += rec * X[(size_t)k * d + j];
    }
    Mx[t] = acc;
}

void launch_procrustes(const uint8_t* codes, const float* cb, int M, int K, int ds, const float* X,
                       int ns, int d, float* Mx, hipStream_t s) {
    const size_t n = (size_t)d * d;
    hipLaunchKernelGGL(procrustes_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, codes, cb,
                       M, K, ds, X, ns, d, Mx);
}

}  // namespace vgpu
